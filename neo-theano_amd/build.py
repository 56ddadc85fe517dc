"""Builds libtq.so (HIP kernels + C ABI, gfx950 only) and the C++ host layer.

Run as ``python neo-theano_amd/build.py`` or through ``__graft_entry__.build()``.
Everything is compiled in-tree so that the shared objects travel with the
source tree; nothing is installed.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libtq.so")
HOSTLIB = os.path.join(PKG, "libtheano_quantize_rocm.so")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed f32 VALU forms are kept out of the generated code on this fleet
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(ROOT, 'include')}",
]

SOURCES = ["tq_api.hip", "tq_quant.hip", "tq_gemv.hip", "tq_decode_w4.hip", "tq_decode_tiled.hip", "tq_gemm.hip", "tq_mlp.hip", "tq_ffn.hip", "tq_generic.hip", "tq_convert.hip", "tq_attention.hip"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    return out


def scratch_kernels(remarks):
    """Kernels whose resource-usage remarks report per-lane scratch (register
    spills or stack): [(kernel, bytes)]."""
    bad, cur = [], None
    for line in remarks.splitlines():
        if "Function Name:" in line:
            cur = line.split("Function Name:")[1].split()[0]
        elif "ScratchSize [bytes/lane]:" in line and cur:
            nbytes = int(line.split("ScratchSize [bytes/lane]:")[1].split()[0])
            if nbytes:
                bad.append((cur, nbytes))
    return bad


def build_lib(verbose=False, jobs=8):
    os.makedirs(OBJ, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]

    def compile_one(src):
        obj = os.path.join(OBJ, src.replace(".hip", ".o"))
        out = _run([HIPCC, *HIP_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", os.path.join(CSRC, src),
                    "-o", obj])
        # every kernel keeps its working set in registers: a spill to scratch
        # memory fails the build
        bad = scratch_kernels(out)
        if bad:
            raise RuntimeError(f"{src}: kernels spill to scratch: " +
                               ", ".join(f"{k} ({b} B/lane)" for k, b in bad))
        out = "\n".join(l for l in out.splitlines() if "kernel-resource-usage" not in l)
        if verbose and out.strip():
            print(out)
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


def build_host(verbose=False):
    """C++ host layer (theano_quantize mirror) over libtq.so."""
    src = os.path.join(HOST, "theano_quantize.cpp")
    if not os.path.exists(src):
        return None
    tmp = HOSTLIB + ".tmp"
    out = _run([HIPCC, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
                f"-I{os.path.join(ROOT, 'include')}", f"-I{HOST}", src, os.path.join(HOST, "theano_serialize.cpp"),
                os.path.join(HOST, "theano_rocm.cpp"),
                "-o", tmp,
                f"-L{PKG}", "-ltq", "-Wl,-rpath,$ORIGIN"])
    if verbose and out.strip():
        print(out)
    os.replace(tmp, HOSTLIB)
    # measurement driver of the storage layer (run by bench.py)
    bsrc = os.path.join(HOST, "bench_storage.cpp")
    if os.path.exists(bsrc):
        bout = os.path.join(PKG, "bench_storage")
        _run([HIPCC, "-O2", "-std=c++17", "-Wall", f"-I{os.path.join(ROOT, 'include')}", f"-I{HOST}", bsrc,
              "-o", bout + ".tmp", f"-L{PKG}", "-ltheano_quantize_rocm", "-ltq", "-Wl,-rpath,$ORIGIN"])
        os.replace(bout + ".tmp", bout)
    return HOSTLIB


def build_cpp_tests(verbose=False):
    """C++ tests of the host layer (test infrastructure: links the C oracle)."""
    src = os.path.join(ROOT, "tests", "cpp", "test_theano_quantize.cpp")
    if not os.path.exists(src) or not os.path.exists(HOSTLIB):
        return None
    out = os.path.join(ROOT, "tests", "cpp", "test_theano_quantize")
    tmp = out + ".tmp"
    odir = os.path.join(ROOT, "oracle")
    log = _run([HIPCC, "-O2", "-std=c++17", "-Wall", f"-I{os.path.join(ROOT, 'include')}", f"-I{HOST}", src,
                "-o", tmp, f"-L{PKG}", "-ltheano_quantize_rocm", "-ltq", f"-L{odir}", "-ltq_oracle",
                "-Wl,-rpath,$ORIGIN/../../neo-theano_amd", "-Wl,-rpath,$ORIGIN/../../oracle"])
    if verbose and log.strip():
        print(log)
    os.replace(tmp, out)
    return out


def build_oracle():
    """The C oracle (test infrastructure) -- compiled, never linked into libtq."""
    odir = os.path.join(ROOT, "oracle")
    out = os.path.join(odir, "libtq_oracle.so")
    tmp = out + ".tmp"
    _run(["gcc", "-O3", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared", "-std=c11",
          "-Wall", "-Werror", os.path.join(odir, "tq_oracle.c"), "-o", tmp, "-lm"])
    os.replace(tmp, out)
    return out


def build_peaks():
    """Measurement kernels of bench.py (libtq_peaks.so): HBM stream and MFMA peak loops."""
    src = os.path.join(CSRC, "bench", "tq_peaks.hip")
    out = os.path.join(PKG, "libtq_peaks.so")
    _run([HIPCC, *HIP_FLAGS, "-shared", src, "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


SAN_DIR = os.path.join(OBJ, "sanitize")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-g", "-O1"]


def build_sanitized(verbose=False):
    """CPU-only sanitizer builds (test infrastructure, opt-in: `build.py --sanitize`):
    * _build/sanitize/libtq_oracle.so: the C oracle under gcc's ASan + UBSan, for
      the Python oracle tests (TQ_ORACLE_LIB, with gcc's libasan preloaded);
    * _build/sanitize/test_theano_quantize: the C++ host-layer tests, with the
      host layer (allocator, storage, serialization, Module API) and the C oracle
      compiled in under clang's ASan + UBSan and linked to the ordinary libtq.so.
      These sources hold no device code, so ROCm's plain clang++ compiles them
      against the HIP runtime headers (no GPU pass, nothing device-side
      instrumented)."""
    os.makedirs(SAN_DIR, exist_ok=True)
    odir = os.path.join(ROOT, "oracle")
    olib = os.path.join(SAN_DIR, "libtq_oracle.so")
    _run(["gcc", *SAN, "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared", "-std=c11", "-Wall", "-Werror",
          os.path.join(odir, "tq_oracle.c"), "-o", olib + ".tmp", "-lm"])
    os.replace(olib + ".tmp", olib)
    rocm = os.path.dirname(os.path.dirname(os.path.realpath(HIPCC)))
    llvm = os.path.join(rocm, "llvm", "bin")
    if not os.path.exists(os.path.join(llvm, "clang++")):
        llvm = "/opt/rocm/llvm/bin"
    objs = []
    oobj = os.path.join(SAN_DIR, "tq_oracle.o")
    _run([os.path.join(llvm, "clang"), "-x", "c", "-std=c11", *SAN, "-ffp-contract=off", "-c",
          os.path.join(odir, "tq_oracle.c"), "-o", oobj])
    objs.append(oobj)
    for src in (os.path.join(ROOT, "tests", "cpp", "test_theano_quantize.cpp"), os.path.join(HOST, "theano_quantize.cpp"),
                os.path.join(HOST, "theano_serialize.cpp"), os.path.join(HOST, "theano_rocm.cpp")):
        obj = os.path.join(SAN_DIR, os.path.basename(src).replace(".cpp", ".o"))
        log = _run([os.path.join(llvm, "clang++"), "-std=c++17", *SAN, "-Wall", "-D__HIP_PLATFORM_AMD__",
                    f"-I{os.path.join(rocm, 'include')}", f"-I{os.path.join(ROOT, 'include')}", f"-I{HOST}", "-c", src,
                    "-o", obj])
        if verbose and log.strip():
            print(log)
        objs.append(obj)
    exe = os.path.join(SAN_DIR, "test_theano_quantize")
    _run([os.path.join(llvm, "clang++"), *SAN, *objs, "-o", exe + ".tmp", f"-L{PKG}", "-ltq",
          f"-L{os.path.join(rocm, 'lib')}", "-lamdhip64", f"-Wl,-rpath,{PKG}", f"-Wl,-rpath,{os.path.join(rocm, 'lib')}"])
    os.replace(exe + ".tmp", exe)
    return [olib, exe]


def build_all(verbose=False):
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    libs = [build_oracle(), build_lib(verbose=verbose), build_peaks()]
    h = build_host(verbose=verbose)
    if h:
        libs.append(h)
        t = build_cpp_tests(verbose=verbose)
        if t:
            libs.append(t)
    return libs


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        for p in build_sanitized(verbose="-v" in sys.argv):
            print("built", p)
    else:
        for p in build_all(verbose="-v" in sys.argv):
            print("built", p)
