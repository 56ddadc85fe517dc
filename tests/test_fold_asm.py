"""The decode down kernel's inline-asm loads against the compiler's register use (CPU only).

`k_decode_fold32` (neo-theano_amd/csrc/tq_decode_tiled.hip) issues its weight and
scale loads as inline asm and waits for them with explicit `s_waitcnt vmcnt(N)`
counts, so the compiler believes each destination register is written when the
asm statement runs, while the data lands later.  The kernel is correct only if
no compiler-placed instruction reads or writes such a register between the load
and the wait that retires it.  These tests compile tq_decode_tiled.hip to gfx950
assembly with the library's flags and replay every instance's instruction stream
through a model of the in-order vmcnt queue over the control-flow graph (the
group loop is fully unrolled, so every path is forward), and fail on any access
to a register whose load may still be in flight.  A planted case checks that
the model catches the early-exit pattern it is there for: a wave that leaves
the loop with loads in flight whose registers the compiler then reuses."""
import os
import re
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "neo-theano_amd"))

VMEM = ("global_", "buffer_", "flat_", "scratch_")


def _vgprs(tok):
    m = re.fullmatch(r"v(\d+)", tok)
    if m:
        return {int(m.group(1))}
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    return set()


def _merge(a, b):
    """Queues from two predecessors, aligned at their newest entries."""
    if a is None:
        return b
    if b is None:
        return a
    n = max(len(a), len(b))
    pad_a = [frozenset()] * (n - len(a)) + list(a)
    pad_b = [frozenset()] * (n - len(b)) + list(b)
    return [x | y for x, y in zip(pad_a, pad_b)]


def inflight_hazards(body):
    """Instructions of one function body that touch a VGPR loaded by a vector
    memory instruction that an `s_waitcnt vmcnt` has not yet retired."""
    pending, state, dead, found = {}, [], False, []
    for raw in body.split("\n"):
        line = raw.split(";")[0].strip()
        if not line:
            continue
        label = re.fullmatch(r"(\.LBB\w+):", line)
        if label:
            state = _merge(None if dead else state, pending.get(label.group(1))) or []
            dead = False
            continue
        if line.startswith(".") or dead:
            continue
        op = line.split()[0]
        rest = line[len(op):]
        args = [a.strip() for a in rest.split(",")] if rest.strip() else []
        if op.startswith("s_waitcnt"):
            m = re.search(r"vmcnt\((\d+)\)", line)
            if m and int(m.group(1)) < len(state):
                n = int(m.group(1))
                state = state[len(state) - n:] if n else []
            continue
        if op.startswith("s_cbranch") or op == "s_branch":
            target = args[0]
            pending[target] = _merge(pending.get(target), list(state))
            dead = op == "s_branch"
            continue
        if op in ("s_endpgm", "s_setpc_b64"):
            dead = True
            continue
        inflight = set().union(*state) if state else set()
        touched = set()
        for tok in re.findall(r"v\[\d+:\d+\]|v\d+", rest):
            touched |= _vgprs(tok)
        if op.startswith(VMEM):
            dest = frozenset()
            if "load" in op and "lds" not in op and args:
                dest = frozenset(_vgprs(args[0]))
                touched -= dest
            if touched & inflight:
                found.append(line)
            state = state + [dest]
            continue
        if touched & inflight:
            found.append(line)
    return found


def _functions(asm, kernel):
    pat = r"^(_Z\w*" + kernel + r"(\w*)):.*?\n(.*?)\.Lfunc_end"
    return {m.group(2): m.group(3) for m in re.finditer(pat, asm, re.S | re.M)}


@pytest.fixture(scope="module")
def fold_asm(tmp_path_factory):
    import build
    if not os.path.exists(build.HIPCC) and not shutil.which("hipcc"):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "tq_decode_tiled.s"
    flags = [f for f in build.HIP_FLAGS if f not in ("-fPIC", "-Wall")]
    r = subprocess.run([build.HIPCC, *flags, "--cuda-device-only", "-S",
                        os.path.join(build.CSRC, "tq_decode_tiled.hip"), "-o", str(out)],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    return _functions(out.read_text(), "k_decode_fold32")


def test_every_fold32_instance_waits_before_touching_its_loads(fold_asm):
    # 1-8 groups per wave, one or two sets of 16 rows of h
    assert len(fold_asm) == 16, sorted(fold_asm)
    for name, body in sorted(fold_asm.items()):
        loads = len(re.findall(r"^\s*global_load_dwordx[24] ", body, re.M))
        assert loads > 0, name
        assert inflight_hazards(body) == [], name


PLANTED = """
\tglobal_load_dwordx4 v[2:5], v10, s[4:5] nt
\tglobal_load_dwordx2 v[6:7], v11, s[4:5]
\ts_cbranch_vccnz .LBB0_2
\ts_waitcnt vmcnt(1)
\tv_add_u32_e32 v8, v2, v3
\ts_waitcnt vmcnt(0)
\tv_add_u32_e32 v9, v6, v7
\ts_branch .LBB0_3
.LBB0_2:
\tv_lshl_add_u32 v4, v1, 6, v0
\ts_waitcnt vmcnt(0)
.LBB0_3:
\ts_endpgm
"""


def test_model_flags_register_reuse_on_an_early_exit():
    # the fall-through path waits before each use; the branch target reuses v4,
    # which the first load may still be writing
    assert inflight_hazards(PLANTED) == ["v_lshl_add_u32 v4, v1, 6, v0"]
    fixed = PLANTED.replace(".LBB0_2:\n\tv_lshl_add_u32 v4, v1, 6, v0\n\ts_waitcnt vmcnt(0)",
                            ".LBB0_2:\n\ts_waitcnt vmcnt(0)\n\tv_lshl_add_u32 v4, v1, 6, v0")
    assert inflight_hazards(fixed) == []
    # a use ahead of its wait is caught too
    early = fixed.replace("\ts_waitcnt vmcnt(1)\n", "")
    assert inflight_hazards(early) == ["v_add_u32_e32 v8, v2, v3"]
