// theano_serialize.hpp -- the safetensors container of
// crates/theano-serialize/src/safetensors.rs, extended for quantized weights.
//
// Container: 8-byte little-endian header length, a JSON header, the data
// section (safetensors.rs:3, to_bytes :83-95).  Two dialects are read:
//  * the reference's own: dtype names as DType prints them ("float32",
//    "float64", "int8", ...; crates/theano-types/src/dtype.rs:79-100), every
//    payload written as f64 little-endian whatever the name
//    (add_tensor :36-54).  A payload of 8 bytes per element is that f64
//    encoding; a payload of the named type's size is raw.
//  * standard safetensors: dtype codes F64 F32 F16 BF16 I64 I32 I16 I8 U8 BOOL
//    F8_E4M3
//    with payloads of that type and an optional "__metadata__" string map.
// Written: standard safetensors (tensors in name order, contiguous, header
// padded with spaces to a multiple of 8 bytes).  add_tensor writes F64, whose
// payload is also what the reference's own reader decodes.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <utility>
#include <vector>

#include "theano_quantize.hpp"

namespace theano {
namespace serialize {

// TensorInfo (safetensors.rs:9-16); dtype is the header's dtype string.
struct TensorInfo {
    std::string name;
    std::string dtype;
    std::vector<size_t> shape;
    std::pair<size_t, size_t> data_offsets;  // (start, end) in the data section
};

// Bytes per element of a dtype string (either dialect); 0 if unknown.
size_t element_size(const std::string& dtype);

// SafeTensorsFile (safetensors.rs:18-136).
class SafeTensorsFile {
   public:
    std::map<std::string, TensorInfo> tensors;
    std::vector<uint8_t> data;
    std::map<std::string, std::string> metadata;

    // f64 tensor as F64 (safetensors.rs:35-54)
    void add_tensor(const std::string& name, const Tensor& tensor);
    // raw payload of `dtype` (standard code), shape-checked
    Result<void> add_raw(const std::string& name, const std::string& dtype, std::vector<size_t> shape,
                         const void* bytes, size_t nbytes);
    // any numeric dtype decoded to f64 values (safetensors.rs:56-71)
    Result<Tensor> get_tensor(const std::string& name) const;
    // the payload of `name`, which must hold `dtype` (standard code or the
    // reference name of the same element type) with the given shape
    Result<std::vector<uint8_t>> get_raw(const std::string& name, const std::string& dtype,
                                         const std::vector<size_t>& shape) const;
    std::vector<std::string> tensor_names() const;
    // safetensors.rs:82-95 / 97-121
    std::vector<uint8_t> to_bytes() const;
    static Result<SafeTensorsFile> from_bytes(const std::vector<uint8_t>& bytes);
};

// save_safetensors / load_safetensors (safetensors.rs:143-160)
std::vector<uint8_t> save_safetensors(const std::map<std::string, Tensor>& tensors);
Result<std::map<std::string, Tensor>> load_safetensors(const std::vector<uint8_t>& bytes);

// Quantized checkpoints (build-defined layout, shared with the Python package):
//   <name>.weight        I8 [N, K] | U8 [N, K/2] (INT4 g128, low nibble = even k)
//                        | F8_E4M3 [N, K] (FP8 per channel)
//   <name>.weight_scale  F32 [N]   | F16 [N, K/128] (INT4)
//   <name>.bias          F32 [N]   (optional)
//   metadata <name>.quant = int8_per_channel | int8_per_channel_a8 | int4_g128
//   | fp8_e4m3_per_channel (FP8 weight-only) | fp8_e4m3_per_channel_a8 (FP8 W8A8),
//   <name>.group_size = 128 (INT4), <name>.in_features, <name>.out_features;
//   a QuantizedMLP <name>: <name>.{gate,up,down}.{weight,weight_scale},
//   <name>.quant = mlp_int4_g128, <name>.hidden, <name>.intermediate;
//   format = theano-quantize/1.
constexpr const char* kFormat = "theano-quantize/1";

}  // namespace serialize
}  // namespace theano
