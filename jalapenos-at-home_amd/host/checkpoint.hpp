// checkpoint.hpp -- the on-disk weight format of the reference engine:
// safetensors files whose metadata `format` is "jalapenos-mxfp4-v1", with every
// 2-D weight stored as `<name>.mxfp4_packed` (U8 [N][K/2]) and
// `<name>.mxfp4_scales` (U8 [N][K/32]) and 1-D tensors kept as BF16/U16 bits.
//
//   load    -- engine/src/lib.rs:89-202 (try_load): same checks, same messages;
//              the tensors it returns feed Hip::matmul unchanged (the stored
//              layout is the kernels' layout).
//   convert -- python/quantize_mxfp4.py:52-119: a BF16 checkpoint directory to
//              "<dir>-MXFP4", with the quantization done on the GPU by the
//              library's quantizer (bit-exact to python/quantize_mxfp4.py:18-39).
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <utility>
#include <vector>

#include "engine.hpp"

namespace jalapenos {

inline constexpr const char* kMxfp4Format = "jalapenos-mxfp4-v1";  // python/quantize_mxfp4.py:10

// engine/src/lib.rs:68-71
struct Weights {
    std::string model_name;
    std::map<std::string, Tensor> tensors;
};

// engine/src/lib.rs:89-202 for the model directory `folder` (the reference
// resolves a name under weights/): every *.safetensors file, in path order.
// Throws std::runtime_error with the reference's message on any problem.
Weights load(const std::string& folder);

// One tensor of a safetensors file: dtype ("U8", "U16", "BF16"), shape and
// little-endian payload.
struct RawTensor {
    std::string dtype;
    std::vector<size_t> shape;
    std::vector<uint8_t> bytes;
};

// Writes a safetensors file: 8-byte little-endian header length, the JSON
// header (padded with spaces to a multiple of 8 bytes), then the payloads in
// the order given.
void save_safetensors(const std::string& path, const std::vector<std::pair<std::string, RawTensor>>& tensors,
                      const std::map<std::string, std::string>& metadata);

// python/quantize_mxfp4.py:52-119; returns the destination directory.
std::string convert(const Hip& hip, const std::string& source);

}  // namespace jalapenos
