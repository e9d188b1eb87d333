// engine.hpp -- C++ host side of the HIP backend, over the C ABI of mx4.h.
//
// The reference engine is Rust; its matmul interface for this path is the
// tensor types of engine/src/lib.rs:34-76 and engine/src/mxfp4.rs:5-49 and the
// Metal wrapper of engine/src/metal.rs:21-79. This header keeps those names,
// argument meanings and failure behaviour in C++:
//   * Mxfp4::validate returns the reference's error strings;
//   * Tensor::quantized fails (returns no tensor) where the Rust returns Err;
//   * Hip::create fails where Metal::new returns Err("could not initialize
//     Metal"), and Hip::matmul throws where Metal::matmul panics.
// Compute always runs on the GPU through libmx4hip.so: there is no CPU path.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "mx4.h"

namespace jalapenos {

// engine/src/mxfp4.rs:5-8
struct Mxfp4 {
    std::vector<uint8_t> packed;
    std::vector<uint8_t> scales;

    // engine/src/mxfp4.rs:11-25: empty on success, else the reference's message.
    std::optional<std::string> validate(const std::vector<size_t>& shape) const;
};

// engine/src/lib.rs:34-41 (Tensor) and :63-66 (TensorF32)
struct Tensor {
    std::vector<size_t> shape;
    std::vector<uint16_t> data;  // bf16 bits; empty for a quantized tensor
    std::optional<Mxfp4> mxfp4;

    // engine/src/lib.rs:43-49
    static Tensor bf16(std::vector<size_t> shape, std::vector<uint16_t> data);
    // engine/src/lib.rs:51-62: nullopt (with the message in *error) where the reference returns Err
    static std::optional<Tensor> quantized(std::vector<size_t> shape, std::vector<uint8_t> packed,
                                           std::vector<uint8_t> scales, std::string* error = nullptr);
};

struct TensorF32 {
    std::vector<size_t> shape;
    std::vector<float> data;
};

// The error Metal::matmul would panic with.
class HipError : public std::runtime_error {
   public:
    using std::runtime_error::runtime_error;
};

// engine/src/metal.rs:21-79 over qwen_hip_* (per-call, synchronous, device
// copies of weights cached by host address). Like the reference's wrapper it
// is neither copyable nor thread-safe.
class Hip {
   public:
    // Metal::new (engine/src/metal.rs:24-31): nullopt when no gfx950 device exists.
    static std::optional<Hip> create();
    Hip(Hip&& other) noexcept;
    Hip& operator=(Hip&& other) noexcept;
    Hip(const Hip&) = delete;
    Hip& operator=(const Hip&) = delete;
    ~Hip();

    // Metal::matmul (engine/src/metal.rs:34-72): y[rows][cols] = input . weights^T.
    // Weights must stay alive and unchanged while cached (engine/src/metal.rs:33).
    TensorF32 matmul(const TensorF32& input, const Tensor& weights) const;

    // Tensor::values (engine/src/lib.rs:56-61) of a whole quantized tensor,
    // decoded on the device, bit-exact.
    std::vector<float> values(const Tensor& weights) const;

    // argmax over each row of logits (engine/src/model.rs:288-296), on the device.
    std::vector<uint32_t> argmax_rows(const TensorF32& logits) const;

    // python/quantize_mxfp4.py:18-39 on the device, bit-exact: bf16 bits
    // [rows][cols] -> packed [rows][cols/2] and scales [rows][cols/32]. Throws
    // on a width not divisible by 32 or non-finite input (the reference raises).
    std::pair<std::vector<uint8_t>, std::vector<uint8_t>> quantize(const std::vector<uint16_t>& bf16, size_t rows,
                                                                   size_t cols) const;

   private:
    explicit Hip(void* context, mx4_context* resident);
    void* context_ = nullptr;             // qwen_hip_* context
    mx4_context* resident_ = nullptr;     // mx4_* context for the device-side helpers
};

}  // namespace jalapenos
