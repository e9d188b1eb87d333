// engine.cpp -- see engine.hpp. Host logic only: every product is computed on
// the GPU through the C ABI.
#include "engine.hpp"

#include <algorithm>
#include <utility>

namespace jalapenos {

std::optional<std::string> Mxfp4::validate(const std::vector<size_t>& shape) const {
    // engine/src/mxfp4.rs:12-24, same checks in the same order
    if (shape.size() != 2 || shape[0] == 0 || shape[1] == 0 || shape[1] % 32 != 0)
        return std::string("MXFP4 requires nonempty rows with a width divisible by 32");
    if (shape[0] > SIZE_MAX / shape[1]) return std::string("tensor is too large");
    const size_t elements = shape[0] * shape[1];
    if (packed.size() != elements / 2 || scales.size() != elements / 32)
        return std::string("MXFP4 data length does not match shape");
    if (std::find(scales.begin(), scales.end(), uint8_t{255}) != scales.end())
        return std::string("MXFP4 checkpoint contains a NaN scale");
    return std::nullopt;
}

Tensor Tensor::bf16(std::vector<size_t> shape, std::vector<uint16_t> data) {
    return Tensor{std::move(shape), std::move(data), std::nullopt};
}

std::optional<Tensor> Tensor::quantized(std::vector<size_t> shape, std::vector<uint8_t> packed,
                                        std::vector<uint8_t> scales, std::string* error) {
    Mxfp4 q{std::move(packed), std::move(scales)};
    if (auto e = q.validate(shape)) {
        if (error) *error = *e;
        return std::nullopt;
    }
    return Tensor{std::move(shape), {}, std::move(q)};
}

Hip::Hip(void* context, mx4_context* resident) : context_(context), resident_(resident) {}

std::optional<Hip> Hip::create() {
    void* c = qwen_hip_create();
    if (!c) return std::nullopt;
    mx4_context* r = nullptr;
    if (mx4_create(0, &r) != MX4_OK) {
        qwen_hip_destroy(c);
        return std::nullopt;
    }
    return Hip(c, r);
}

Hip::Hip(Hip&& o) noexcept : context_(std::exchange(o.context_, nullptr)), resident_(std::exchange(o.resident_, nullptr)) {}

Hip& Hip::operator=(Hip&& o) noexcept {
    if (this != &o) {
        this->~Hip();
        context_ = std::exchange(o.context_, nullptr);
        resident_ = std::exchange(o.resident_, nullptr);
    }
    return *this;
}

Hip::~Hip() {
    if (resident_) mx4_destroy(resident_);
    if (context_) qwen_hip_destroy(context_);
    resident_ = nullptr;
    context_ = nullptr;
}

namespace {

void require(bool ok, const char* what) {
    if (!ok) throw HipError(what);
}

// RAII device buffer of the resident context
struct DeviceBuffer {
    mx4_context* ctx;
    void* ptr = nullptr;
    DeviceBuffer(mx4_context* c, uint64_t bytes) : ctx(c) {
        if (mx4_malloc(ctx, bytes, &ptr) != MX4_OK) throw HipError(std::string("device allocation: ") + mx4_last_error());
    }
    ~DeviceBuffer() {
        if (ptr) mx4_free(ctx, ptr);
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
};

void check(mx4_status st, const char* what) {
    if (st != MX4_OK) throw HipError(std::string(what) + ": " + mx4_last_error());
}

}  // namespace

TensorF32 Hip::matmul(const TensorF32& input, const Tensor& weights) const {
    // engine/src/metal.rs:35-71
    require(input.shape.size() == 2 && weights.shape.size() == 2, "matmul takes 2-D tensors");
    const size_t rows = input.shape[0], cols = weights.shape[0], inner = input.shape[1];
    require(weights.shape[1] == inner, "assertion failed: weights.shape[1] == inner");
    require(input.data.size() == rows * inner, "assertion failed: input.data.len() == rows * inner");
    const void* weight_data;
    const uint8_t* scales;
    if (weights.mxfp4) {
        if (auto e = weights.mxfp4->validate(weights.shape)) throw HipError("invalid MXFP4 weight: " + *e);
        weight_data = weights.mxfp4->packed.data();
        scales = weights.mxfp4->scales.data();
    } else {
        require(weights.data.size() == cols * inner, "assertion failed: weights.data.len() == cols * inner");
        weight_data = weights.data.data();
        scales = nullptr;
    }
    require(rows <= UINT32_MAX && cols <= UINT32_MAX && inner <= UINT32_MAX, "tensor is too large");
    TensorF32 out{{rows, cols}, std::vector<float>(rows * cols, 0.0f)};
    const bool ok = qwen_hip_matmul(context_, input.data.data(), weight_data, scales, out.data.data(),
                                    (uint32_t)rows, (uint32_t)cols, (uint32_t)inner);
    if (!ok) throw HipError(std::string("HIP projection failed: ") + mx4_last_error());
    return out;
}

std::vector<float> Hip::values(const Tensor& weights) const {
    require(weights.mxfp4.has_value(), "values() decodes quantized tensors");
    const Mxfp4& q = *weights.mxfp4;
    if (auto e = q.validate(weights.shape)) throw HipError("invalid MXFP4 weight: " + *e);
    const uint32_t rows = (uint32_t)weights.shape[0], cols = (uint32_t)weights.shape[1];
    mx4_weight* w = nullptr;
    check(mx4_weight_upload(resident_, q.packed.data(), q.scales.data(), rows, cols, &w), "weight upload");
    std::unique_ptr<mx4_weight, void (*)(mx4_weight*)> hold(w, mx4_weight_release);
    const uint64_t n = (uint64_t)rows * cols;
    DeviceBuffer out(resident_, n * 4);
    check(mx4_dequantize(resident_, w, static_cast<float*>(out.ptr)), "dequantize");
    std::vector<float> v(n);
    check(mx4_download(resident_, v.data(), out.ptr, n * 4), "download");
    return v;
}

std::vector<uint32_t> Hip::argmax_rows(const TensorF32& logits) const {
    require(logits.shape.size() == 2 && logits.data.size() == logits.shape[0] * logits.shape[1],
            "argmax_rows takes a 2-D tensor");
    const uint32_t rows = (uint32_t)logits.shape[0], width = (uint32_t)logits.shape[1];
    DeviceBuffer x(resident_, (uint64_t)rows * width * 4), idx(resident_, (uint64_t)rows * 4);
    check(mx4_upload(resident_, x.ptr, logits.data.data(), (uint64_t)rows * width * 4), "upload");
    check(mx4_argmax_rows(resident_, static_cast<const float*>(x.ptr), rows, width, static_cast<uint32_t*>(idx.ptr)),
          "argmax_rows");
    std::vector<uint32_t> out(rows);
    check(mx4_download(resident_, out.data(), idx.ptr, (uint64_t)rows * 4), "download");
    return out;
}

std::pair<std::vector<uint8_t>, std::vector<uint8_t>> Hip::quantize(const std::vector<uint16_t>& bf16, size_t rows,
                                                                    size_t cols) const {
    if (cols % 32 != 0) throw HipError("row width must be divisible by 32");
    require(bf16.size() == rows * cols && rows <= UINT32_MAX && cols <= UINT32_MAX, "bad quantize shape");
    const uint64_t n = (uint64_t)rows * cols;
    std::pair<std::vector<uint8_t>, std::vector<uint8_t>> out{std::vector<uint8_t>(n / 2), std::vector<uint8_t>(n / 32)};
    if (n == 0) return out;
    DeviceBuffer in(resident_, n * 2), packed(resident_, n / 2), scales(resident_, n / 32);
    check(mx4_upload(resident_, in.ptr, bf16.data(), n * 2), "upload");
    check(mx4_quantize(resident_, in.ptr, MX4_BF16, rows, (uint32_t)cols, static_cast<uint8_t*>(packed.ptr),
                       static_cast<uint8_t*>(scales.ptr)),
          "quantize");
    check(mx4_download(resident_, out.first.data(), packed.ptr, n / 2), "download");
    check(mx4_download(resident_, out.second.data(), scales.ptr, n / 32), "download");
    return out;
}

}  // namespace jalapenos
