// C++ tests of the host layer (jalapenos-at-home_amd/host/engine.hpp) over the
// HIP library. Each test restates one of the reference's own tests for this
// path (the file:line is in its name's comment) against the C++ mirror of its
// types; expected values are the reference's literals, or the oracle (the C
// restatement of the reference's CPU matmul) where the reference compares with
// its CPU path.
//
// Usage: test_engine [--cpu-only]   (--cpu-only: the host-logic tests, no GPU)
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "engine.hpp"

extern "C" {
#include "mx4_oracle.h"
}

using namespace jalapenos;

namespace {

struct Failure {
    std::string msg;
};

#define CHECK(cond)                                                                                    \
    do {                                                                                               \
        if (!(cond)) throw Failure{std::string(__FILE__) + ":" + std::to_string(__LINE__) + ": " #cond}; \
    } while (0)

uint32_t bits(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return b;
}

struct Test {
    const char* name;
    bool gpu;
    std::function<void()> fn;
};

std::vector<Test>& registry() {
    static std::vector<Test> r;
    return r;
}

struct Reg {
    Reg(const char* n, bool gpu, std::function<void()> f) { registry().push_back({n, gpu, std::move(f)}); }
};

Hip& device() {
    static std::optional<Hip> hip = Hip::create();
    if (!hip) throw Failure{"no gfx950 device (Hip::create failed)"};
    return *hip;
}

// tests/mxfp4.rs:3-7
Tensor packed_weight() {
    const uint8_t row[8] = {0x10, 0x32, 0x54, 0x76, 0x98, 0xba, 0xdc, 0xfe};
    std::vector<uint8_t> packed(row, row + 8);
    packed.insert(packed.end(), row, row + 8);
    return *Tensor::quantized({1, 32}, packed, {126});
}

// tests/mxfp4.rs:35-40
Reg invalid_quantized_storage_is_rejected("invalid_quantized_storage_is_rejected", false, [] {
    std::string e;
    CHECK(!Tensor::quantized({1, 31}, std::vector<uint8_t>(16, 0), {127}, &e));
    CHECK(e == "MXFP4 requires nonempty rows with a width divisible by 32");
    CHECK(!Tensor::quantized({1, 32}, std::vector<uint8_t>(15, 0), {127}, &e));
    CHECK(e == "MXFP4 data length does not match shape");
    CHECK(!Tensor::quantized({1, 32}, std::vector<uint8_t>(16, 0), {255}, &e));
    CHECK(e == "MXFP4 checkpoint contains a NaN scale");
    // engine/src/mxfp4.rs:12-14: empty dimensions and non-2-D shapes
    CHECK(!Tensor::quantized({0, 32}, {}, {}, &e));
    CHECK(!Tensor::quantized({32}, std::vector<uint8_t>(16, 0), {127}, &e));
    CHECK(Tensor::quantized({1, 32}, std::vector<uint8_t>(16, 0), {127}, &e).has_value());
});

// the C ABI's host-only validate agrees with the C++ mirror
Reg abi_validate_matches_mirror("abi_validate_matches_mirror", false, [] {
    const uint8_t ok[2] = {127, 3}, nan[2] = {127, 255};
    CHECK(mx4_validate(1, 64, 32, ok, 2) == MX4_OK);
    CHECK(mx4_validate(1, 31, 16, ok, 1) == MX4_ERR_SHAPE);
    CHECK(mx4_validate(1, 64, 31, ok, 2) == MX4_ERR_LENGTH);
    CHECK(mx4_validate(1, 64, 32, nan, 2) == MX4_ERR_NAN_SCALE);
});

// tests/mxfp4.rs:9-33
Reg matrix_multiply_decodes_nibbles_and_scales("matrix_multiply_decodes_nibbles_and_scales", true, [] {
    const Tensor weights = packed_weight();
    std::vector<float> input(32 * 32, 0.0f);
    for (int i = 0; i < 32; ++i) input[i * 32 + i] = 1.0f;
    const TensorF32 output = device().matmul(TensorF32{{32, 32}, input}, weights);
    const float levels[8] = {0.0f, 0.25f, 0.5f, 0.75f, 1.0f, 1.5f, 2.0f, 3.0f};
    CHECK((output.shape == std::vector<size_t>{32, 1}));
    for (int i = 0; i < 32; ++i) {
        const float value = levels[i % 8];
        CHECK(output.data[i] == (i % 16 >= 8 ? -value : value));
    }
    CHECK(weights.data.empty());
});

// tests/mxfp4.rs:88-105
Reg matrix_rows_and_blocks_use_different_scales("matrix_rows_and_blocks_use_different_scales", true, [] {
    const Tensor weights = *Tensor::quantized({2, 64}, std::vector<uint8_t>(64, 0x77), {127, 126, 125, 124});
    std::vector<float> input(3 * 64, 0.0f);
    input[0] = 1.0f;
    input[64 + 32] = 1.0f;
    input[128] = 1.0f;
    input[128 + 32] = 1.0f;
    const TensorF32 result = device().matmul(TensorF32{{3, 64}, input}, weights);
    CHECK((result.shape == std::vector<size_t>{3, 2}));
    CHECK((result.data == std::vector<float>{6.0f, 1.5f, 3.0f, 0.75f, 9.0f, 2.25f}));
});

// engine/src/mxfp4.rs:56-65
Reg smallest_e8m0_scale_and_signed_zero_decode("smallest_e8m0_scale_and_signed_zero_decode", true, [] {
    const Tensor weights = *Tensor::quantized({1, 32}, std::vector<uint8_t>(16, 0x82), {0});
    const std::vector<float> decoded = device().values(weights);
    CHECK(bits(decoded[0]) == 0x00400000u);
    CHECK(bits(decoded[1]) == bits(-0.0f));
});

// engine/src/metal.rs:86-114 (the HIP backend in place of Metal), rows {1, 19}
// as in the reference plus the skinny and prefill-sized 2, 8, 33
Reg packed_and_bf16_kernels_match_cpu("packed_and_bf16_kernels_match_cpu_for_decode_and_prefill", true, [] {
    std::vector<uint8_t> packed(21 * 32), scales(21 * 2);
    for (size_t i = 0; i < packed.size(); ++i) packed[i] = (uint8_t)(i % 256);
    for (size_t i = 0; i < scales.size(); ++i) scales[i] = (uint8_t)(122 + i % 7);
    const Tensor quantized = *Tensor::quantized({21, 64}, packed, scales);
    std::vector<float> decoded(21 * 64);
    oracle_mx_values(packed.data(), scales.data(), 0, 21 * 64, decoded.data());
    std::vector<uint16_t> bf(21 * 64);
    for (size_t i = 0; i < bf.size(); ++i) bf[i] = (uint16_t)(bits(decoded[i]) >> 16);
    const Tensor bf16 = Tensor::bf16({21, 64}, bf);
    for (size_t rows : {1, 2, 8, 19, 33}) {
        TensorF32 input{{rows, 64}, std::vector<float>(rows * 64)};
        for (size_t i = 0; i < rows * 64; ++i) input.data[i] = ((float)(i % 37) - 18.0f) / 19.0f;
        for (const Tensor* weights : {&quantized, &bf16}) {
            std::vector<float> expected(rows * 21);
            if (weights->mxfp4)
                oracle_matmul(input.data.data(), rows, 64, packed.data(), scales.data(), 21, expected.data());
            else
                oracle_matmul_bf16(input.data.data(), rows, 64, bf.data(), 21, expected.data());
            const TensorF32 actual = device().matmul(input, *weights);
            CHECK((actual.shape == std::vector<size_t>{rows, 21}));
            for (size_t i = 0; i < expected.size(); ++i) {
                const float a = actual.data[i], b = expected[i];
                CHECK(std::fabs(a - b) < 1e-3f + std::fabs(b) * 1e-5f);
            }
        }
    }
});

// Metal::matmul asserts (engine/src/metal.rs:38-44, :66): the mirror throws
Reg shape_mismatch_and_nan_scale_throw("shape_mismatch_and_nan_scale_throw", true, [] {
    const Tensor weights = packed_weight();
    bool threw = false;
    try {
        (void)device().matmul(TensorF32{{1, 64}, std::vector<float>(64, 1.0f)}, weights);
    } catch (const HipError&) {
        threw = true;
    }
    CHECK(threw);
    Tensor bad = packed_weight();
    bad.mxfp4->scales[0] = 255;
    threw = false;
    try {
        (void)device().matmul(TensorF32{{1, 32}, std::vector<float>(32, 1.0f)}, bad);
    } catch (const HipError& e) {
        threw = std::string(e.what()).find("NaN scale") != std::string::npos;
    }
    CHECK(threw);
});

// engine/src/model.rs:288-296: first index of the maximum, on the device
Reg argmax_rows_first_maximum("argmax_rows_first_maximum", true, [] {
    TensorF32 logits{{3, 1000}, std::vector<float>(3000, 0.0f)};
    for (size_t i = 0; i < 3000; ++i) logits.data[i] = std::sin(0.37f * (float)i);
    logits.data[17] = logits.data[905] = 5.0f;           // tie in row 0: the first wins
    logits.data[1000 + 999] = 7.0f;                      // maximum at the last column
    logits.data[2000 + 0] = std::nanf("");               // NaN first: nothing is greater
    const std::vector<uint32_t> idx = device().argmax_rows(logits);
    for (int r = 0; r < 3; ++r) CHECK(idx[r] == (uint32_t)oracle_argmax(logits.data.data() + 1000 * r, 1000));
    CHECK(idx[0] == 17 && idx[1] == 999 && idx[2] == 0);
});

}  // namespace

int main(int argc, char** argv) {
    const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu-only") == 0;
    int failed = 0, ran = 0;
    for (const Test& t : registry()) {
        if (cpu_only && t.gpu) continue;
        ++ran;
        std::printf("%s ... ", t.name);
        std::fflush(stdout);
        try {
            t.fn();
            std::printf("ok\n");
        } catch (const Failure& f) {
            std::printf("FAILED %s\n", f.msg.c_str());
            ++failed;
        } catch (const std::exception& e) {
            std::printf("FAILED exception: %s\n", e.what());
            ++failed;
        }
        std::fflush(stdout);
    }
    std::printf("%d tests, %d failed\n", ran, failed);
    return failed ? 1 : 0;
}
