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
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <functional>
#include <string>
#include <vector>

#include "checkpoint.hpp"
#include "engine.hpp"
#include "json.hpp"

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

// ------------------------------------------------------------------ checkpoint format

namespace fs = std::filesystem;

std::vector<std::string>& temp_dirs() {
    static std::vector<std::string> dirs;
    return dirs;
}

std::string temp_dir() {
    char tmpl[] = "/tmp/mx4ckpt-XXXXXX";
    if (!mkdtemp(tmpl)) throw Failure{"mkdtemp failed"};
    temp_dirs().push_back(tmpl);
    return tmpl;
}

RawTensor u8(std::vector<size_t> shape, std::vector<uint8_t> bytes) { return RawTensor{"U8", std::move(shape), std::move(bytes)}; }

RawTensor u16(const char* dtype, std::vector<size_t> shape, const std::vector<uint16_t>& v) {
    RawTensor t{dtype, std::move(shape), {}};
    for (uint16_t x : v) {
        t.bytes.push_back((uint8_t)(x & 0xff));
        t.bytes.push_back((uint8_t)(x >> 8));
    }
    return t;
}

std::string load_error(const std::string& dir) {
    try {
        (void)load(dir);
    } catch (const std::runtime_error& e) {
        return e.what();
    }
    return "";
}

const std::map<std::string, std::string> kQuantized = {{"format", kMxfp4Format}};

// engine/src/lib.rs:89-202: every rejection, with the reference's message
Reg load_rejects_malformed_checkpoints("load_rejects_malformed_checkpoints", false, [] {
    const std::vector<uint8_t> p16(16 * 2, 0x21), s2{127, 127};
    {
        const std::string d = temp_dir();
        CHECK(load_error(d) == "model directory has no safetensors files");
    }
    {
        const std::string d = temp_dir();
        std::ofstream(d + "/a.safetensors", std::ios::binary) << std::string("\xff\xff\xff\xff\x00\x00\x00\x00{}", 10);
        CHECK(load_error(d) == "invalid safetensors header length");
    }
    auto one = [&](std::vector<std::pair<std::string, RawTensor>> ts, std::map<std::string, std::string> meta) {
        const std::string d = temp_dir();
        save_safetensors(d + "/model.safetensors", ts, meta);
        return d;
    };
    CHECK(load_error(one({{"w.mxfp4_packed", u8({2, 16}, p16)}, {"w.mxfp4_scales", u8({2, 1}, s2)}, {"x", u8({2}, {1, 2})}},
                         kQuantized)) == "unexpected U8 tensor: x");
    CHECK(load_error(one({{"w.mxfp4_packed", u8({2, 16}, p16)}}, kQuantized)) == "missing MXFP4 scales");
    CHECK(load_error(one({{"w.mxfp4_packed", u8({2, 16}, p16)}, {"w.mxfp4_scales", u8({1, 2}, s2)}}, kQuantized)) ==
          "invalid MXFP4 tensor shape: w");
    CHECK(load_error(one({{"w.mxfp4_packed", u8({2, 16}, p16)}, {"w.mxfp4_scales", u8({2, 1}, {127, 255})}}, kQuantized)) ==
          "MXFP4 checkpoint contains a NaN scale");
    CHECK(load_error(one({{"w.mxfp4_scales", u8({2, 1}, s2)}}, kQuantized)) == "MXFP4 scales have no matching packed weights");
    CHECK(load_error(one({{"w.mxfp4_packed", u8({2, 16}, std::vector<uint8_t>(31))}}, kQuantized)) ==
          "invalid packed tensor size: w.mxfp4_packed");
    CHECK(load_error(one({{"n", u16("U16", {4}, {1, 2, 3, 4})}}, {})) == "expected BF16 tensor: n");  // U16 only when quantized
    CHECK(load_error(one({{"n", u16("BF16", {4}, {1, 2, 3})}}, {})) == "expected BF16 tensor: n");
    {
        // offsets past the end of the file
        const std::string d = one({{"n", u16("BF16", {2}, {1, 2})}}, {});
        fs::resize_file(d + "/model.safetensors", fs::file_size(d + "/model.safetensors") - 2);
        CHECK(load_error(d) == "invalid tensor offsets: n");
    }
    {
        // the same name in two shards
        const std::string d = temp_dir();
        save_safetensors(d + "/a.safetensors", {{"n", u16("BF16", {2}, {1, 2})}}, {});
        save_safetensors(d + "/b.safetensors", {{"n", u16("BF16", {2}, {3, 4})}}, {});
        CHECK(load_error(d) == "duplicate tensor");
    }
});

Reg load_reads_quantized_and_bf16_shards("load_reads_quantized_and_bf16_shards", false, [] {
    const std::string d = temp_dir();
    std::vector<uint8_t> packed(3 * 32), scales(3 * 2);
    for (size_t i = 0; i < packed.size(); ++i) packed[i] = (uint8_t)(i * 37);
    for (size_t i = 0; i < scales.size(); ++i) scales[i] = (uint8_t)(120 + i);
    save_safetensors(d + "/model-00001.safetensors",
                     {{"layer.norm", u16("U16", {3}, {0x3f80, 0xbf80, 0x0001})},
                      {"layer.proj.mxfp4_packed", u8({3, 32}, packed)},
                      {"layer.proj.mxfp4_scales", u8({3, 2}, scales)}},
                     kQuantized);
    save_safetensors(d + "/model-00002.safetensors", {{"lm.bias", u16("BF16", {2}, {0x4000, 0xc000})}}, {});
    const Weights w = load(d);
    CHECK(w.tensors.size() == 3);
    const Tensor& proj = w.tensors.at("layer.proj");
    CHECK((proj.shape == std::vector<size_t>{3, 64}));
    CHECK(proj.data.empty() && proj.mxfp4 && proj.mxfp4->packed == packed && proj.mxfp4->scales == scales);
    const Tensor& norm = w.tensors.at("layer.norm");
    CHECK(!norm.mxfp4 && (norm.data == std::vector<uint16_t>{0x3f80, 0xbf80, 0x0001}));
    CHECK((w.tensors.at("lm.bias").data == std::vector<uint16_t>{0x4000, 0xc000}));
});

Reg json_round_trip("json_round_trip", false, [] {
    const std::string text =
        "{\"a\":[1,2.5,-3e2,true,false,null],\"b\":{\"s\":\"q\\\"\\\\\\n\\u00e9\\ud83d\\ude00\",\"n\":18446744073709551615}}";
    const json::Value v = json::parse(text);
    CHECK(v.find("b")->find("n")->as_u64() == 18446744073709551615ull);
    CHECK(v.find("b")->find("s")->str == "q\"\\\n\xc3\xa9\xf0\x9f\x98\x80");
    CHECK(json::parse(json::dump(v)).find("a")->arr.size() == 6);
    CHECK(json::dump(json::parse(json::dump(v, 2))) == json::dump(v));
    bool threw = false;
    try {
        (void)json::parse("{\"a\":1,}");
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK(threw);
});

// python/quantize_mxfp4.py:52-119 on the device, then engine/src/lib.rs:89-202
Reg convert_then_load_then_project("convert_then_load_then_project", true, [] {
    const std::string root = temp_dir();
    const std::string src = root + "/tiny-model";
    fs::create_directory(src);
    auto bf16_of = [](float f) { return (uint16_t)(bits(f) >> 16); };
    std::vector<uint16_t> w1(64 * 96), w2(33 * 64), norm(96);
    for (size_t i = 0; i < w1.size(); ++i) w1[i] = bf16_of(0.02f * std::sin(0.7f * (float)i) * (float)(1 + i % 5));
    for (size_t i = 0; i < w2.size(); ++i) w2[i] = bf16_of(std::cos(0.31f * (float)i) * (i % 97 == 0 ? 0.0f : 1.0f));
    for (size_t i = 0; i < norm.size(); ++i) norm[i] = bf16_of(1.0f + 0.01f * (float)i);
    save_safetensors(src + "/model-00001-of-00002.safetensors",
                     {{"model.layers.0.mlp.up_proj.weight", u16("BF16", {64, 96}, w1)},
                      {"model.norm.weight", u16("BF16", {96}, norm)}}, {});
    save_safetensors(src + "/model-00002-of-00002.safetensors", {{"lm_head.weight", u16("BF16", {33, 64}, w2)}}, {});
    std::ofstream(src + "/config.json") << "{\"hidden_size\": 96, \"torch_dtype\": \"bfloat16\"}";
    std::ofstream(src + "/tokenizer.json") << "{}";
    std::ofstream(src + "/model.safetensors.index.json") << "{}";

    const std::string dst = convert(device(), src);
    CHECK(dst == root + "/tiny-model-MXFP4");
    CHECK(fs::exists(dst + "/tokenizer.json") && !fs::exists(dst + "/model.safetensors.index.json"));
    std::ifstream cin(dst + "/config.json");
    const json::Value config = json::parse(std::string(std::istreambuf_iterator<char>(cin), {}));
    CHECK(config.find("hidden_size")->as_u64() == 96);
    const json::Value* qc = config.find("quantization_config");
    CHECK(qc && qc->find("format")->str == kMxfp4Format && qc->find("block_size")->as_u64() == 32);

    const Weights w = load(dst);
    CHECK(w.tensors.size() == 3);
    auto check_quantized = [&](const char* name, const std::vector<uint16_t>& src_bits, size_t rows, size_t cols) {
        const Tensor& t = w.tensors.at(name);
        CHECK((t.shape == std::vector<size_t>{rows, cols}) && t.mxfp4);
        std::vector<float> f(rows * cols);
        for (size_t i = 0; i < f.size(); ++i) f[i] = oracle_bf16_to_f32(src_bits[i]);
        std::vector<uint8_t> packed(rows * cols / 2), scales(rows * cols / 32);
        CHECK(oracle_quantize(f.data(), rows, cols, packed.data(), scales.data()) == 0);
        CHECK(t.mxfp4->packed == packed && t.mxfp4->scales == scales);  // the device quantizer is the rule, bit for bit
    };
    check_quantized("model.layers.0.mlp.up_proj.weight", w1, 64, 96);
    check_quantized("lm_head.weight", w2, 33, 64);
    CHECK(w.tensors.at("model.norm.weight").data == norm);

    // the loaded tensors feed the projection unchanged
    const Tensor& up = w.tensors.at("model.layers.0.mlp.up_proj.weight");
    TensorF32 x{{3, 96}, std::vector<float>(3 * 96)};
    for (size_t i = 0; i < x.data.size(); ++i) x.data[i] = std::sin(0.13f * (float)i);
    std::vector<float> expected(3 * 64);
    oracle_matmul(x.data.data(), 3, 96, up.mxfp4->packed.data(), up.mxfp4->scales.data(), 64, expected.data());
    const TensorF32 y = device().matmul(x, up);
    for (size_t i = 0; i < expected.size(); ++i) CHECK(std::fabs(y.data[i] - expected[i]) < 1e-3f + 1e-5f * std::fabs(expected[i]));

    bool threw = false;
    try {
        (void)convert(device(), src);
    } catch (const std::runtime_error& e) {
        threw = std::string(e.what()).find("destination already exists") == 0;
    }
    CHECK(threw);
    // a 2-D tensor whose width is not a multiple of 32 fails and leaves no partial output
    const std::string bad = root + "/bad";
    fs::create_directory(bad);
    save_safetensors(bad + "/m.safetensors", {{"w", u16("BF16", {2, 40}, std::vector<uint16_t>(80, 0x3f80))}}, {});
    std::ofstream(bad + "/config.json") << "{}";
    threw = false;
    try {
        (void)convert(device(), bad);
    } catch (const std::runtime_error& e) {
        threw = std::string(e.what()) == "row width must be divisible by 32: w";
    }
    CHECK(threw && !fs::exists(root + "/bad-MXFP4"));
    size_t leftovers = 0;
    for (const auto& item : fs::directory_iterator(root)) leftovers += item.path().filename().string().rfind(".bad", 0) == 0;
    CHECK(leftovers == 0);
    fs::remove_all(root);
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
    for (const std::string& d : temp_dirs()) {
        std::error_code ec;
        std::filesystem::remove_all(d, ec);
    }
    std::printf("%d tests, %d failed\n", ran, failed);
    return failed ? 1 : 0;
}
