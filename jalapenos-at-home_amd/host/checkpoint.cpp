// checkpoint.cpp -- see checkpoint.hpp.
#include "checkpoint.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <filesystem>
#include <fstream>
#include <stdexcept>
#include <unordered_map>

#include "json.hpp"

namespace fs = std::filesystem;

namespace jalapenos {

namespace {

[[noreturn]] void fail(const std::string& msg) { throw std::runtime_error(msg); }

uint64_t read_u64_le(const uint8_t* p) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];
    return v;
}

struct Entry {
    std::string name;
    std::string dtype;
    std::vector<size_t> shape;
    uint64_t start = 0, end = 0;
};

Entry parse_entry(const std::string& name, const json::Value& v) {
    // engine/src/lib.rs:78-83 (HeaderEntry): dtype, shape, data_offsets
    Entry e;
    e.name = name;
    const json::Value* dtype = v.find("dtype");
    const json::Value* shape = v.find("shape");
    const json::Value* offs = v.find("data_offsets");
    if (v.kind != json::Value::Kind::Object || !dtype || dtype->kind != json::Value::Kind::String || !shape ||
        shape->kind != json::Value::Kind::Array || !offs || offs->kind != json::Value::Kind::Array ||
        offs->arr.size() != 2)
        fail("invalid safetensors header entry: " + name);
    e.dtype = dtype->str;
    for (const json::Value& d : shape->arr) e.shape.push_back((size_t)d.as_u64());
    e.start = offs->arr[0].as_u64();
    e.end = offs->arr[1].as_u64();
    return e;
}

bool checked_elements(const std::vector<size_t>& shape, size_t& out) {
    size_t n = 1;
    for (size_t d : shape) {
        if (d != 0 && n > SIZE_MAX / d) return false;
        n *= d;
    }
    out = n;
    return true;
}

bool ends_with(const std::string& s, const std::string& suffix, std::string& stem) {
    if (s.size() < suffix.size() || s.compare(s.size() - suffix.size(), suffix.size(), suffix) != 0) return false;
    stem = s.substr(0, s.size() - suffix.size());
    return true;
}

std::vector<fs::path> shards_of(const fs::path& folder) {
    std::vector<fs::path> paths;
    for (const auto& item : fs::directory_iterator(folder))
        if (item.path().extension() == ".safetensors") paths.push_back(item.path());
    std::sort(paths.begin(), paths.end());
    return paths;
}

// All tensors of one safetensors file (header entries in offset order).
struct File {
    std::vector<uint8_t> bytes;
    uint64_t base = 0;
    json::Value metadata;
    bool has_metadata = false;
    std::vector<Entry> entries;
};

File read_file(const fs::path& path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) fail("could not open " + path.string());
    File f;
    f.bytes.assign(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>());
    if (f.bytes.size() < 8) fail("failed to fill whole buffer");
    const uint64_t header_len = read_u64_le(f.bytes.data());
    // engine/src/lib.rs:109-112
    if (header_len > 100000000ull || header_len + 8 > f.bytes.size()) fail("invalid safetensors header length");
    json::Value header = json::parse(std::string(f.bytes.begin() + 8, f.bytes.begin() + 8 + header_len));
    if (header.kind != json::Value::Kind::Object) fail("invalid safetensors header");
    if (const json::Value* m = header.find("__metadata__")) {
        f.metadata = *m;
        f.has_metadata = true;
        header.erase("__metadata__");
    }
    for (const auto& kv : header.obj) f.entries.push_back(parse_entry(kv.first, kv.second));
    std::stable_sort(f.entries.begin(), f.entries.end(), [](const Entry& a, const Entry& b) { return a.start < b.start; });
    f.base = 8 + header_len;
    return f;
}

}  // namespace

Weights load(const std::string& folder_str) {
    const fs::path folder(folder_str);
    std::error_code ec;
    if (!fs::is_directory(folder, ec)) fail("No such file or directory: " + folder_str);
    const std::vector<fs::path> paths = shards_of(folder);
    if (paths.empty()) fail("model directory has no safetensors files");
    Weights w;
    w.model_name = folder.filename().string();
    std::unordered_map<std::string, std::pair<std::vector<size_t>, std::vector<uint8_t>>> packed, scales;
    for (const fs::path& path : paths) {
        File f = read_file(path);
        const json::Value* format = f.has_metadata ? f.metadata.find("format") : nullptr;
        const bool quantized = format && format->kind == json::Value::Kind::String && format->str == kMxfp4Format;
        for (const Entry& e : f.entries) {
            // engine/src/lib.rs:133-137
            if (e.start > e.end || e.end > f.bytes.size() - f.base) fail("invalid tensor offsets: " + e.name);
            std::vector<uint8_t> bytes(f.bytes.begin() + (ptrdiff_t)(f.base + e.start),
                                       f.bytes.begin() + (ptrdiff_t)(f.base + e.end));
            size_t elements = 0;
            if (!checked_elements(e.shape, elements)) fail("tensor shape overflow");
            if (quantized && e.dtype == "U8") {
                // engine/src/lib.rs:146-171
                if (elements != bytes.size()) fail("invalid packed tensor size: " + e.name);
                std::string stem;
                if (ends_with(e.name, ".mxfp4_packed", stem)) {
                    if (!packed.emplace(stem, std::make_pair(e.shape, std::move(bytes))).second)
                        fail("duplicate packed tensor");
                } else if (ends_with(e.name, ".mxfp4_scales", stem)) {
                    if (!scales.emplace(stem, std::make_pair(e.shape, std::move(bytes))).second)
                        fail("duplicate scale tensor");
                } else {
                    fail("unexpected U8 tensor: " + e.name);
                }
            } else {
                // engine/src/lib.rs:172-189
                if (!(e.dtype == "BF16" || (quantized && e.dtype == "U16")) || elements > SIZE_MAX / 2 ||
                    elements * 2 != bytes.size())
                    fail("expected BF16 tensor: " + e.name);
                std::vector<uint16_t> data(elements);
                for (size_t i = 0; i < elements; ++i) data[i] = (uint16_t)(bytes[2 * i] | (bytes[2 * i + 1] << 8));
                if (!w.tensors.emplace(e.name, Tensor::bf16(e.shape, std::move(data))).second) fail("duplicate tensor");
            }
        }
    }
    // engine/src/lib.rs:192-207
    for (auto& kv : packed) {
        auto it = scales.find(kv.first);
        if (it == scales.end()) fail("missing MXFP4 scales");
        const std::vector<size_t>& shape = kv.second.first;
        const std::vector<size_t>& scale_shape = it->second.first;
        if (shape.size() != 2 || shape[1] % 16 != 0 || scale_shape != std::vector<size_t>{shape[0], shape[1] / 16})
            fail("invalid MXFP4 tensor shape: " + kv.first);
        if (shape[1] > SIZE_MAX / 2) fail("shape overflow");
        std::string error;
        auto t = Tensor::quantized({shape[0], shape[1] * 2}, std::move(kv.second.second), std::move(it->second.second),
                                   &error);
        scales.erase(it);
        if (!t) fail(error);
        if (!w.tensors.emplace(kv.first, std::move(*t)).second) fail("duplicate tensor");
    }
    if (!scales.empty()) fail("MXFP4 scales have no matching packed weights");
    return w;
}

void save_safetensors(const std::string& path, const std::vector<std::pair<std::string, RawTensor>>& tensors,
                      const std::map<std::string, std::string>& metadata) {
    json::Value header = json::Value::object();
    if (!metadata.empty()) {
        json::Value m = json::Value::object();
        for (const auto& kv : metadata) m.set(kv.first, json::Value::string(kv.second));
        header.set("__metadata__", std::move(m));
    }
    uint64_t offset = 0;
    for (const auto& [name, t] : tensors) {
        json::Value e = json::Value::object();
        e.set("dtype", json::Value::string(t.dtype));
        json::Value shape = json::Value::array();
        for (size_t d : t.shape) shape.arr.push_back(json::Value::integer(d));
        e.set("shape", std::move(shape));
        json::Value offs = json::Value::array();
        offs.arr.push_back(json::Value::integer(offset));
        offs.arr.push_back(json::Value::integer(offset + t.bytes.size()));
        e.set("data_offsets", std::move(offs));
        header.set(name, std::move(e));
        offset += t.bytes.size();
    }
    std::string text = json::dump(header);
    text.append((8 - text.size() % 8) % 8, ' ');
    std::ofstream out(path, std::ios::binary | std::ios::trunc);
    if (!out) fail("could not create " + path);
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)((uint64_t)text.size() >> (8 * i));
    out.write(reinterpret_cast<const char*>(len), 8);
    out.write(text.data(), (std::streamsize)text.size());
    for (const auto& kv : tensors)
        out.write(reinterpret_cast<const char*>(kv.second.bytes.data()), (std::streamsize)kv.second.bytes.size());
    if (!out) fail("could not write " + path);
}

std::string convert(const Hip& hip, const std::string& source_str) {
    // python/quantize_mxfp4.py:52-119
    const fs::path source = fs::absolute(fs::path(source_str)).lexically_normal();
    const fs::path destination = source.parent_path() / (source.filename().string() + "-MXFP4");
    if (fs::exists(destination)) fail("destination already exists: " + destination.string());
    const std::vector<fs::path> shards = shards_of(source);
    if (shards.empty()) fail("no safetensors weights in " + source.string());

    // publish the directory only after every shard and config was written
    std::string tmpl = (source.parent_path() / ("." + destination.filename().string() + "-XXXXXX")).string();
    std::vector<char> buf(tmpl.begin(), tmpl.end());
    buf.push_back('\0');
    if (!mkdtemp(buf.data())) fail("could not create a temporary directory next to " + source.string());
    const fs::path temporary(buf.data());
    try {
        for (const fs::path& shard : shards) {
            File f = read_file(shard);
            std::vector<std::pair<std::string, RawTensor>> output;
            for (const Entry& e : f.entries) {
                if (e.dtype != "BF16") fail("expected BF16 weights: " + e.name);
                if (e.start > e.end || e.end > f.bytes.size() - f.base) fail("invalid tensor offsets: " + e.name);
                const uint8_t* p = f.bytes.data() + f.base + e.start;
                const size_t n = (size_t)(e.end - e.start);
                if (e.shape.size() == 2) {
                    const size_t rows = e.shape[0], width = e.shape[1];
                    if (width % 32) fail("row width must be divisible by 32: " + e.name);
                    if (rows * width * 2 != n) fail("expected BF16 weights: " + e.name);
                    std::vector<uint16_t> bits(rows * width);
                    for (size_t i = 0; i < bits.size(); ++i) bits[i] = (uint16_t)(p[2 * i] | (p[2 * i + 1] << 8));
                    auto q = hip.quantize(bits, rows, width);
                    output.push_back({e.name + ".mxfp4_packed", RawTensor{"U8", {rows, width / 2}, std::move(q.first)}});
                    output.push_back({e.name + ".mxfp4_scales", RawTensor{"U8", {rows, width / 32}, std::move(q.second)}});
                } else if (e.shape.size() == 1) {
                    // the BF16 bit pattern of normalization weights, saved as U16
                    output.push_back({e.name, RawTensor{"U16", e.shape, std::vector<uint8_t>(p, p + n)}});
                } else {
                    fail("unsupported tensor shape: " + e.name);
                }
            }
            save_safetensors((temporary / shard.filename()).string(), output, {{"format", kMxfp4Format}});
        }
        for (const auto& item : fs::directory_iterator(source)) {
            const fs::path& path = item.path();
            if (item.is_regular_file() &&
                (path.extension() == ".json" || path.extension() == ".txt" || path.filename() == "LICENSE") &&
                path.filename() != "model.safetensors.index.json")
                fs::copy_file(path, temporary / path.filename());
        }
        const fs::path config_path = temporary / "config.json";
        std::ifstream cin(config_path);
        if (!cin) fail("No such file or directory: " + config_path.string());
        json::Value config = json::parse(std::string(std::istreambuf_iterator<char>(cin), std::istreambuf_iterator<char>()));
        cin.close();
        json::Value qc = json::Value::object();
        qc.set("quant_method", json::Value::string("mxfp4"));
        qc.set("format", json::Value::string(kMxfp4Format));
        qc.set("block_size", json::Value::integer(32));
        json::Value yes;
        yes.kind = json::Value::Kind::Bool;
        yes.b = true;
        qc.set("weights_only", yes);
        config.set("quantization_config", std::move(qc));
        std::ofstream cout(config_path, std::ios::trunc);
        cout << json::dump(config, 2) << "\n";
        if (!cout) fail("could not write " + config_path.string());
        cout.close();
        fs::rename(temporary, destination);
    } catch (...) {
        std::error_code ec;
        fs::remove_all(temporary, ec);
        throw;
    }
    return destination.string();
}

}  // namespace jalapenos
