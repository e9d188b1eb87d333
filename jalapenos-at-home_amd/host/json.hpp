// json.hpp -- the small JSON subset the checkpoint files use (safetensors
// headers and config.json): objects, arrays, strings, numbers, booleans and
// null. Object members keep their order, so a config read and written back is
// unchanged apart from the edited keys.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace jalapenos::json {

struct Value {
    enum class Kind { Null, Bool, Number, String, Array, Object } kind = Kind::Null;
    bool b = false;
    double num = 0.0;
    std::string num_text;  // the number as written, so integers round-trip exactly
    std::string str;
    std::vector<Value> arr;
    std::vector<std::pair<std::string, Value>> obj;

    const Value* find(const std::string& key) const;
    Value& set(const std::string& key, Value v);  // replaces or appends
    bool erase(const std::string& key);
    uint64_t as_u64() const;                      // throws unless a non-negative integer

    static Value string(std::string s);
    static Value integer(uint64_t v);
    static Value object();
    static Value array();
};

// Throws std::runtime_error with the byte offset on malformed input.
Value parse(const std::string& text);
// Compact when indent < 0, else pretty-printed with `indent` spaces.
std::string dump(const Value& v, int indent = -1);

}  // namespace jalapenos::json
