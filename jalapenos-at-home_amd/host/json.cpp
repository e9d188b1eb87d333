// json.cpp -- see json.hpp.
#include "json.hpp"

#include <cctype>
#include <cerrno>
#include <cstdio>
#include <cstdlib>

namespace jalapenos::json {

const Value* Value::find(const std::string& key) const {
    for (const auto& kv : obj)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

Value& Value::set(const std::string& key, Value v) {
    for (auto& kv : obj)
        if (kv.first == key) return kv.second = std::move(v);
    obj.emplace_back(key, std::move(v));
    return obj.back().second;
}

bool Value::erase(const std::string& key) {
    for (auto it = obj.begin(); it != obj.end(); ++it)
        if (it->first == key) {
            obj.erase(it);
            return true;
        }
    return false;
}

uint64_t Value::as_u64() const {
    if (kind != Kind::Number || num_text.empty()) throw std::runtime_error("expected an integer");
    for (char c : num_text)
        if (!std::isdigit((unsigned char)c)) throw std::runtime_error("expected a non-negative integer");
    errno = 0;
    const unsigned long long v = std::strtoull(num_text.c_str(), nullptr, 10);
    if (errno) throw std::runtime_error("integer out of range");
    return v;
}

Value Value::string(std::string s) {
    Value v;
    v.kind = Kind::String;
    v.str = std::move(s);
    return v;
}

Value Value::integer(uint64_t x) {
    Value v;
    v.kind = Kind::Number;
    v.num = (double)x;
    v.num_text = std::to_string(x);
    return v;
}

Value Value::object() {
    Value v;
    v.kind = Kind::Object;
    return v;
}

Value Value::array() {
    Value v;
    v.kind = Kind::Array;
    return v;
}

namespace {

struct Parser {
    const std::string& s;
    size_t i = 0;

    [[noreturn]] void error(const char* what) const {
        throw std::runtime_error(std::string("JSON: ") + what + " at byte " + std::to_string(i));
    }
    void ws() {
        while (i < s.size() && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) ++i;
    }
    bool eat(char c) {
        ws();
        if (i < s.size() && s[i] == c) {
            ++i;
            return true;
        }
        return false;
    }
    void expect(char c) {
        if (!eat(c)) error("unexpected character");
    }
    static void put_utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xc0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            out += (char)(0xe0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3f));
            out += (char)(0x80 | (cp & 0x3f));
        } else {
            out += (char)(0xf0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3f));
            out += (char)(0x80 | ((cp >> 6) & 0x3f));
            out += (char)(0x80 | (cp & 0x3f));
        }
    }
    uint32_t hex4() {
        if (i + 4 > s.size()) error("short \\u escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = s[i++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else error("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        expect('"');
        std::string out;
        while (true) {
            if (i >= s.size()) error("unterminated string");
            const char c = s[i++];
            if (c == '"') return out;
            if ((unsigned char)c < 0x20) error("control character in string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (i >= s.size()) error("unterminated escape");
            const char e = s[i++];
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp = hex4();
                    if (cp >= 0xd800 && cp < 0xdc00 && i + 2 <= s.size() && s[i] == '\\' && s[i + 1] == 'u') {
                        i += 2;
                        const uint32_t lo = hex4();
                        if (lo < 0xdc00 || lo >= 0xe000) error("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: error("bad escape");
            }
        }
    }
    Value value(int depth) {
        if (depth > 64) error("nesting too deep");
        ws();
        if (i >= s.size()) error("unexpected end");
        const char c = s[i];
        Value v;
        if (c == '{') {
            ++i;
            v.kind = Value::Kind::Object;
            if (eat('}')) return v;
            do {
                ws();
                std::string key = string();
                expect(':');
                v.obj.emplace_back(std::move(key), value(depth + 1));
            } while (eat(','));
            expect('}');
        } else if (c == '[') {
            ++i;
            v.kind = Value::Kind::Array;
            if (eat(']')) return v;
            do v.arr.push_back(value(depth + 1));
            while (eat(','));
            expect(']');
        } else if (c == '"') {
            v.kind = Value::Kind::String;
            v.str = string();
        } else if (s.compare(i, 4, "true") == 0) {
            i += 4;
            v.kind = Value::Kind::Bool;
            v.b = true;
        } else if (s.compare(i, 5, "false") == 0) {
            i += 5;
            v.kind = Value::Kind::Bool;
        } else if (s.compare(i, 4, "null") == 0) {
            i += 4;
        } else if (c == '-' || std::isdigit((unsigned char)c)) {
            const size_t start = i;
            if (s[i] == '-') ++i;
            while (i < s.size() && (std::isdigit((unsigned char)s[i]) || s[i] == '.' || s[i] == 'e' || s[i] == 'E' ||
                                    s[i] == '+' || s[i] == '-'))
                ++i;
            v.kind = Value::Kind::Number;
            v.num_text = s.substr(start, i - start);
            char* end = nullptr;
            v.num = std::strtod(v.num_text.c_str(), &end);
            if (!end || *end) error("bad number");
        } else {
            error("unexpected character");
        }
        return v;
    }
};

void quote(std::string& out, const std::string& s) {
    out += '"';
    for (unsigned char c : s) {
        switch (c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            default:
                if (c < 0x20) {
                    char buf[8];
                    std::snprintf(buf, sizeof buf, "\\u%04x", c);
                    out += buf;
                } else {
                    out += (char)c;
                }
        }
    }
    out += '"';
}

void write(std::string& out, const Value& v, int indent, int level) {
    auto nl = [&](int lv) {
        if (indent < 0) return;
        out += '\n';
        out.append((size_t)(indent * lv), ' ');
    };
    switch (v.kind) {
        case Value::Kind::Null: out += "null"; break;
        case Value::Kind::Bool: out += v.b ? "true" : "false"; break;
        case Value::Kind::Number: {
            if (!v.num_text.empty()) {
                out += v.num_text;
            } else {
                char buf[40];
                std::snprintf(buf, sizeof buf, "%.17g", v.num);
                out += buf;
            }
            break;
        }
        case Value::Kind::String: quote(out, v.str); break;
        case Value::Kind::Array:
            out += '[';
            for (size_t k = 0; k < v.arr.size(); ++k) {
                if (k) out += indent < 0 ? "," : ",";
                nl(level + 1);
                write(out, v.arr[k], indent, level + 1);
            }
            if (!v.arr.empty()) nl(level);
            out += ']';
            break;
        case Value::Kind::Object:
            out += '{';
            for (size_t k = 0; k < v.obj.size(); ++k) {
                if (k) out += ',';
                nl(level + 1);
                quote(out, v.obj[k].first);
                out += indent < 0 ? ":" : ": ";
                write(out, v.obj[k].second, indent, level + 1);
            }
            if (!v.obj.empty()) nl(level);
            out += '}';
            break;
    }
}

}  // namespace

Value parse(const std::string& text) {
    Parser p{text};
    Value v = p.value(0);
    p.ws();
    if (p.i != text.size()) p.error("trailing characters");
    return v;
}

std::string dump(const Value& v, int indent) {
    std::string out;
    write(out, v, indent, 0);
    return out;
}

}  // namespace jalapenos::json
