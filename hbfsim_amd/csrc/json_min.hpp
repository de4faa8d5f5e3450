// json_min.hpp -- a small JSON reader for device profiles.
//
// The reference parses profiles with nlohmann::json, which is not available
// here.  This reader covers what profiles use: objects, arrays, strings,
// numbers (integers kept exact as 64-bit), booleans and null.  Errors throw
// json_min::error with a position-bearing message.
#pragma once

#include <cerrno>
#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace json_min {

struct error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

struct value {
    enum kind_t { null_t, bool_t, int_t, uint_t, float_t, string_t, array_t, object_t };
    kind_t kind{null_t};
    bool b{false};
    std::int64_t i{0};
    std::uint64_t u{0};
    double d{0.0};
    std::string s;
    std::vector<value> a;
    std::vector<std::pair<std::string, value>> o;

    bool is_number() const { return kind == int_t || kind == uint_t || kind == float_t; }
    const value* find(const std::string& key) const
    {
        for (const auto& kv : o) {
            if (kv.first == key) {
                return &kv.second;
            }
        }
        return nullptr;
    }
    const value& at(const std::string& key) const
    {
        if (kind != object_t) {
            throw error("type_error: cannot use at() with non-object");
        }
        const value* v = find(key);
        if (v == nullptr) {
            throw error("out_of_range: key '" + key + "' not found");
        }
        return *v;
    }
    bool contains(const std::string& key) const
    {
        return kind == object_t && find(key) != nullptr;
    }
    std::uint64_t as_u64() const
    {
        if (kind == uint_t) return u;
        if (kind == int_t) return static_cast<std::uint64_t>(i);
        if (kind == float_t) return static_cast<std::uint64_t>(d);
        throw error("type_error: type must be number");
    }
    std::uint32_t as_u32() const { return static_cast<std::uint32_t>(as_u64()); }
    double as_double() const
    {
        if (kind == float_t) return d;
        if (kind == uint_t) return static_cast<double>(u);
        if (kind == int_t) return static_cast<double>(i);
        throw error("type_error: type must be number");
    }
    const std::string& as_string() const
    {
        if (kind != string_t) throw error("type_error: type must be string");
        return s;
    }
};

class parser {
  public:
    explicit parser(const std::string& text) : t_(text) {}
    value parse()
    {
        skip();
        value v = parse_value(0);
        skip();
        if (p_ != t_.size()) fail("unexpected trailing characters");
        return v;
    }

  private:
    const std::string& t_;
    std::size_t p_{0};

    [[noreturn]] void fail(const std::string& why) const
    {
        throw error("parse_error at byte " + std::to_string(p_) + ": " + why);
    }
    void skip()
    {
        while (p_ < t_.size() &&
               (t_[p_] == ' ' || t_[p_] == '\n' || t_[p_] == '\r' || t_[p_] == '\t')) {
            ++p_;
        }
    }
    bool eat(char c)
    {
        if (p_ < t_.size() && t_[p_] == c) {
            ++p_;
            return true;
        }
        return false;
    }
    void expect_word(const char* w)
    {
        for (const char* c = w; *c; ++c) {
            if (!eat(*c)) fail(std::string("invalid literal, expected ") + w);
        }
    }
    value parse_value(int depth)
    {
        if (depth > 64) fail("nesting too deep");
        if (p_ >= t_.size()) fail("unexpected end of input");
        value v;
        const char c = t_[p_];
        if (c == '{') {
            ++p_;
            v.kind = value::object_t;
            skip();
            if (eat('}')) return v;
            for (;;) {
                skip();
                if (p_ >= t_.size() || t_[p_] != '"') fail("expected object key");
                std::string key = parse_string();
                skip();
                if (!eat(':')) fail("expected ':'");
                skip();
                value item = parse_value(depth + 1);
                for (const auto& kv : v.o) {
                    if (kv.first == key) fail("duplicate key '" + key + "'");
                }
                v.o.emplace_back(std::move(key), std::move(item));
                skip();
                if (eat('}')) return v;
                if (!eat(',')) fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            ++p_;
            v.kind = value::array_t;
            skip();
            if (eat(']')) return v;
            for (;;) {
                skip();
                v.a.push_back(parse_value(depth + 1));
                skip();
                if (eat(']')) return v;
                if (!eat(',')) fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = value::string_t;
            v.s = parse_string();
            return v;
        }
        if (c == 't') { expect_word("true"); v.kind = value::bool_t; v.b = true; return v; }
        if (c == 'f') { expect_word("false"); v.kind = value::bool_t; v.b = false; return v; }
        if (c == 'n') { expect_word("null"); v.kind = value::null_t; return v; }
        return parse_number();
    }
    std::string parse_string()
    {
        ++p_;  // opening quote
        std::string out;
        while (p_ < t_.size()) {
            const char c = t_[p_++];
            if (c == '"') return out;
            if (static_cast<unsigned char>(c) < 0x20) fail("control character in string");
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (p_ >= t_.size()) break;
            const char e = t_[p_++];
            switch (e) {
            case '"': out.push_back('"'); break;
            case '\\': out.push_back('\\'); break;
            case '/': out.push_back('/'); break;
            case 'b': out.push_back('\b'); break;
            case 'f': out.push_back('\f'); break;
            case 'n': out.push_back('\n'); break;
            case 'r': out.push_back('\r'); break;
            case 't': out.push_back('\t'); break;
            case 'u': {
                if (p_ + 4 > t_.size()) fail("truncated \\u escape");
                unsigned cp = static_cast<unsigned>(std::strtoul(t_.substr(p_, 4).c_str(), nullptr, 16));
                p_ += 4;
                if (cp < 0x80) {
                    out.push_back(static_cast<char>(cp));
                } else if (cp < 0x800) {
                    out.push_back(static_cast<char>(0xc0 | (cp >> 6)));
                    out.push_back(static_cast<char>(0x80 | (cp & 0x3f)));
                } else {
                    out.push_back(static_cast<char>(0xe0 | (cp >> 12)));
                    out.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3f)));
                    out.push_back(static_cast<char>(0x80 | (cp & 0x3f)));
                }
                break;
            }
            default: fail("invalid escape");
            }
        }
        fail("unterminated string");
    }
    value parse_number()
    {
        const std::size_t start = p_;
        bool negative = eat('-');
        bool is_float = false;
        if (p_ >= t_.size() || t_[p_] < '0' || t_[p_] > '9') fail("invalid number");
        while (p_ < t_.size() && t_[p_] >= '0' && t_[p_] <= '9') ++p_;
        if (eat('.')) {
            is_float = true;
            if (p_ >= t_.size() || t_[p_] < '0' || t_[p_] > '9') fail("invalid fraction");
            while (p_ < t_.size() && t_[p_] >= '0' && t_[p_] <= '9') ++p_;
        }
        if (p_ < t_.size() && (t_[p_] == 'e' || t_[p_] == 'E')) {
            is_float = true;
            ++p_;
            if (p_ < t_.size() && (t_[p_] == '+' || t_[p_] == '-')) ++p_;
            if (p_ >= t_.size() || t_[p_] < '0' || t_[p_] > '9') fail("invalid exponent");
            while (p_ < t_.size() && t_[p_] >= '0' && t_[p_] <= '9') ++p_;
        }
        const std::string text = t_.substr(start, p_ - start);
        value v;
        if (is_float) {
            v.kind = value::float_t;
            v.d = std::strtod(text.c_str(), nullptr);
            return v;
        }
        errno = 0;
        if (negative) {
            v.kind = value::int_t;
            v.i = std::strtoll(text.c_str(), nullptr, 10);
        } else {
            v.kind = value::uint_t;
            v.u = std::strtoull(text.c_str(), nullptr, 10);
        }
        if (errno == ERANGE) {
            v.kind = value::float_t;
            v.d = std::strtod(text.c_str(), nullptr);
        }
        return v;
    }
};

inline value parse(const std::string& text) { return parser(text).parse(); }

}  // namespace json_min
