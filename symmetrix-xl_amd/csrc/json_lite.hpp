// Minimal strict JSON reader for Symmetrix model files.
//
// The model files hold ~10^7 numbers; arrays whose elements are all numbers are
// stored flat (Value::nums) so a medium model parses in about a second without
// one heap node per number.  Objects keep insertion order.  Errors throw
// std::invalid_argument with the byte offset.
#pragma once

#include <cerrno>
#include <charconv>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace json_lite {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object };
    Kind kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<double> nums;          // Array whose elements are all numbers
    std::vector<Value> items;          // Array of non-numbers (or mixed)
    std::vector<std::pair<std::string, Value>> members;
    bool numeric_array = false;

    bool is_object() const { return kind == Object; }
    bool is_array() const { return kind == Array; }
    bool is_number() const { return kind == Number; }
    bool is_string() const { return kind == String; }
    bool is_bool() const { return kind == Bool; }

    std::size_t size() const {
        if (kind == Array) return numeric_array ? nums.size() : items.size();
        if (kind == Object) return members.size();
        return 0;
    }
    const Value* find(const std::string& key) const {
        for (const auto& m : members)
            if (m.first == key) return &m.second;
        return nullptr;
    }
    bool contains(const std::string& key) const { return find(key) != nullptr; }
    const Value& at(const std::string& key) const {
        const Value* v = find(key);
        if (!v) throw std::invalid_argument("model JSON is missing key '" + key + "'");
        return *v;
    }
    const Value& at(std::size_t i) const {
        if (kind != Array || numeric_array || i >= items.size())
            throw std::invalid_argument("model JSON array index out of range");
        return items[i];
    }
    double as_number() const {
        if (kind != Number) throw std::invalid_argument("model JSON value is not a number");
        return num;
    }
    int as_int() const {
        const double v = as_number();
        if (v != static_cast<double>(static_cast<long long>(v)))
            throw std::invalid_argument("model JSON value is not an integer");
        return static_cast<int>(v);
    }
    bool as_bool() const {
        if (kind != Bool) throw std::invalid_argument("model JSON value is not a boolean");
        return b;
    }
    const std::string& as_string() const {
        if (kind != String) throw std::invalid_argument("model JSON value is not a string");
        return str;
    }
    // Flat numbers of an array (an empty array gives an empty vector).
    std::vector<double> as_doubles() const {
        if (kind != Array) throw std::invalid_argument("model JSON value is not an array");
        if (numeric_array || items.empty()) return nums;
        throw std::invalid_argument("model JSON array holds non-numbers");
    }
    std::vector<int> as_ints() const {
        std::vector<int> out;
        for (double v : as_doubles()) {
            if (v != static_cast<double>(static_cast<long long>(v)))
                throw std::invalid_argument("model JSON array holds a non-integer");
            out.push_back(static_cast<int>(v));
        }
        return out;
    }
    int get_int(const std::string& key, int fallback) const {
        const Value* v = find(key);
        return v ? v->as_int() : fallback;
    }
    bool get_bool(const std::string& key, bool fallback) const {
        const Value* v = find(key);
        return v ? v->as_bool() : fallback;
    }
    std::string get_string(const std::string& key, const std::string& fallback) const {
        const Value* v = find(key);
        return v ? v->as_string() : fallback;
    }
};

class Parser {
public:
    Parser(const char* begin, const char* end) : p_(begin), begin_(begin), end_(end) {}

    Value parse_document() {
        Value v = parse_value();
        skip_ws();
        if (p_ != end_) fail("trailing characters");
        return v;
    }

private:
    const char* p_;
    const char* begin_;
    const char* end_;

    [[noreturn]] void fail(const char* what) const {
        std::ostringstream s;
        s << "model JSON parse error at byte " << (p_ - begin_) << ": " << what;
        throw std::invalid_argument(s.str());
    }
    void skip_ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }
    bool consume(char c) {
        skip_ws();
        if (p_ < end_ && *p_ == c) { ++p_; return true; }
        return false;
    }
    void expect(char c) {
        if (!consume(c)) fail("unexpected character");
    }
    bool starts_number() const {
        return p_ < end_ && (*p_ == '-' || (*p_ >= '0' && *p_ <= '9'));
    }
    double parse_number() {
        // from_chars is correctly rounded (the same double as strtod) and
        // needs no terminated copy; a number must end in a digit or '.', so
        // "inf"/"nan" spellings are refused as JSON requires.
        double v = 0.0;
        const auto r = std::from_chars(p_, end_, v, std::chars_format::general);
        if (r.ec != std::errc() || r.ptr == p_) fail("invalid number");
        const char last = r.ptr[-1];
        if (!((last >= '0' && last <= '9') || last == '.')) fail("invalid number");
        p_ = r.ptr;
        return v;
    }
    std::string parse_string() {
        if (p_ >= end_ || *p_ != '"') fail("expected string");
        ++p_;
        std::string out;
        while (p_ < end_ && *p_ != '"') {
            if (*p_ == '\\') {
                ++p_;
                if (p_ >= end_) fail("bad escape");
                switch (*p_) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    if (end_ - p_ < 5) fail("bad unicode escape");
                    unsigned code = 0;
                    for (int i = 1; i <= 4; ++i) {
                        const char c = p_[i];
                        code <<= 4;
                        if (c >= '0' && c <= '9') code |= c - '0';
                        else if (c >= 'a' && c <= 'f') code |= c - 'a' + 10;
                        else if (c >= 'A' && c <= 'F') code |= c - 'A' + 10;
                        else fail("bad unicode escape");
                    }
                    p_ += 4;
                    if (code < 0x80) out += static_cast<char>(code);
                    else if (code < 0x800) {
                        out += static_cast<char>(0xC0 | (code >> 6));
                        out += static_cast<char>(0x80 | (code & 0x3F));
                    } else {
                        out += static_cast<char>(0xE0 | (code >> 12));
                        out += static_cast<char>(0x80 | ((code >> 6) & 0x3F));
                        out += static_cast<char>(0x80 | (code & 0x3F));
                    }
                    break;
                }
                default: fail("bad escape");
                }
                ++p_;
            } else {
                out += *p_++;
            }
        }
        if (p_ >= end_) fail("unterminated string");
        ++p_;
        return out;
    }
    Value parse_value() {
        skip_ws();
        if (p_ >= end_) fail("unexpected end");
        Value v;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = Value::Object;
            if (consume('}')) return v;
            do {
                skip_ws();
                std::string key = parse_string();
                expect(':');
                v.members.emplace_back(std::move(key), parse_value());
            } while (consume(','));
            expect('}');
        } else if (c == '[') {
            ++p_;
            v.kind = Value::Array;
            v.numeric_array = true;
            if (consume(']')) return v;
            do {
                skip_ws();
                if (v.numeric_array && starts_number()) {
                    v.nums.push_back(parse_number());
                } else {
                    if (v.numeric_array) {
                        // demote: previously read numbers become items
                        for (double x : v.nums) {
                            Value n;
                            n.kind = Value::Number;
                            n.num = x;
                            v.items.push_back(std::move(n));
                        }
                        v.nums.clear();
                        v.numeric_array = false;
                    }
                    v.items.push_back(parse_value());
                }
            } while (consume(','));
            expect(']');
            if (v.numeric_array && v.nums.empty()) v.numeric_array = false;
        } else if (c == '"') {
            v.kind = Value::String;
            v.str = parse_string();
        } else if (c == 't') {
            if (end_ - p_ < 4 || std::strncmp(p_, "true", 4) != 0) fail("bad literal");
            p_ += 4;
            v.kind = Value::Bool;
            v.b = true;
        } else if (c == 'f') {
            if (end_ - p_ < 5 || std::strncmp(p_, "false", 5) != 0) fail("bad literal");
            p_ += 5;
            v.kind = Value::Bool;
            v.b = false;
        } else if (c == 'n') {
            if (end_ - p_ < 4 || std::strncmp(p_, "null", 4) != 0) fail("bad literal");
            p_ += 4;
        } else if (starts_number()) {
            v.kind = Value::Number;
            v.num = parse_number();
        } else {
            fail("unexpected character");
        }
        return v;
    }
};

inline Value parse_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::invalid_argument("cannot open model file '" + path + "'");
    f.seekg(0, std::ios::end);
    const std::streamoff size = f.tellg();
    f.seekg(0, std::ios::beg);
    std::string text(static_cast<std::size_t>(size), '\0');
    f.read(text.data(), size);
    if (!f) throw std::invalid_argument("cannot read model file '" + path + "'");
    Parser parser(text.data(), text.data() + text.size());
    return parser.parse_document();
}

}  // namespace json_lite
