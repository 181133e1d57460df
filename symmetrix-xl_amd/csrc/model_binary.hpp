// Binary form of a Symmetrix model file ("SMXB"), beside the JSON v4 text.
//
// The binary file holds the same document tree as the JSON (objects in key
// order, arrays, strings, numbers, booleans, null) with every all-number
// array stored as raw little-endian IEEE doubles, so a medium model (about
// 12M numbers) loads with memcpy instead of number parsing.  Converting JSON
// -> binary -> JSON gives the same document: numbers are written back with
// the shortest decimal form that reads to the same double.
//
// Layout (little-endian):
//   bytes 0-7    "SMXB" magic, uint32 version (1)
//   bytes 8-15   uint64 payload size P
//   bytes 16-23  uint64 checksum of the payload (FNV-1a over 64-bit words,
//                the last partial word zero-padded)
//   bytes 24..   payload: one encoded value
// A value is a one-byte tag followed by its body:
//   0 null, 1 false, 2 true                      (no body)
//   3 number                                     double
//   4 string                                     uint64 length, bytes (UTF-8)
//   5 array of numbers                           uint64 count, count doubles
//   6 array of values                            uint64 count, count values
//   7 object                                     uint64 count, count x (string body, value)
// Empty arrays are written with tag 6.  Readers refuse a wrong magic or
// version, a size or checksum mismatch, unknown tags, counts that run past
// the payload and trailing bytes.
#pragma once

#include <charconv>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "json_lite.hpp"

namespace json_lite {

constexpr char kBinaryMagic[4] = {'S', 'M', 'X', 'B'};
constexpr std::uint32_t kBinaryVersion = 1;
constexpr std::size_t kBinaryHeader = 24;

enum BinaryTag : unsigned char { TagNull, TagFalse, TagTrue, TagNumber, TagString, TagNumbers, TagArray, TagObject };

inline std::uint64_t binary_checksum(const unsigned char* p, std::size_t n) {
    std::uint64_t h = 0xcbf29ce484222325ull;
    std::size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        std::uint64_t w;
        std::memcpy(&w, p + i, 8);
        h = (h ^ w) * 0x100000001b3ull;
    }
    if (i < n) {
        std::uint64_t w = 0;
        std::memcpy(&w, p + i, n - i);
        h = (h ^ w) * 0x100000001b3ull;
    }
    return h;
}

namespace detail {

class BinaryWriter {
public:
    std::string out;

    void value(const Value& v) {
        switch (v.kind) {
        case Value::Null: tag(TagNull); break;
        case Value::Bool: tag(v.b ? TagTrue : TagFalse); break;
        case Value::Number: tag(TagNumber); raw(&v.num, 8); break;
        case Value::String: tag(TagString); string(v.str); break;
        case Value::Array:
            if (v.numeric_array && !v.nums.empty()) {
                tag(TagNumbers);
                count(v.nums.size());
                raw(v.nums.data(), v.nums.size() * 8);
            } else {
                tag(TagArray);
                count(v.items.size());
                for (const Value& item : v.items) value(item);
            }
            break;
        case Value::Object:
            tag(TagObject);
            count(v.members.size());
            for (const auto& m : v.members) {
                string(m.first);
                value(m.second);
            }
            break;
        }
    }

private:
    void tag(BinaryTag t) { out.push_back(static_cast<char>(t)); }
    void raw(const void* p, std::size_t n) { out.append(static_cast<const char*>(p), n); }
    void count(std::uint64_t n) { raw(&n, 8); }
    void string(const std::string& s) {
        count(s.size());
        raw(s.data(), s.size());
    }
};

class BinaryReader {
public:
    BinaryReader(const unsigned char* p, std::size_t n) : p_(p), end_(p + n), begin_(p) {}

    Value document() {
        Value v = value(0);
        if (p_ != end_) fail("trailing bytes");
        return v;
    }

private:
    const unsigned char* p_;
    const unsigned char* end_;
    const unsigned char* begin_;

    [[noreturn]] void fail(const char* what) const {
        throw std::invalid_argument("binary model file is corrupt at payload byte " +
                                    std::to_string(p_ - begin_) + ": " + what);
    }
    void need(std::uint64_t n) {
        if (n > static_cast<std::uint64_t>(end_ - p_)) fail("a count runs past the end");
    }
    std::uint64_t count() {
        need(8);
        std::uint64_t n;
        std::memcpy(&n, p_, 8);
        p_ += 8;
        return n;
    }
    std::string string() {
        const std::uint64_t n = count();
        need(n);
        std::string s(reinterpret_cast<const char*>(p_), n);
        p_ += n;
        return s;
    }
    Value value(int depth) {
        if (depth > 256) fail("nesting too deep");
        need(1);
        const unsigned char t = *p_++;
        Value v;
        switch (t) {
        case TagNull: break;
        case TagFalse: v.kind = Value::Bool; v.b = false; break;
        case TagTrue: v.kind = Value::Bool; v.b = true; break;
        case TagNumber:
            need(8);
            v.kind = Value::Number;
            std::memcpy(&v.num, p_, 8);
            p_ += 8;
            break;
        case TagString: v.kind = Value::String; v.str = string(); break;
        case TagNumbers: {
            const std::uint64_t n = count();
            if (n == 0) fail("an empty number array must use the value-array tag");
            if (n > (std::uint64_t(1) << 60)) fail("count too large");
            need(n * 8);
            v.kind = Value::Array;
            v.numeric_array = true;
            v.nums.resize(n);
            std::memcpy(v.nums.data(), p_, n * 8);
            p_ += n * 8;
            break;
        }
        case TagArray: {
            const std::uint64_t n = count();
            need(n);  // every value is at least one byte
            v.kind = Value::Array;
            v.items.reserve(n);
            for (std::uint64_t i = 0; i < n; ++i) v.items.push_back(value(depth + 1));
            break;
        }
        case TagObject: {
            const std::uint64_t n = count();
            need(n);
            v.kind = Value::Object;
            v.members.reserve(n);
            for (std::uint64_t i = 0; i < n; ++i) {
                std::string key = string();
                v.members.emplace_back(std::move(key), value(depth + 1));
            }
            break;
        }
        default: --p_; fail("unknown tag");
        }
        return v;
    }
};

inline void json_string(std::string& out, const std::string& s) {
    out.push_back('"');
    for (const char c : s) {
        const unsigned char u = static_cast<unsigned char>(c);
        switch (c) {
        case '"': out += "\\\""; break;
        case '\\': out += "\\\\"; break;
        case '\n': out += "\\n"; break;
        case '\r': out += "\\r"; break;
        case '\t': out += "\\t"; break;
        case '\b': out += "\\b"; break;
        case '\f': out += "\\f"; break;
        default:
            if (u < 0x20) {
                char buf[8];
                std::snprintf(buf, sizeof(buf), "\\u%04x", u);
                out += buf;
            } else {
                out.push_back(c);
            }
        }
    }
    out.push_back('"');
}

inline void json_number(std::string& out, double v) {
    if (!std::isfinite(v)) throw std::invalid_argument("a model number is not finite and has no JSON form");
    char buf[32];
    // shortest form that reads back to the same double
    const auto r = std::to_chars(buf, buf + sizeof(buf), v);
    if (r.ec != std::errc()) throw std::runtime_error("number formatting failed");
    out.append(buf, r.ptr);
}

inline void json_value(std::string& out, const Value& v) {
    switch (v.kind) {
    case Value::Null: out += "null"; break;
    case Value::Bool: out += v.b ? "true" : "false"; break;
    case Value::Number: json_number(out, v.num); break;
    case Value::String: json_string(out, v.str); break;
    case Value::Array:
        out.push_back('[');
        if (v.numeric_array) {
            for (std::size_t i = 0; i < v.nums.size(); ++i) {
                if (i) out.push_back(',');
                json_number(out, v.nums[i]);
            }
        } else {
            for (std::size_t i = 0; i < v.items.size(); ++i) {
                if (i) out.push_back(',');
                json_value(out, v.items[i]);
            }
        }
        out.push_back(']');
        break;
    case Value::Object:
        out.push_back('{');
        for (std::size_t i = 0; i < v.members.size(); ++i) {
            if (i) out.push_back(',');
            json_string(out, v.members[i].first);
            out.push_back(':');
            json_value(out, v.members[i].second);
        }
        out.push_back('}');
        break;
    }
}

inline std::string read_all(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::invalid_argument("cannot open model file '" + path + "'");
    f.seekg(0, std::ios::end);
    const std::streamoff size = f.tellg();
    f.seekg(0, std::ios::beg);
    std::string bytes(static_cast<std::size_t>(size), '\0');
    f.read(bytes.data(), size);
    if (!f) throw std::invalid_argument("cannot read model file '" + path + "'");
    return bytes;
}

inline void write_all(const std::string& path, const std::string& a, const std::string& b = std::string()) {
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    if (!f) throw std::invalid_argument("cannot create '" + path + "'");
    f.write(a.data(), static_cast<std::streamsize>(a.size()));
    f.write(b.data(), static_cast<std::streamsize>(b.size()));
    f.close();
    if (!f) throw std::runtime_error("writing '" + path + "' failed");
}

}  // namespace detail

inline bool is_binary_document(const std::string& bytes) {
    return bytes.size() >= 4 && std::memcmp(bytes.data(), kBinaryMagic, 4) == 0;
}

inline Value parse_binary(const std::string& bytes) {
    if (bytes.size() < kBinaryHeader || !is_binary_document(bytes))
        throw std::invalid_argument("not a binary model file (no SMXB header)");
    std::uint32_t version;
    std::uint64_t size, sum;
    std::memcpy(&version, bytes.data() + 4, 4);
    std::memcpy(&size, bytes.data() + 8, 8);
    std::memcpy(&sum, bytes.data() + 16, 8);
    if (version != kBinaryVersion)
        throw std::invalid_argument("binary model file version " + std::to_string(version) + " is not supported");
    if (size != bytes.size() - kBinaryHeader)
        throw std::invalid_argument("binary model file is truncated or has trailing bytes");
    const auto* payload = reinterpret_cast<const unsigned char*>(bytes.data()) + kBinaryHeader;
    if (binary_checksum(payload, size) != sum) throw std::invalid_argument("binary model file checksum mismatch");
    detail::BinaryReader reader(payload, size);
    return reader.document();
}

// A model document from either form, told apart by the SMXB magic.
inline Value parse_model_file(const std::string& path) {
    const std::string bytes = detail::read_all(path);
    if (is_binary_document(bytes)) return parse_binary(bytes);
    Parser parser(bytes.data(), bytes.data() + bytes.size());
    return parser.parse_document();
}

inline void write_binary_file(const Value& v, const std::string& path) {
    detail::BinaryWriter w;
    w.value(v);
    std::string header(kBinaryHeader, '\0');
    const std::uint64_t size = w.out.size();
    const std::uint64_t sum = binary_checksum(reinterpret_cast<const unsigned char*>(w.out.data()), size);
    std::memcpy(header.data(), kBinaryMagic, 4);
    std::memcpy(header.data() + 4, &kBinaryVersion, 4);
    std::memcpy(header.data() + 8, &size, 8);
    std::memcpy(header.data() + 16, &sum, 8);
    detail::write_all(path, header, w.out);
}

inline void write_json_file(const Value& v, const std::string& path) {
    std::string out;
    detail::json_value(out, v);
    out.push_back('\n');
    detail::write_all(path, out);
}

}  // namespace json_lite
