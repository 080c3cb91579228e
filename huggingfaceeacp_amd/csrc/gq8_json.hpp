// gq8_json.hpp -- a small JSON reader for the checkpoint's header, config.json
// and tokenizer.json: every value kind, depth-limited, nothing trusted.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

namespace gq8 {

// ---- a small JSON reader: every value kind, depth-limited, no trust --------
struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool boolean = false;
    double number = 0.0;
    bool integral = false; // the literal had no fraction or exponent
    int64_t integer = 0;   // its value when integral and in range
    std::string text;
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> members;

    const Json *find(const std::string &key) const
    {
        for (const auto &m : members)
            if (m.first == key)
                return &m.second;
        return nullptr;
    }
};

class JsonReader {
public:
    JsonReader(const char *p, size_t n) : p_(p), end_(p + n) {}
    bool read(Json &out)
    {
        if (!value(out, 0))
            return false;
        space();
        return p_ == end_;
    }

private:
    void space()
    {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r'))
            ++p_;
    }
    bool literal(const char *word)
    {
        const size_t n = std::strlen(word);
        if ((size_t) (end_ - p_) < n || std::memcmp(p_, word, n) != 0)
            return false;
        p_ += n;
        return true;
    }
    bool string(std::string &out)
    {
        if (p_ >= end_ || *p_ != '"')
            return false;
        ++p_;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if ((unsigned char) c < 0x20)
                return false;
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (p_ >= end_)
                return false;
            c = *p_++;
            switch (c) {
            case '"': case '\\': case '/': out.push_back(c); break;
            case 'b': out.push_back('\b'); break;
            case 'f': out.push_back('\f'); break;
            case 'n': out.push_back('\n'); break;
            case 'r': out.push_back('\r'); break;
            case 't': out.push_back('\t'); break;
            case 'u': {
                uint32_t cp = 0;
                if (!hex4(cp))
                    return false;
                if (cp >= 0xD800 && cp < 0xDC00) { // a surrogate pair
                    uint32_t lo = 0;
                    if (!literal("\\u") || !hex4(lo) || lo < 0xDC00 || lo >= 0xE000)
                        return false;
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(cp, out);
                break;
            }
            default: return false;
            }
        }
        if (p_ >= end_)
            return false;
        ++p_;
        return true;
    }
    bool hex4(uint32_t &v)
    {
        if (end_ - p_ < 4)
            return false;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t) (c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t) (c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t) (c - 'A' + 10);
            else return false;
        }
        return true;
    }
    static void utf8(uint32_t cp, std::string &out)
    {
        if (cp < 0x80) {
            out.push_back((char) cp);
        } else if (cp < 0x800) {
            out.push_back((char) (0xC0 | (cp >> 6)));
            out.push_back((char) (0x80 | (cp & 0x3F)));
        } else if (cp < 0x10000) {
            out.push_back((char) (0xE0 | (cp >> 12)));
            out.push_back((char) (0x80 | ((cp >> 6) & 0x3F)));
            out.push_back((char) (0x80 | (cp & 0x3F)));
        } else {
            out.push_back((char) (0xF0 | (cp >> 18)));
            out.push_back((char) (0x80 | ((cp >> 12) & 0x3F)));
            out.push_back((char) (0x80 | ((cp >> 6) & 0x3F)));
            out.push_back((char) (0x80 | (cp & 0x3F)));
        }
    }
    bool number(Json &out)
    {
        const char *start = p_;
        if (p_ < end_ && *p_ == '-')
            ++p_;
        if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9'))
            return false;
        if (*p_ == '0')
            ++p_;
        else
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9')
                ++p_;
        bool integral = true;
        if (p_ < end_ && *p_ == '.') {
            integral = false;
            ++p_;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9'))
                return false;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9')
                ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integral = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-'))
                ++p_;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9'))
                return false;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9')
                ++p_;
        }
        const std::string token(start, p_);
        out.kind = Json::Number;
        out.number = std::strtod(token.c_str(), nullptr);
        out.integral = false;
        if (integral) {
            errno = 0;
            char *stop = nullptr;
            const long long v = std::strtoll(token.c_str(), &stop, 10);
            if (errno == 0 && stop && *stop == '\0') {
                out.integral = true;
                out.integer = v;
            }
        }
        return true;
    }
    bool value(Json &out, int depth)
    {
        if (depth > 64)
            return false;
        space();
        if (p_ >= end_)
            return false;
        switch (*p_) {
        case '{': {
            ++p_;
            out.kind = Json::Object;
            space();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            for (;;) {
                space();
                std::string key;
                if (!string(key))
                    return false;
                space();
                if (p_ >= end_ || *p_ != ':')
                    return false;
                ++p_;
                Json v;
                if (!value(v, depth + 1))
                    return false;
                out.members.emplace_back(std::move(key), std::move(v));
                space();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        case '[': {
            ++p_;
            out.kind = Json::Array;
            space();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            for (;;) {
                Json v;
                if (!value(v, depth + 1))
                    return false;
                out.items.push_back(std::move(v));
                space();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        case '"': out.kind = Json::String; return string(out.text);
        case 't': out.kind = Json::Bool; out.boolean = true; return literal("true");
        case 'f': out.kind = Json::Bool; out.boolean = false; return literal("false");
        case 'n': out.kind = Json::Null; return literal("null");
        default: return number(out);
        }
    }

    const char *p_, *end_;
};

} // namespace gq8
