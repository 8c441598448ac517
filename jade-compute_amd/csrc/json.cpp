#include "json.hpp"

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>

namespace jade {
namespace json {
namespace {

struct Parser {
    const std::string &s;
    size_t pos = 0;
    int depth = 0;
    std::string error;

    explicit Parser(const std::string &src) : s(src) {}

    bool fail(const char *what) {
        if (error.empty()) error = std::string(what) + " at byte " + std::to_string(pos);
        return false;
    }
    void skip() {
        while (pos < s.size() && (s[pos] == ' ' || s[pos] == '\n' || s[pos] == '\r' || s[pos] == '\t')) ++pos;
    }
    bool literal(const char *word) {
        size_t n = 0;
        while (word[n]) ++n;
        if (s.compare(pos, n, word) != 0) return fail("invalid literal");
        pos += n;
        return true;
    }
    bool hex4(uint32_t &code) {
        if (pos + 4 > s.size()) return fail("truncated unicode escape");
        code = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = s[pos++];
            code <<= 4;
            if (c >= '0' && c <= '9') code |= uint32_t(c - '0');
            else if (c >= 'a' && c <= 'f') code |= uint32_t(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') code |= uint32_t(c - 'A' + 10);
            else return fail("invalid unicode escape");
        }
        return true;
    }
    static void utf8(std::string &out, uint32_t cp) {
        if (cp < 0x80) out += char(cp);
        else if (cp < 0x800) { out += char(0xC0 | (cp >> 6)); out += char(0x80 | (cp & 0x3F)); }
        else if (cp < 0x10000) { out += char(0xE0 | (cp >> 12)); out += char(0x80 | ((cp >> 6) & 0x3F)); out += char(0x80 | (cp & 0x3F)); }
        else { out += char(0xF0 | (cp >> 18)); out += char(0x80 | ((cp >> 12) & 0x3F)); out += char(0x80 | ((cp >> 6) & 0x3F)); out += char(0x80 | (cp & 0x3F)); }
    }
    bool string(std::string &out) {
        if (pos >= s.size() || s[pos] != '"') return fail("expected string");
        ++pos;
        while (pos < s.size()) {
            const char c = s[pos++];
            if (c == '"') return true;
            if (static_cast<unsigned char>(c) < 0x20) return fail("control character in string");
            if (c != '\\') { out += c; continue; }
            if (pos >= s.size()) break;
            const char e = s[pos++];
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
                    uint32_t cp = 0;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {
                        uint32_t low = 0;
                        if (pos + 2 > s.size() || s[pos] != '\\' || s[pos + 1] != 'u') return fail("unpaired surrogate");
                        pos += 2;
                        if (!hex4(low) || low < 0xDC00 || low > 0xDFFF) return fail("invalid surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (low - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return fail("unpaired surrogate");
                    }
                    utf8(out, cp);
                    break;
                }
                default: return fail("invalid escape");
            }
        }
        return fail("unterminated string");
    }
    bool number(Value &v) {
        const size_t start = pos;
        if (pos < s.size() && s[pos] == '-') ++pos;
        if (pos >= s.size()) return fail("truncated number");
        if (s[pos] == '0') ++pos;
        else if (s[pos] >= '1' && s[pos] <= '9') while (pos < s.size() && s[pos] >= '0' && s[pos] <= '9') ++pos;
        else return fail("invalid number");
        if (pos < s.size() && s[pos] == '.') {
            ++pos;
            if (pos >= s.size() || s[pos] < '0' || s[pos] > '9') return fail("invalid fraction");
            while (pos < s.size() && s[pos] >= '0' && s[pos] <= '9') ++pos;
        }
        if (pos < s.size() && (s[pos] == 'e' || s[pos] == 'E')) {
            ++pos;
            if (pos < s.size() && (s[pos] == '+' || s[pos] == '-')) ++pos;
            if (pos >= s.size() || s[pos] < '0' || s[pos] > '9') return fail("invalid exponent");
            while (pos < s.size() && s[pos] >= '0' && s[pos] <= '9') ++pos;
        }
        v.kind = Value::Kind::Number;
        v.text = s.substr(start, pos - start);
        return true;
    }
    bool value(Value &v) {
        if (++depth > 128) return fail("nesting too deep");
        skip();
        if (pos >= s.size()) return fail("unexpected end of input");
        const char c = s[pos];
        bool ok;
        if (c == '{') ok = object(v);
        else if (c == '[') ok = array(v);
        else if (c == '"') { v.kind = Value::Kind::String; ok = string(v.text); }
        else if (c == 't') { v.kind = Value::Kind::Bool; v.boolean = true; ok = literal("true"); }
        else if (c == 'f') { v.kind = Value::Kind::Bool; v.boolean = false; ok = literal("false"); }
        else if (c == 'n') { v.kind = Value::Kind::Null; ok = literal("null"); }
        else ok = number(v);
        --depth;
        return ok;
    }
    bool object(Value &v) {
        v.kind = Value::Kind::Object;
        ++pos;
        skip();
        if (pos < s.size() && s[pos] == '}') { ++pos; return true; }
        for (;;) {
            skip();
            std::string key;
            if (!string(key)) return false;
            for (const auto &m : v.members)
                if (m.first == key) return fail("duplicate field");
            skip();
            if (pos >= s.size() || s[pos] != ':') return fail("expected ':'");
            ++pos;
            Value child;
            if (!value(child)) return false;
            v.members.emplace_back(std::move(key), std::move(child));
            skip();
            if (pos < s.size() && s[pos] == ',') { ++pos; continue; }
            if (pos < s.size() && s[pos] == '}') { ++pos; return true; }
            return fail("expected ',' or '}'");
        }
    }
    bool array(Value &v) {
        v.kind = Value::Kind::Array;
        ++pos;
        skip();
        if (pos < s.size() && s[pos] == ']') { ++pos; return true; }
        for (;;) {
            Value child;
            if (!value(child)) return false;
            v.items.push_back(std::move(child));
            skip();
            if (pos < s.size() && s[pos] == ',') { ++pos; continue; }
            if (pos < s.size() && s[pos] == ']') { ++pos; return true; }
            return fail("expected ',' or ']'");
        }
    }
};

}  // namespace

bool parse(const std::string &source, Value &out, std::string &error) {
    Parser p(source);
    out = Value();
    if (!p.value(out)) {
        error = p.error.empty() ? "invalid JSON" : p.error;
        return false;
    }
    p.skip();
    if (p.pos != source.size()) {
        error = "trailing characters at byte " + std::to_string(p.pos);
        return false;
    }
    return true;
}

bool as_u32(const Value &v, uint32_t &out) {
    if (v.kind != Value::Kind::Number || v.text.empty()) return false;
    uint64_t acc = 0;
    for (const char c : v.text) {
        if (c < '0' || c > '9') return false;  // sign, fraction or exponent
        acc = acc * 10 + uint64_t(c - '0');
        if (acc > 0xFFFFFFFFull) return false;
    }
    out = static_cast<uint32_t>(acc);
    return true;
}

bool as_f32(const Value &v, float &out) {
    if (v.kind != Value::Kind::Number) return false;
    errno = 0;
    // Parsed to f64 first and narrowed, matching serde_json's f32 path.
    const double d = std::strtod(v.text.c_str(), nullptr);
    out = static_cast<float>(d);
    return true;
}

std::string format_f32(float value) {
    char buf[64];
    for (int precision = 1; precision <= 9; ++precision) {
        std::snprintf(buf, sizeof buf, "%.*g", precision, static_cast<double>(value));
        if (std::strtof(buf, nullptr) == value) break;
    }
    return buf;
}

std::string quote(const std::string &s) {
    std::string out = "\"";
    for (const char c : s) {
        switch (c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            default:
                if (static_cast<unsigned char>(c) < 0x20) {
                    char esc[8];
                    std::snprintf(esc, sizeof esc, "\\u%04x", c);
                    out += esc;
                } else {
                    out += c;
                }
        }
    }
    return out + "\"";
}

}  // namespace json
}  // namespace jade
