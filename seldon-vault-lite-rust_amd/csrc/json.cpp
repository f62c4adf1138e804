// Strict JSON parser (the grammar and limits of src/json/mod.rs:192-557).
#include "json.hpp"

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string_view>
#include <unordered_set>

namespace svl::json {

namespace {

struct Parser {
    const unsigned char *in;
    size_t n, pos = 0, values = 0;
    const Limits &lim;
    Doc &doc;
    std::string &err;
    svl_status st = SVL_OK;

    bool corrupt(const char *msg) {
        char buf[160];
        snprintf(buf, sizeof buf, "JSON at byte %zu: %s", pos, msg);
        err = buf;
        st = SVL_CORRUPT;
        return false;
    }
    bool limit(const char *msg, size_t cap) {
        char buf[160];
        snprintf(buf, sizeof buf, msg, cap);
        err = buf;
        st = SVL_LIMIT;
        return false;
    }
    int peek() const { return pos < n ? in[pos] : -1; }
    void ws() {
        while (pos < n && (in[pos] == ' ' || in[pos] == '\t' || in[pos] == '\n' || in[pos] == '\r'))
            ++pos;
    }
    bool literal(const char *lit) {
        const size_t l = strlen(lit);
        if (n - pos < l || memcmp(in + pos, lit, l) != 0) return corrupt("invalid literal");
        pos += l;
        return true;
    }
    uint32_t push(Type t) {
        Node nd{};
        nd.type = t;
        doc.nodes.push_back(nd);
        return (uint32_t)(doc.nodes.size() - 1);
    }

    bool value(size_t depth) {
        if (depth > lim.max_depth) return limit("JSON nesting exceeds the depth cap of %zu", lim.max_depth);
        if (++values > lim.max_total_values)
            return limit("JSON document exceeds the %zu-value cap", lim.max_total_values);
        ws();
        const int c = peek();
        if (c < 0) return corrupt("unexpected end of input");
        uint32_t idx;
        switch (c) {
            case 'n':
                if (!literal("null")) return false;
                idx = push(Type::Null);
                break;
            case 't':
                if (!literal("true")) return false;
                idx = push(Type::Bool);
                doc.nodes[idx].b = true;
                break;
            case 'f':
                if (!literal("false")) return false;
                idx = push(Type::Bool);
                break;
            case '"':
                idx = push(Type::String);
                if (!string(idx)) return false;
                break;
            case '[':
                return array(depth);
            case '{':
                return object(depth);
            default:
                if (c == '-' || (c >= '0' && c <= '9')) return number();
                return corrupt("unexpected byte");
        }
        doc.nodes[idx].next = (uint32_t)doc.nodes.size();
        return true;
    }

    bool array(size_t depth) {
        const uint32_t idx = push(Type::Array);
        ++pos;
        ws();
        uint32_t count = 0;
        if (peek() == ']') {
            ++pos;
        } else {
            for (;;) {
                if (count >= lim.max_container_entries)
                    return limit("JSON array exceeds the %zu-entry cap", lim.max_container_entries);
                if (!value(depth + 1)) return false;
                ++count;
                ws();
                const int c = peek();
                if (c < 0) return corrupt("unexpected end of input");
                ++pos;
                if (c == ',') {
                    ws();
                    if (peek() == ']') return corrupt("trailing comma in array");
                } else if (c == ']') {
                    break;
                } else {
                    return corrupt("expected ',' or ']' after an array element");
                }
            }
        }
        doc.nodes[idx].count = count;
        doc.nodes[idx].next = (uint32_t)doc.nodes.size();
        return true;
    }

    bool object(size_t depth) {
        const uint32_t idx = push(Type::Object);
        ++pos;
        ws();
        uint32_t count = 0;
        std::vector<uint32_t> keys;
        if (peek() == '}') {
            ++pos;
        } else {
            for (;;) {
                if (count >= lim.max_container_entries)
                    return limit("JSON object exceeds the %zu-entry cap", lim.max_container_entries);
                ws();
                if (peek() != '"') return corrupt("object key must be a string");
                const uint32_t k = push(Type::String);
                if (!string(k)) return false;
                doc.nodes[k].next = (uint32_t)doc.nodes.size();
                keys.push_back(k);
                ws();
                if (peek() != ':') {
                    if (peek() < 0) return corrupt("unexpected end of input");
                    ++pos;
                    return corrupt("expected ':' after an object key");
                }
                ++pos;
                if (!value(depth + 1)) return false;
                ++count;
                ws();
                const int c = peek();
                if (c < 0) return corrupt("unexpected end of input");
                ++pos;
                if (c == ',') {
                    ws();
                    if (peek() == '}') return corrupt("trailing comma in object");
                } else if (c == '}') {
                    break;
                } else {
                    return corrupt("expected ',' or '}' after an object member");
                }
            }
        }
        if (keys.size() > 1) {
            std::unordered_set<std::string_view> seen;
            seen.reserve(keys.size() * 2);
            for (uint32_t k : keys)
                if (!seen.insert(doc.str(k)).second) return corrupt("duplicate object key");
        }
        doc.nodes[idx].count = count;
        doc.nodes[idx].next = (uint32_t)doc.nodes.size();
        return true;
    }

    bool hex4(uint32_t &v) {
        v = 0;
        for (int i = 0; i < 4; ++i) {
            if (pos >= n) return corrupt("unexpected end of input");
            const int c = in[pos++];
            int d;
            if (c >= '0' && c <= '9') d = c - '0';
            else if (c >= 'a' && c <= 'f') d = c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') d = c - 'A' + 10;
            else return corrupt("invalid hexadecimal digit in \\u escape");
            v = (v << 4) | (uint32_t)d;
        }
        return true;
    }

    void put_utf8(uint32_t cp) {
        std::string &a = doc.arena;
        if (cp < 0x80) {
            a.push_back((char)cp);
        } else if (cp < 0x800) {
            a.push_back((char)(0xC0 | (cp >> 6)));
            a.push_back((char)(0x80 | (cp & 0x3F)));
        } else if (cp < 0x10000) {
            a.push_back((char)(0xE0 | (cp >> 12)));
            a.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            a.push_back((char)(0x80 | (cp & 0x3F)));
        } else {
            a.push_back((char)(0xF0 | (cp >> 18)));
            a.push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
            a.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            a.push_back((char)(0x80 | (cp & 0x3F)));
        }
    }

    bool string(uint32_t idx) {
        ++pos;
        const size_t start = doc.arena.size();
        for (;;) {
            if (pos >= n) return corrupt("unexpected end of input");
            const unsigned char c = in[pos++];
            if (c == '"') break;
            if (c == '\\') {
                if (pos >= n) return corrupt("unexpected end of input");
                const unsigned char e = in[pos++];
                switch (e) {
                    case '"': doc.arena.push_back('"'); break;
                    case '\\': doc.arena.push_back('\\'); break;
                    case '/': doc.arena.push_back('/'); break;
                    case 'b': doc.arena.push_back('\b'); break;
                    case 'f': doc.arena.push_back('\f'); break;
                    case 'n': doc.arena.push_back('\n'); break;
                    case 'r': doc.arena.push_back('\r'); break;
                    case 't': doc.arena.push_back('\t'); break;
                    case 'u': {
                        uint32_t first;
                        if (!hex4(first)) return false;
                        uint32_t cp = first;
                        if (first >= 0xD800 && first <= 0xDBFF) {
                            if (pos >= n) return corrupt("unexpected end of input");
                            if (in[pos++] != '\\')
                                return corrupt("high surrogate is not followed by an escape");
                            if (pos >= n) return corrupt("unexpected end of input");
                            if (in[pos++] != 'u')
                                return corrupt("high surrogate is not followed by a \\u escape");
                            uint32_t second;
                            if (!hex4(second)) return false;
                            if (second < 0xDC00 || second > 0xDFFF)
                                return corrupt("high surrogate is not followed by a low surrogate");
                            cp = 0x10000 + ((first - 0xD800) << 10) + (second - 0xDC00);
                        } else if (first >= 0xDC00 && first <= 0xDFFF) {
                            return corrupt("lone low surrogate");
                        }
                        put_utf8(cp);
                        break;
                    }
                    default:
                        return corrupt("invalid escape sequence");
                }
            } else if (c < 0x20) {
                return corrupt("unescaped control character in string");
            } else {
                doc.arena.push_back((char)c);
            }
            if (doc.arena.size() - start > lim.max_string_bytes)
                return limit("JSON string exceeds the %zu-byte cap", lim.max_string_bytes);
        }
        doc.nodes[idx].off = (uint32_t)start;
        doc.nodes[idx].len = (uint32_t)(doc.arena.size() - start);
        return true;
    }

    static bool digit(int c) { return c >= '0' && c <= '9'; }

    bool number() {
        const size_t start = pos;
        const bool negative = peek() == '-';
        if (negative) ++pos;
        if (peek() == '0') {
            ++pos;
            if (digit(peek())) return corrupt("leading zero in number");
        } else if (peek() >= '1' && peek() <= '9') {
            while (digit(peek())) ++pos;
        } else {
            return corrupt("invalid number: expected a digit");
        }
        bool is_float = false;
        if (peek() == '.') {
            is_float = true;
            ++pos;
            if (!digit(peek())) return corrupt("invalid number: expected a digit after the decimal point");
            while (digit(peek())) ++pos;
        }
        if (peek() == 'e' || peek() == 'E') {
            is_float = true;
            ++pos;
            if (peek() == '+' || peek() == '-') ++pos;
            if (!digit(peek())) return corrupt("invalid number: expected a digit in the exponent");
            while (digit(peek())) ++pos;
        }
        const std::string tok((const char *)in + start, pos - start);
        const uint32_t idx = push(Type::Float);
        Node &nd = doc.nodes[idx];
        bool integral = false;
        if (!is_float) {
            errno = 0;
            char *end = nullptr;
            if (negative) {
                const long long v = strtoll(tok.c_str(), &end, 10);
                if (errno == 0 && *end == 0) {
                    nd.type = Type::Int;
                    nd.i = v;
                    integral = true;
                }
            } else {
                const unsigned long long v = strtoull(tok.c_str(), &end, 10);
                if (errno == 0 && *end == 0) {
                    nd.type = Type::UInt;
                    nd.u = v;
                    integral = true;
                }
            }
        }
        if (!integral) {
            const double v = strtod(tok.c_str(), nullptr);
            if (!std::isfinite(v)) return corrupt("number overflows to a non-finite value");
            nd.type = Type::Float;
            nd.f = v;
        }
        nd.next = (uint32_t)doc.nodes.size();
        return true;
    }
};

}  // namespace

uint32_t Doc::get(uint32_t i, std::string_view key) const {
    if (nodes[i].type != Type::Object) return UINT32_MAX;
    uint32_t k = i + 1;
    for (uint32_t m = 0; m < nodes[i].count; ++m) {
        if (str(k) == key) return k + 1;
        k = nodes[k + 1].next;
    }
    return UINT32_MAX;
}

bool Doc::as_u64(uint32_t i, uint64_t &out) const {
    if (nodes[i].type == Type::UInt) {
        out = nodes[i].u;
        return true;
    }
    if (nodes[i].type == Type::Int && nodes[i].i >= 0) {
        out = (uint64_t)nodes[i].i;
        return true;
    }
    return false;
}

bool valid_utf8(const char *text, size_t len) {
    const unsigned char *s = (const unsigned char *)text;
    size_t i = 0;
    while (i < len) {
        const unsigned char c = s[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        int extra;
        uint32_t cp;
        if ((c & 0xE0) == 0xC0) { extra = 1; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { extra = 2; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { extra = 3; cp = c & 0x07; }
        else return false;
        if (len - i <= (size_t)extra) return false;
        for (int k = 1; k <= extra; ++k) {
            if ((s[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        if ((extra == 1 && cp < 0x80) || (extra == 2 && cp < 0x800) || (extra == 3 && cp < 0x10000) ||
            cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF))
            return false;
        i += (size_t)extra + 1;
    }
    return true;
}

svl_status parse(const char *text, size_t len, const Limits &limits, Doc &doc, std::string &err) {
    doc.nodes.clear();
    doc.arena.clear();
    if (len > limits.max_input_bytes) {
        char buf[160];
        snprintf(buf, sizeof buf, "JSON input is %zu bytes, above the %zu-byte cap", len,
                 limits.max_input_bytes);
        err = buf;
        return SVL_LIMIT;
    }
    doc.arena.reserve(len);
    Parser p{(const unsigned char *)text, len, 0, 0, limits, doc, err};
    p.ws();
    if (!p.value(0)) return p.st;
    p.ws();
    if (p.pos != len) {
        p.corrupt("trailing content after the top-level value");
        return p.st;
    }
    return SVL_OK;
}

}  // namespace svl::json
