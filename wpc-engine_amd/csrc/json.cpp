// A small JSON reader (RFC 8259) for the host side: safetensors headers,
// model.safetensors.index.json and config.json. Values keep their kind;
// numbers keep the double value and, for integer literals, the exact
// unsigned value, so "size" fields can reject fractions the way serde's
// usize does.
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "wpcg_internal.hpp"

namespace wpcg {
namespace {

struct JParser {
    const char* p;
    const char* end;
    std::string err;

    void ws() { while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p; }
    bool fail_at(const char* why) { err = why; return false; }

    bool hex4(unsigned& v)
    {
        if (end - p < 4) return fail_at("bad \\u escape");
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = p[i];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
            else return fail_at("bad \\u escape");
        }
        p += 4;
        return true;
    }

    static void utf8(std::string& out, unsigned v)
    {
        if (v < 0x80) {
            out += (char)v;
        } else if (v < 0x800) {
            out += (char)(0xC0 | (v >> 6));
            out += (char)(0x80 | (v & 63));
        } else if (v < 0x10000) {
            out += (char)(0xE0 | (v >> 12));
            out += (char)(0x80 | ((v >> 6) & 63));
            out += (char)(0x80 | (v & 63));
        } else {
            out += (char)(0xF0 | (v >> 18));
            out += (char)(0x80 | ((v >> 12) & 63));
            out += (char)(0x80 | ((v >> 6) & 63));
            out += (char)(0x80 | (v & 63));
        }
    }

    bool str(std::string& out)
    {
        if (p >= end || *p != '"') return fail_at("expected string");
        ++p;
        out.clear();
        while (true) {
            if (p >= end) return fail_at("unterminated string");
            const char c = *p++;
            if (c == '"') return true;
            if ((unsigned char)c < 0x20) return fail_at("control character in string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p >= end) return fail_at("unterminated string");
            const char e = *p++;
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
                unsigned v;
                if (!hex4(v)) return false;
                if (v >= 0xD800 && v < 0xDC00) {  // a surrogate pair
                    unsigned lo;
                    if (end - p < 6 || p[0] != '\\' || p[1] != 'u') return fail_at("lone surrogate");
                    p += 2;
                    if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail_at("lone surrogate");
                    v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
                } else if (v >= 0xDC00 && v < 0xE000) {
                    return fail_at("lone surrogate");
                }
                utf8(out, v);
                break;
            }
            default: return fail_at("bad escape");
            }
        }
    }

    bool number(JsonValue& v)
    {
        const char* s = p;
        bool integral = true;
        if (p < end && *p == '-') ++p;
        if (p >= end || *p < '0' || *p > '9') return fail_at("bad number");
        if (*p == '0') ++p;
        else while (p < end && *p >= '0' && *p <= '9') ++p;
        if (p < end && *p == '.') {
            integral = false;
            ++p;
            if (p >= end || *p < '0' || *p > '9') return fail_at("bad number");
            while (p < end && *p >= '0' && *p <= '9') ++p;
        }
        if (p < end && (*p == 'e' || *p == 'E')) {
            integral = false;
            ++p;
            if (p < end && (*p == '+' || *p == '-')) ++p;
            if (p >= end || *p < '0' || *p > '9') return fail_at("bad number");
            while (p < end && *p >= '0' && *p <= '9') ++p;
        }
        const std::string lit(s, p);
        v.kind = JsonValue::NUM;
        v.num = std::strtod(lit.c_str(), nullptr);
        v.is_uint = false;
        if (integral && lit[0] != '-') {
            uint64_t u = 0;
            bool ok = true;
            for (char c : lit) {
                const uint64_t d = (uint64_t)(c - '0');
                if (u > (UINT64_MAX - d) / 10) { ok = false; break; }
                u = u * 10 + d;
            }
            v.is_uint = ok;
            v.u = u;
        }
        return true;
    }

    bool value(JsonValue& v, int depth)
    {
        if (depth > 128) return fail_at("nesting too deep");
        ws();
        if (p >= end) return fail_at("unexpected end");
        const char c = *p;
        if (c == '{') {
            ++p;
            v.kind = JsonValue::OBJ;
            ws();
            if (p < end && *p == '}') { ++p; return true; }
            while (true) {
                ws();
                std::string k;
                if (!str(k)) return false;
                ws();
                if (p >= end || *p != ':') return fail_at("expected ':'");
                ++p;
                JsonValue item;
                if (!value(item, depth + 1)) return false;
                v.obj.emplace_back(std::move(k), std::move(item));
                ws();
                if (p < end && *p == ',') { ++p; continue; }
                if (p < end && *p == '}') { ++p; return true; }
                return fail_at("expected ',' or '}'");
            }
        }
        if (c == '[') {
            ++p;
            v.kind = JsonValue::ARR;
            ws();
            if (p < end && *p == ']') { ++p; return true; }
            while (true) {
                JsonValue item;
                if (!value(item, depth + 1)) return false;
                v.arr.push_back(std::move(item));
                ws();
                if (p < end && *p == ',') { ++p; continue; }
                if (p < end && *p == ']') { ++p; return true; }
                return fail_at("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = JsonValue::STR;
            return str(v.str);
        }
        auto word = [&](const char* w) {
            const size_t n = std::strlen(w);
            if ((size_t)(end - p) >= n && std::memcmp(p, w, n) == 0) { p += n; return true; }
            return false;
        };
        if (word("true")) { v.kind = JsonValue::BOOL; v.b = true; return true; }
        if (word("false")) { v.kind = JsonValue::BOOL; v.b = false; return true; }
        if (word("null")) { v.kind = JsonValue::NUL; return true; }
        return number(v);
    }
};

}  // namespace

const JsonValue* JsonValue::get(const std::string& key) const
{
    if (kind != OBJ) return nullptr;
    const JsonValue* found = nullptr;
    for (const auto& kv : obj)
        if (kv.first == key) found = &kv.second;  // the last occurrence, as a map insert would keep
    return found;
}

bool json_parse(const char* text, size_t n, JsonValue& out, std::string& err)
{
    JParser ps{text, text + n, {}};
    out = JsonValue{};
    if (!ps.value(out, 0)) {
        err = ps.err + " at byte " + std::to_string(ps.p - text);
        return false;
    }
    ps.ws();
    if (ps.p != ps.end) {
        err = "trailing characters at byte " + std::to_string(ps.p - text);
        return false;
    }
    return true;
}

}  // namespace wpcg
