// Reader for the artifact manifest model_v{3,4}.meta, the JSON that the
// reference's compiler writes (wpc-compiler/src/main.rs:55-67, 650-683):
//   {"layers":[{"name":S,"shape":[N,...],"offset_bytes":N,"size_bytes":N},...],
//    "block_size":N}
// Unknown keys are skipped, as serde does for the reference's reader
// (wpc_weights_v4.rs:22-35).
#include <cstdlib>
#include <cstring>

#include "wpcg_internal.hpp"

namespace wpcg {
namespace {

struct Parser {
    const char* p;
    const char* end;
    std::string err;

    void ws() { while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p; }
    bool eat(char c) { ws(); if (p < end && *p == c) { ++p; return true; } return false; }
    bool expect(char c)
    {
        if (eat(c)) return true;
        err = std::string("expected '") + c + "'";
        return false;
    }

    bool str(std::string& out)
    {
        ws();
        if (p >= end || *p != '"') { err = "expected string"; return false; }
        ++p;
        out.clear();
        while (p < end && *p != '"') {
            char c = *p++;
            if (c == '\\') {
                if (p >= end) break;
                char e = *p++;
                switch (e) {
                case 'n': out += '\n'; break;
                case 't': out += '\t'; break;
                case 'r': out += '\r'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'u': {
                    if (end - p < 4) { err = "bad \\u escape"; return false; }
                    unsigned v = (unsigned)std::strtoul(std::string(p, 4).c_str(), nullptr, 16);
                    p += 4;
                    if (v < 0x80) out += (char)v;
                    else if (v < 0x800) { out += (char)(0xC0 | (v >> 6)); out += (char)(0x80 | (v & 63)); }
                    else { out += (char)(0xE0 | (v >> 12)); out += (char)(0x80 | ((v >> 6) & 63)); out += (char)(0x80 | (v & 63)); }
                    break;
                }
                default: out += e;
                }
            } else {
                out += c;
            }
        }
        if (p >= end) { err = "unterminated string"; return false; }
        ++p;
        return true;
    }

    bool uint(uint64_t& v)
    {
        ws();
        if (p >= end || *p < '0' || *p > '9') { err = "expected non-negative integer"; return false; }
        v = 0;
        while (p < end && *p >= '0' && *p <= '9') {
            uint64_t d = (uint64_t)(*p - '0');
            if (v > (UINT64_MAX - d) / 10) { err = "integer overflow"; return false; }
            v = v * 10 + d;
            ++p;
        }
        if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) { err = "expected integer"; return false; }
        return true;
    }

    // Skips any JSON value.
    bool skip(int depth = 0)
    {
        if (depth > 64) { err = "nesting too deep"; return false; }
        ws();
        if (p >= end) { err = "unexpected end"; return false; }
        char c = *p;
        if (c == '"') { std::string s; return str(s); }
        if (c == '{') {
            ++p;
            if (eat('}')) return true;
            do {
                std::string k;
                if (!str(k) || !expect(':') || !skip(depth + 1)) return false;
            } while (eat(','));
            return expect('}');
        }
        if (c == '[') {
            ++p;
            if (eat(']')) return true;
            do {
                if (!skip(depth + 1)) return false;
            } while (eat(','));
            return expect(']');
        }
        const char* s = p;
        while (p < end && std::strchr(",}] \n\r\t", *p) == nullptr) ++p;
        if (p == s) { err = "bad value"; return false; }
        return true;
    }

    bool layer(std::string& name, MetaEntry& e, bool& has_off, bool& has_size)
    {
        if (!expect('{')) return false;
        bool has_name = false, has_shape = false;
        has_off = has_size = false;
        if (eat('}')) { err = "empty layer entry"; return false; }
        do {
            std::string k;
            if (!str(k) || !expect(':')) return false;
            if (k == "name") {
                if (!str(name)) return false;
                has_name = true;
            } else if (k == "shape") {
                has_shape = true;
                if (!expect('[')) return false;
                e.shape.clear();
                if (!eat(']')) {
                    do {
                        uint64_t v;
                        if (!uint(v)) return false;
                        e.shape.push_back(v);
                    } while (eat(','));
                    if (!expect(']')) return false;
                }
            } else if (k == "offset_bytes") {
                if (!uint(e.offset)) return false;
                has_off = true;
            } else if (k == "size_bytes") {
                if (!uint(e.size)) return false;
                has_size = true;
            } else if (!skip()) {
                return false;
            }
        } while (eat(','));
        if (!expect('}')) return false;
        if (!has_name || !has_shape || !has_off || !has_size) {
            err = "layer entry lacks name/shape/offset_bytes/size_bytes";
            return false;
        }
        return true;
    }
};

}  // namespace

int parse_meta(const std::string& text, std::unordered_map<std::string, MetaEntry>& out,
               uint64_t& block_size)
{
    Parser ps{text.data(), text.data() + text.size(), {}};
    bool have_layers = false, have_bs = false;
    out.clear();
    auto bad = [&](const std::string& why) {
        return fail(WPCG_E_FORMAT, "model meta: " + why + " at byte " +
                                       std::to_string(ps.p - text.data()));
    };
    if (!ps.expect('{')) return bad(ps.err);
    if (!ps.eat('}')) {
        do {
            std::string k;
            if (!ps.str(k) || !ps.expect(':')) return bad(ps.err);
            if (k == "layers") {
                if (!ps.expect('[')) return bad(ps.err);
                have_layers = true;
                if (!ps.eat(']')) {
                    do {
                        std::string name;
                        MetaEntry e;
                        bool ho, hs;
                        if (!ps.layer(name, e, ho, hs)) return bad(ps.err);
                        out[name] = e;  // last entry wins, like HashMap::insert
                    } while (ps.eat(','));
                    if (!ps.expect(']')) return bad(ps.err);
                }
            } else if (k == "block_size") {
                if (!ps.uint(block_size)) return bad(ps.err);
                have_bs = true;
            } else if (!ps.skip()) {
                return bad(ps.err);
            }
        } while (ps.eat(','));
        if (!ps.expect('}')) return bad(ps.err);
    }
    ps.ws();
    if (ps.p != ps.end) return bad("trailing characters");
    if (!have_layers) return bad("missing field `layers`");
    if (!have_bs) return bad("missing field `block_size`");
    return WPCG_OK;
}

}  // namespace wpcg
