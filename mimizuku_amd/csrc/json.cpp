// Strict JSON parser (src/json.rs:1-218 semantics), recursive descent over bytes.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "mz_json.h"

namespace {

constexpr int MAX_DEPTH = 64;

struct Parser {
    const unsigned char* s;
    size_t n, i = 0;
    std::string err;

    bool fail(const char* what, size_t at) {
        char b[160];
        snprintf(b, sizeof b, "json: %s at byte %zu", what, at);
        err = b;
        return false;
    }
    void ws() {
        while (i < n && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) i++;
    }
    bool expect(unsigned char c) {
        ws();
        if (i >= n) return fail("unexpected end", i);
        if (s[i] != c) {
            char w[32];
            snprintf(w, sizeof w, "expected '%c'", c);
            return fail(w, i);
        }
        i++;
        return true;
    }
    bool hex4(unsigned* out) {
        if (i + 4 > n) return fail("bad \\u escape", i);
        unsigned v = 0;
        for (int k = 0; k < 4; k++) {
            const unsigned char c = s[i + k];
            unsigned d;
            if (c >= '0' && c <= '9') d = c - '0';
            else if (c >= 'a' && c <= 'f') d = c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') d = c - 'A' + 10;
            else return fail("bad \\u escape", i);
            v = v * 16 + d;
        }
        i += 4;
        *out = v;
        return true;
    }
    static void put_utf8(std::string& o, unsigned cp) {
        if (cp < 0x80) {
            o += (char)cp;
        } else if (cp < 0x800) {
            o += (char)(0xc0 | (cp >> 6));
            o += (char)(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            o += (char)(0xe0 | (cp >> 12));
            o += (char)(0x80 | ((cp >> 6) & 0x3f));
            o += (char)(0x80 | (cp & 0x3f));
        } else {
            o += (char)(0xf0 | (cp >> 18));
            o += (char)(0x80 | ((cp >> 12) & 0x3f));
            o += (char)(0x80 | ((cp >> 6) & 0x3f));
            o += (char)(0x80 | (cp & 0x3f));
        }
    }
    // well-formed UTF-8 as Unicode defines it: no overlong forms, no encoded surrogates, nothing past U+10FFFF
    static bool utf8_ok(const std::string& t) {
        const unsigned char* p = (const unsigned char*)t.data();
        size_t k = 0, m = t.size();
        while (k < m) {
            const unsigned c = p[k];
            if (c < 0x80) {
                k++;
                continue;
            }
            int len;
            unsigned cp, min;
            if ((c & 0xe0) == 0xc0) len = 2, cp = c & 0x1f, min = 0x80;
            else if ((c & 0xf0) == 0xe0) len = 3, cp = c & 0x0f, min = 0x800;
            else if ((c & 0xf8) == 0xf0) len = 4, cp = c & 0x07, min = 0x10000;
            else return false;
            if (k + len > m) return false;
            for (int q = 1; q < len; q++) {
                if ((p[k + q] & 0xc0) != 0x80) return false;
                cp = (cp << 6) | (p[k + q] & 0x3f);
            }
            if (cp < min || cp > 0x10ffff || (cp >= 0xd800 && cp < 0xe000)) return false;
            k += len;
        }
        return true;
    }
    bool string(std::string* out) {
        if (!expect('"')) return false;
        std::string o;
        for (;;) {
            if (i >= n) return fail("unexpected end", i);
            const unsigned char c = s[i++];
            if (c == '"') break;
            if (c == '\\') {
                if (i >= n) return fail("unexpected end", i);
                const unsigned char e = s[i++];
                switch (e) {
                    case 'n': o += '\n'; break;
                    case 't': o += '\t'; break;
                    case 'r': o += '\r'; break;
                    case 'b': o += '\b'; break;
                    case 'f': o += '\f'; break;
                    case '"': case '\\': case '/': o += (char)e; break;
                    case 'u': {
                        unsigned cp;
                        if (!hex4(&cp)) return false;
                        // a high surrogate pairs with an immediately following low one; unpaired ones become U+FFFD
                        if (cp >= 0xd800 && cp < 0xdc00 && i + 2 <= n && s[i] == '\\' && s[i + 1] == 'u') {
                            const size_t save = i;
                            i += 2;
                            unsigned lo;
                            if (!hex4(&lo)) return false;
                            if (lo >= 0xdc00 && lo < 0xe000) cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                            else i = save;
                        }
                        if (cp >= 0xd800 && cp < 0xe000) cp = 0xfffd;
                        put_utf8(o, cp);
                        break;
                    }
                    default: return fail("bad escape", i - 1);
                }
                continue;
            }
            if (c < 0x20) return fail("control character in a string", i - 1);
            o += (char)c;
        }
        if (!utf8_ok(o)) return fail("invalid UTF-8 in a string", i - 1);
        *out = std::move(o);
        return true;
    }
    size_t digits() {
        const size_t d = i;
        while (i < n && s[i] >= '0' && s[i] <= '9') i++;
        return i - d;
    }
    // -?(0|[1-9][0-9]*)(.[0-9]+)?([eE][+-]?[0-9]+)?, finite
    bool number(MzJson* out) {
        const size_t st = i;
        if (i < n && s[i] == '-') i++;
        const int lead = i < n ? s[i] : -1;
        const size_t nd = digits();
        bool ok = nd == 1 || (nd > 1 && lead != '0');
        if (i < n && s[i] == '.') {
            i++;
            ok &= digits() > 0;
        }
        if (i < n && (s[i] == 'e' || s[i] == 'E')) {
            i++;
            if (i < n && (s[i] == '+' || s[i] == '-')) i++;
            ok &= digits() > 0;
        }
        if (!ok) return fail("bad number", st);
        const std::string tok((const char*)s + st, i - st);
        const double v = strtod(tok.c_str(), nullptr);
        if (!isfinite(v)) return fail("bad number", st);
        out->kind = MzJson::NUM;
        out->num = v;
        return true;
    }
    bool val(MzJson* out, int depth) {
        if (depth > MAX_DEPTH) return fail("nested too deeply", i);
        ws();
        if (i >= n) return fail("unexpected end", i);
        const unsigned char c = s[i];
        if (c == '{') {
            i++;
            out->kind = MzJson::OBJ;
            ws();
            if (i < n && s[i] == '}') {
                i++;
                return true;
            }
            for (;;) {
                ws();
                std::string k;
                if (!string(&k)) return false;
                if (!expect(':')) return false;
                out->obj.emplace_back(std::move(k), MzJson{});
                if (!val(&out->obj.back().second, depth + 1)) return false;
                ws();
                if (i >= n) return fail("unexpected end", i);
                const unsigned char d = s[i++];
                if (d == ',') continue;
                if (d == '}') return true;
                return fail("expected ',' or '}'", i - 1);
            }
        }
        if (c == '[') {
            i++;
            out->kind = MzJson::ARR;
            ws();
            if (i < n && s[i] == ']') {
                i++;
                return true;
            }
            for (;;) {
                out->arr.emplace_back();
                if (!val(&out->arr.back(), depth + 1)) return false;
                ws();
                if (i >= n) return fail("unexpected end", i);
                const unsigned char d = s[i++];
                if (d == ',') continue;
                if (d == ']') return true;
                return fail("expected ',' or ']'", i - 1);
            }
        }
        if (c == '"') {
            out->kind = MzJson::STR;
            return string(&out->str);
        }
        if (c == 't' || c == 'f' || c == 'n') {
            const size_t st = i;
            while (i < n && ((s[i] >= 'a' && s[i] <= 'z') || (s[i] >= 'A' && s[i] <= 'Z'))) i++;
            const size_t len = i - st;
            if (len == 4 && !memcmp(s + st, "true", 4)) {
                out->kind = MzJson::BOOL;
                out->b = true;
            } else if (len == 5 && !memcmp(s + st, "false", 5)) {
                out->kind = MzJson::BOOL;
                out->b = false;
            } else if (len == 4 && !memcmp(s + st, "null", 4)) {
                out->kind = MzJson::NUL;
            } else {
                return fail("bad literal", st);
            }
            return true;
        }
        return number(out);
    }
};

}  // namespace

const MzJson* MzJson::get(const char* key) const {
    if (kind != OBJ) return nullptr;
    for (auto& kv : obj)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

bool MzJson::uint(size_t* out) const {
    if (kind != NUM || !(num >= 0.0) || num != floor(num) || num > 9007199254740992.0) return false;
    *out = (size_t)num;
    return true;
}

bool MzJson::uints(std::vector<size_t>* out) const {
    if (kind != ARR) return false;
    std::vector<size_t> v(arr.size());
    for (size_t k = 0; k < arr.size(); k++)
        if (!arr[k].uint(&v[k])) return false;
    *out = std::move(v);
    return true;
}

bool mz_json_parse(const char* s, size_t n, MzJson* out, std::string* err) {
    Parser p{(const unsigned char*)s, n};
    MzJson v;
    if (!p.val(&v, 0)) {
        if (err) *err = p.err;
        return false;
    }
    p.ws();
    if (p.i != n) {
        p.fail("trailing data", p.i);
        if (err) *err = p.err;
        return false;
    }
    *out = std::move(v);
    return true;
}
