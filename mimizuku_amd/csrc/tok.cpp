// Text side, host only: the decoding half of Whisper's byte-level BPE tokenizer (src/tok.rs: vocab.json, byte
// table, decode with the HF clean-up of spaces, whole-character pieces with times) and the CLI's JSON result
// (src/main.rs:97-138: string escaping, Python's round(x, 2) as json.dumps prints it).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../include/mimizuku.h"
#include "mz_internal.h"
#include "mz_json.h"

struct mz_tok {
    std::vector<std::string> bytes;  // id -> raw bytes
};

namespace {

// GPT-2's byte <-> printable character table (tok.rs:10-22): bytes '!'..'~', 0xa1..0xac and 0xae..0xff map to the
// code point of the same value, every other byte to 256 + its rank among them. Returns the byte of code point cp,
// or -1.
int char_to_byte(unsigned cp) {
    static int table[324];
    static bool init = false;
    if (!init) {
        for (int& v : table) v = -1;
        bool printable[256] = {};
        for (int b = '!'; b <= '~'; b++) printable[b] = true;
        for (int b = 0xa1; b <= 0xac; b++) printable[b] = true;
        for (int b = 0xae; b <= 0xff; b++) printable[b] = true;
        int n = 0;
        for (int b = 0; b < 256; b++) {
            if (printable[b]) table[b] = b;
            else table[256 + n++] = b;
        }
        init = true;
    }
    return cp < 324 ? table[cp] : -1;
}

// next code point of UTF-8 text s (valid, from the JSON parser)
unsigned next_cp(const std::string& s, size_t* i) {
    const unsigned char c = (unsigned char)s[*i];
    int len = c < 0x80 ? 1 : (c & 0xe0) == 0xc0 ? 2 : (c & 0xf0) == 0xe0 ? 3 : 4;
    unsigned cp = len == 1 ? c : len == 2 ? (c & 0x1f) : len == 3 ? (c & 0x0f) : (c & 0x07);
    for (int k = 1; k < len; k++) cp = (cp << 6) | ((unsigned char)s[*i + k] & 0x3f);
    *i += len;
    return cp;
}

// String::from_utf8_lossy: every maximal invalid subsequence becomes U+FFFD (the WHATWG / Unicode "substitution of
// maximal subparts" rule that Rust follows)
std::string lossy(const std::string& b) {
    std::string o;
    const unsigned char* p = (const unsigned char*)b.data();
    size_t i = 0, n = b.size();
    while (i < n) {
        const unsigned c = p[i];
        if (c < 0x80) {
            o += (char)c;
            i++;
            continue;
        }
        int len;
        unsigned lo = 0x80, hi = 0xbf;
        if (c >= 0xc2 && c <= 0xdf) len = 2;
        else if (c >= 0xe0 && c <= 0xef) {
            len = 3;
            if (c == 0xe0) lo = 0xa0;
            if (c == 0xed) hi = 0x9f;
        } else if (c >= 0xf0 && c <= 0xf4) {
            len = 4;
            if (c == 0xf0) lo = 0x90;
            if (c == 0xf4) hi = 0x8f;
        } else {
            o += "\xef\xbf\xbd";
            i++;
            continue;
        }
        size_t k = 1;
        for (; k < (size_t)len; k++) {
            if (i + k >= n) break;
            const unsigned d = p[i + k];
            const unsigned l = k == 1 ? lo : 0x80, h = k == 1 ? hi : 0xbf;
            if (d < l || d > h) break;
        }
        if (k == (size_t)len) o.append(b, i, len);
        else o += "\xef\xbf\xbd";
        i += k;
    }
    return o;
}

// 0: valid UTF-8; 1: an incomplete sequence at the end only (more bytes could complete it); 2: invalid
int utf8_state(const std::string& b) {
    const unsigned char* p = (const unsigned char*)b.data();
    size_t i = 0, n = b.size();
    while (i < n) {
        const unsigned c = p[i];
        if (c < 0x80) {
            i++;
            continue;
        }
        int len;
        unsigned lo = 0x80, hi = 0xbf;
        if (c >= 0xc2 && c <= 0xdf) len = 2;
        else if (c >= 0xe0 && c <= 0xef) {
            len = 3;
            if (c == 0xe0) lo = 0xa0;
            if (c == 0xed) hi = 0x9f;
        } else if (c >= 0xf0 && c <= 0xf4) {
            len = 4;
            if (c == 0xf0) lo = 0x90;
            if (c == 0xf4) hi = 0x8f;
        } else {
            return 2;
        }
        for (size_t k = 1; k < (size_t)len; k++) {
            if (i + k >= n) return 1;
            const unsigned d = p[i + k];
            if (d < (k == 1 ? lo : 0x80u) || d > (k == 1 ? hi : 0xbfu)) return 2;
        }
        i += len;
    }
    return 0;
}

void replace_all(std::string& s, const char* a, const char* r) {
    const size_t la = strlen(a), lr = strlen(r);
    size_t at = 0;
    while ((at = s.find(a, at)) != std::string::npos) {
        s.replace(at, la, r);
        at += lr;
    }
}

const std::string& raw(const mz_tok* t, int id) {
    static const std::string empty;
    return id >= 0 && (size_t)id < t->bytes.size() ? t->bytes[id] : empty;
}

std::string decode(const mz_tok* t, const int32_t* ids, int n) {
    std::string b;
    for (int i = 0; i < n; i++) b += raw(t, ids[i]);
    std::string s = lossy(b);
    // clean_up_tokenization_spaces (tok.rs:50-54), in this order
    static const char* rep[][2] = {{" .", "."}, {" ?", "?"}, {" !", "!"}, {" ,", ","}, {" ' ", "'"},
                                   {" n't", "n't"}, {" 'm", "'m"}, {" 's", "'s"}, {" 've", "'ve"}, {" 're", "'re"}};
    for (auto& r : rep) replace_all(s, r[0], r[1]);
    return s;
}

struct Piece {
    std::string text;
    float t0, t1;
};

// tok.rs:63-86
std::vector<Piece> pieces(const mz_tok* t, const int32_t* ids, const float* ts, int n, int eos) {
    std::vector<Piece> out;
    std::vector<int32_t> buf;
    std::string bytes;
    float t0 = 0.f;
    for (int i = 0; i < n; i++) {
        if (ids[i] >= eos) continue;
        if (buf.empty()) t0 = ts[i];
        buf.push_back(ids[i]);
        bytes += raw(t, ids[i]);
        // complete once the bytes are valid UTF-8, or once they can no longer become valid
        if (utf8_state(bytes) != 1) {
            out.push_back({decode(t, buf.data(), (int)buf.size()), t0, i + 1 < n ? ts[i + 1] : ts[i]});
            buf.clear();
            bytes.clear();
        }
    }
    if (!buf.empty()) out.push_back({decode(t, buf.data(), (int)buf.size()), t0, n ? ts[n - 1] : t0});
    return out;
}

// main.rs:97-111
std::string json_str(const std::string& s) {
    std::string o = "\"";
    for (unsigned char c : s) {
        if (c == '"') o += "\\\"";
        else if (c == '\\') o += "\\\\";
        else if (c == '\n') o += "\\n";
        else if (c == '\r') o += "\\r";
        else if (c == '\t') o += "\\t";
        else if (c < 0x20) {
            char b[8];
            snprintf(b, sizeof b, "\\u%04x", c);
            o += b;
        } else o += (char)c;
    }
    return o + "\"";
}

// Python's round(x, 2) printed as json.dumps prints a float (main.rs:113-117): the value rounded to two decimals
// (correctly rounded from the exact binary value), then the shortest decimal that reads back as that double,
// with ".0" for whole numbers
std::string json_t(float x) {
    char b[64];
    snprintf(b, sizeof b, "%.2f", (double)x);
    const double v = strtod(b, nullptr);
    for (int prec = 1; prec <= 17; prec++) {
        snprintf(b, sizeof b, "%.*g", prec, v);
        if (strtod(b, nullptr) == v) break;
    }
    std::string s = b;
    // %g may use an exponent; two-decimal values below 1e16 print positionally in Rust's {:?}
    if (s.find('e') != std::string::npos) {
        snprintf(b, sizeof b, "%.2f", v);
        s = b;
        while (s.back() == '0') s.pop_back();
        if (s.back() == '.') s.pop_back();
    }
    if (s.find('.') == std::string::npos && s.find("inf") == std::string::npos && s.find("nan") == std::string::npos)
        s += ".0";
    return s;
}

int put_out(const std::string& s, char* out, size_t cap, size_t* len) {
    if (len) *len = s.size();
    if (out && cap > s.size()) memcpy(out, s.c_str(), s.size() + 1);
    return MZ_OK;
}

}  // namespace

extern "C" int mz_tok_open(const char* model_dir, int vocab, int eos, mz_tok** out) {
    if (!model_dir || !out) return mz_fail(MZ_ERR_ARG, "mz_tok_open: null argument");
    *out = nullptr;
    if (vocab <= 0) return mz_fail(MZ_ERR_ARG, "mz_tok_open: vocab %d", vocab);
    const std::string path = std::string(model_dir) + "/vocab.json";
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return mz_fail(MZ_ERR_ARG, "%s: cannot read", path.c_str());
    std::string text;
    char buf[1 << 16];
    size_t r;
    while ((r = fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, r);
    fclose(f);
    MzJson v;
    std::string err;
    if (!mz_json_parse(text.data(), text.size(), &v, &err)) return mz_fail(MZ_ERR_ARG, "vocab.json: %s", err.c_str());
    if (v.kind != MzJson::OBJ) return mz_fail(MZ_ERR_ARG, "vocab.json: not an object");
    std::vector<std::string> bytes(vocab);
    std::vector<char> set(vocab, 0);
    for (auto& kv : v.obj) {
        size_t id;
        if (!kv.second.uint(&id) || id >= (size_t)vocab)
            return mz_fail(MZ_ERR_ARG, "vocab.json: id of %s is not below the model's %d", kv.first.c_str(), vocab);
        if (set[id]) return mz_fail(MZ_ERR_ARG, "vocab.json: id of %s is used twice", kv.first.c_str());
        std::string b;
        size_t i = 0;
        while (i < kv.first.size()) {
            const unsigned cp = next_cp(kv.first, &i);
            const int byte = char_to_byte(cp);
            if (byte < 0) return mz_fail(MZ_ERR_ARG, "vocab.json: char U+%04X", cp);
            b += (char)byte;
        }
        bytes[id] = std::move(b);
        set[id] = 1;
    }
    for (int i = 0; i < eos && i < vocab; i++)
        if (!set[i]) return mz_fail(MZ_ERR_ARG, "vocab.json: no entry for text token %d", i);
    auto t = new mz_tok;
    t->bytes = std::move(bytes);
    *out = t;
    return MZ_OK;
}

extern "C" int mz_tok_from_bytes(const char* const* entries, const size_t* lens, int n, mz_tok** out) {
    if ((!entries && n) || (!lens && n) || !out || n < 0) return mz_fail(MZ_ERR_ARG, "mz_tok_from_bytes: bad argument");
    auto t = new mz_tok;
    for (int i = 0; i < n; i++) t->bytes.emplace_back(entries[i] ? std::string(entries[i], lens[i]) : std::string());
    *out = t;
    return MZ_OK;
}

extern "C" int mz_tok_free(mz_tok* t) {
    delete t;
    return MZ_OK;
}

extern "C" int mz_tok_decode(const mz_tok* t, const int32_t* ids, int n, char* out, size_t cap, size_t* len) {
    if (!t || (!ids && n > 0) || n < 0) return mz_fail(MZ_ERR_ARG, "mz_tok_decode: bad argument");
    return put_out(decode(t, ids, n), out, cap, len);
}

extern "C" int mz_tok_pieces(const mz_tok* t, const int32_t* ids, const float* ts, int n, int eos, char* text,
                             size_t cap, size_t* len, int32_t* offsets, float* t0, float* t1, int* n_pieces) {
    if (!t || (n > 0 && (!ids || !ts)) || n < 0 || !n_pieces) return mz_fail(MZ_ERR_ARG, "mz_tok_pieces: bad argument");
    auto ps = pieces(t, ids, ts, n, eos);
    std::string all;
    *n_pieces = (int)ps.size();
    for (size_t k = 0; k < ps.size(); k++) {
        if (offsets) offsets[k] = (int32_t)all.size();
        if (t0) t0[k] = ps[k].t0;
        if (t1) t1[k] = ps[k].t1;
        all += ps[k].text;
    }
    if (offsets) offsets[ps.size()] = (int32_t)all.size();
    return put_out(all, text, cap, len);
}

extern "C" int mz_json_time(float x, char* out, size_t cap, size_t* len) { return put_out(json_t(x), out, cap, len); }

// to_json (src/main.rs:121-138) for n clips: {path: {"language", "text", "words": [[piece, start, end], ...]}}
extern "C" int mz_results_json(const mz_tok* t, const mz_model* m, int n, const char* const* paths,
                               const int32_t* seq, const int32_t* seq_len, int stride, const float* ts,
                               const int32_t* langs, char* out, size_t cap, size_t* len) {
    if (!t || !m || n < 0 || (n > 0 && (!paths || !seq || !seq_len || !ts || !langs)))
        return mz_fail(MZ_ERR_ARG, "mz_results_json: bad argument");
    mz_gencfg g;
    mz_model_gencfg(m, &g);
    std::string o = "{";
    for (int i = 0; i < n; i++) {
        const int32_t* s = seq + (size_t)i * stride;
        const float* tt = ts + (size_t)i * stride;
        const int L = seq_len[i];
        auto ws = pieces(t, s, tt, L, g.eos);
        std::vector<int32_t> text_ids;
        for (int k = 0; k < L; k++)
            if (s[k] < g.eos) text_ids.push_back(s[k]);
        const std::string text = decode(t, text_ids.data(), (int)text_ids.size());
        std::string lang = "en";
        if (g.n_langs > 0) {
            lang = "";
            for (int k = 0; k < g.n_langs; k++) {
                const char* code;
                int32_t tok;
                mz_model_lang(m, k, &code, &tok);
                if (tok == langs[i]) {
                    lang = code;
                    break;
                }
            }
        }
        std::string wj;
        for (size_t k = 0; k < ws.size(); k++) {
            if (k) wj += ", ";
            wj += "[" + json_str(ws[k].text) + ", " + json_t(ws[k].t0) + ", " + json_t(ws[k].t1) + "]";
        }
        o += (i ? ", " : "") + json_str(paths[i]) + ": {\"language\": " + json_str(lang) + ", \"text\": " +
             json_str(text) + ", \"words\": [" + wj + "]}";
    }
    o += "}\n";
    return put_out(o, out, cap, len);
}
