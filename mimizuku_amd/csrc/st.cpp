// Model directory readers, host side: the safetensors file (src/st.rs), config.json (Dims::load, src/model.rs:33-61)
// and generation_config.json (GenCfg::load, src/model.rs:78-146), plus the engine's one-call open from a directory
// (Engine::new, src/model.rs:333-514) on top of mz_engine_new / mz_engine_put / mz_engine_finish.
#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/mimizuku.h"
#include "mz_internal.h"
#include "mz_json.h"

namespace {

// element size of a safetensors dtype, 0 if unknown (st.rs:83-91)
size_t elem_size(const std::string& dt) {
    if (dt == "F64" || dt == "I64" || dt == "U64") return 8;
    if (dt == "F32" || dt == "I32" || dt == "U32") return 4;
    if (dt == "F16" || dt == "BF16" || dt == "I16" || dt == "U16") return 2;
    if (dt == "I8" || dt == "U8" || dt == "BOOL" || dt == "F8_E4M3" || dt == "F8_E5M2") return 1;
    return 0;
}

bool read_file(const std::string& path, std::string* out) {
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return false;
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        close(fd);
        return false;
    }
    out->resize((size_t)sb.st_size);
    size_t got = 0;
    while (got < out->size()) {
        const ssize_t r = read(fd, &(*out)[got], out->size() - got);
        if (r <= 0) break;
        got += (size_t)r;
    }
    close(fd);
    out->resize(got);
    return true;
}

}  // namespace

struct mz_st {
    const unsigned char* bytes = nullptr;
    size_t len = 0;
    bool mapped = false;
    std::vector<unsigned char> owned;  // when the file cannot be mapped
    size_t start = 0;                  // first data byte
    struct Tensor {
        std::string name, dtype;
        std::vector<int64_t> shape;
        size_t a, b;  // data byte range relative to start
    };
    std::vector<Tensor> tensors;  // header order
    std::unordered_map<std::string, size_t> index;
    std::vector<std::pair<std::string, std::string>> meta;

    ~mz_st() {
        if (mapped) munmap((void*)bytes, len);
    }
};

extern "C" int mz_st_open(const char* path, mz_st** out) {
    if (!path || !out) return mz_fail(MZ_ERR_ARG, "mz_st_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return mz_fail(MZ_ERR_ARG, "%s: cannot open (%s)", path, strerror(errno));
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        close(fd);
        return mz_fail(MZ_ERR_ARG, "%s: cannot stat", path);
    }
    auto f = new mz_st;
    f->len = (size_t)sb.st_size;
    // a read-only private mapping of the whole file (no copy of a multi-GB checkpoint), read into memory otherwise
    void* m = f->len ? mmap(nullptr, f->len, PROT_READ, MAP_PRIVATE, fd, 0) : MAP_FAILED;
    if (m != MAP_FAILED) {
        madvise(m, f->len, MADV_WILLNEED);  // read ahead; a failure only costs speed
        f->bytes = (const unsigned char*)m;
        f->mapped = true;
    } else {
        f->owned.resize(f->len);
        size_t got = 0;
        while (got < f->len) {
            const ssize_t r = read(fd, f->owned.data() + got, f->len - got);
            if (r <= 0) break;
            got += (size_t)r;
        }
        f->owned.resize(got);
        f->len = got;
        f->bytes = f->owned.data();
    }
    close(fd);
    auto bad = [&](const std::string& what) {
        delete f;
        return mz_fail(MZ_ERR_ARG, "%s: not a valid safetensors file (%s)", path, what.c_str());
    };
    if (f->len < 8) return bad("too short");
    uint64_t n = 0;
    for (int k = 7; k >= 0; k--) n = (n << 8) | f->bytes[k];
    if (n > f->len - 8) return bad("header length");
    MzJson head;
    std::string err;
    if (!mz_json_parse((const char*)f->bytes + 8, (size_t)n, &head, &err)) {
        delete f;
        return mz_fail(MZ_ERR_ARG, "%s: %s", path, err.c_str());
    }
    if (head.kind != MzJson::OBJ) return bad("header is not an object");
    f->start = 8 + (size_t)n;
    const size_t data_len = f->len - f->start;
    std::vector<std::pair<size_t, size_t>> ranges;
    for (auto& kv : head.obj) {
        const std::string& k = kv.first;
        const MzJson& v = kv.second;
        if (k == "__metadata__") {
            if (v.kind == MzJson::OBJ)
                for (auto& mv : v.obj) f->meta.emplace_back(mv.first, mv.second.kind == MzJson::STR ? mv.second.str : "");
            continue;
        }
        const MzJson* dt = v.get("dtype");
        if (!dt || dt->kind != MzJson::STR) return bad("dtype");
        std::vector<size_t> shape, off;
        const MzJson* sh = v.get("shape");
        if (!sh || !sh->uints(&shape)) return bad("shape of " + k);
        const MzJson* of = v.get("data_offsets");
        if (of) of->uints(&off);
        // element count and byte size without overflow
        size_t numel = 1, size = 0;
        bool ok = elem_size(dt->str) != 0;
        for (size_t d : shape) {
            if (d && numel > SIZE_MAX / d) ok = false;
            else numel *= d;
        }
        if (ok && numel > SIZE_MAX / elem_size(dt->str)) ok = false;
        if (ok) size = numel * elem_size(dt->str);
        if (!ok || off.size() != 2 || off[0] > off[1] || off[1] > data_len || size != off[1] - off[0])
            return bad("offsets of " + k);
        ranges.emplace_back(off[0], off[1]);
        if (f->index.count(k)) return bad(k + " appears twice");
        f->index[k] = f->tensors.size();
        mz_st::Tensor t;
        t.name = k;
        t.dtype = dt->str;
        for (size_t d : shape) t.shape.push_back((int64_t)d);
        t.a = off[0];
        t.b = off[1];
        f->tensors.push_back(std::move(t));
    }
    std::sort(ranges.begin(), ranges.end());
    for (size_t i = 1; i < ranges.size(); i++)
        if (ranges[i].first < ranges[i - 1].second) return bad("overlapping tensors");
    *out = f;
    return MZ_OK;
}

extern "C" int mz_st_count(const mz_st* f, int* n) {
    if (!f || !n) return mz_fail(MZ_ERR_ARG, "mz_st_count: null argument");
    *n = (int)f->tensors.size();
    return MZ_OK;
}

extern "C" int mz_st_info(const mz_st* f, int i, const char** name, const char** dtype, int* ndim,
                          const int64_t** shape, const void** data, uint64_t* bytes) {
    if (!f) return mz_fail(MZ_ERR_ARG, "mz_st_info: null file");
    if (i < 0 || i >= (int)f->tensors.size()) return mz_fail(MZ_ERR_ARG, "mz_st_info: index %d out of range", i);
    const auto& t = f->tensors[i];
    if (name) *name = t.name.c_str();
    if (dtype) *dtype = t.dtype.c_str();
    if (ndim) *ndim = (int)t.shape.size();
    if (shape) *shape = t.shape.data();
    if (data) *data = f->bytes + f->start + t.a;
    if (bytes) *bytes = t.b - t.a;
    return MZ_OK;
}

extern "C" int mz_st_find(const mz_st* f, const char* name, int* i) {
    if (!f || !name || !i) return mz_fail(MZ_ERR_ARG, "mz_st_find: null argument");
    auto it = f->index.find(name);
    if (it == f->index.end()) return mz_fail(MZ_ERR_ARG, "missing tensor %s", name);
    *i = (int)it->second;
    return MZ_OK;
}

extern "C" int mz_st_meta(const mz_st* f, const char* key, const char** value) {
    if (!f || !key || !value) return mz_fail(MZ_ERR_ARG, "mz_st_meta: null argument");
    for (auto& kv : f->meta)
        if (kv.first == key) {
            *value = kv.second.c_str();
            return MZ_OK;
        }
    return mz_fail(MZ_ERR_ARG, "no metadata %s", key);
}

extern "C" int mz_st_close(mz_st* f) {
    delete f;
    return MZ_OK;
}

extern "C" int mz_json_check(const char* s, size_t n) {
    if (!s && n) return mz_fail(MZ_ERR_ARG, "mz_json_check: null text");
    MzJson v;
    std::string err;
    if (!mz_json_parse(s, n, &v, &err)) return mz_fail(MZ_ERR_ARG, "%s", err.c_str());
    return MZ_OK;
}

// ---------------------------------------------------------------- config.json and generation_config.json

struct mz_model {
    mz_dims dims{};
    int sot = 0, eos = 0, no_timestamps = 0;
    std::vector<int32_t> suppress, begin_suppress, lang_tokens, align;
    std::vector<std::string> lang_codes, task_names;
    std::vector<int32_t> task_tokens;
    std::string dir;
};

namespace {

int read_json(const std::string& path, MzJson* out) {
    std::string text;
    if (!read_file(path, &text)) return mz_fail(MZ_ERR_ARG, "%s: cannot read", path.c_str());
    std::string err;
    if (!mz_json_parse(text.data(), text.size(), out, &err))
        return mz_fail(MZ_ERR_ARG, "%s: %s", path.c_str(), err.c_str());
    return MZ_OK;
}

// Dims::load (src/model.rs:33-61)
int load_dims(const std::string& dir, mz_dims* d) {
    MzJson c;
    if (int r = read_json(dir + "/config.json", &c)) return r;
    int r = MZ_OK;
    auto n = [&](const char* k) -> int {
        size_t v = 0;
        const MzJson* j = c.get(k);
        if (!j || !j->uint(&v) || v < 1 || v >= (1u << 20)) {
            if (!r) r = mz_fail(MZ_ERR_ARG, "config.json: %s missing or out of range", k);
            return 0;
        }
        return (int)v;
    };
    d->d = n("d_model");
    d->ff = n("encoder_ffn_dim");
    d->nh = n("encoder_attention_heads");
    d->enc_layers = n("encoder_layers");
    d->dec_layers = n("decoder_layers");
    d->n_mels = n("num_mel_bins");
    d->vocab = n("vocab_size");
    d->max_t = n("max_target_positions");
    const int dh = n("decoder_attention_heads"), dff = n("decoder_ffn_dim"), src = n("max_source_positions");
    if (r) return r;
    if (d->nh * 64 != d->d || dh != d->nh || dff != d->ff)
        return mz_fail(MZ_ERR_ARG,
                       "unsupported shape (d %d, nh %d, ff %d): the kernels need 64-wide heads and equal "
                       "encoder/decoder widths",
                       d->d, d->nh, d->ff);
    if (src != 1500 || d->max_t < 16 || d->max_t > 448 || d->d % 128 != 0 || d->ff % 8 != 0 || d->enc_layers > 64 ||
        d->dec_layers > 64)
        return mz_fail(MZ_ERR_ARG, "unsupported shape (d %d, ff %d, max_t %d, layers %d/%d, source positions %d)",
                       d->d, d->ff, d->max_t, d->enc_layers, d->dec_layers, src);
    return MZ_OK;
}

// GenCfg::load (src/model.rs:78-146)
int load_gencfg(const std::string& dir, mz_model* m) {
    MzJson g;
    if (int r = read_json(dir + "/generation_config.json", &g)) return r;
    const int vocab = m->dims.vocab;
    auto token = [&](const MzJson* v, int32_t* t) {
        size_t u;
        if (!v || !v->uint(&u) || u >= (size_t)vocab) return false;
        *t = (int32_t)u;
        return true;
    };
    auto id = [&](const char* k, int* t) {
        int32_t v;
        if (!token(g.get(k), &v)) return mz_fail(MZ_ERR_ARG, "generation_config.json: %s missing or not a token id", k);
        *t = v;
        return MZ_OK;
    };
    auto map = [&](const char* k, bool strip, std::vector<std::string>* names, std::vector<int32_t>* toks) {
        const MzJson* j = g.get(k);
        if (!j) return MZ_OK;
        if (j->kind != MzJson::OBJ) return mz_fail(MZ_ERR_ARG, "generation_config.json: %s is not an object", k);
        for (auto& kv : j->obj) {
            std::string s = kv.first;
            if (strip) {
                // trim_start_matches("<|") / trim_end_matches("|>") remove every repetition of the pattern
                while (s.compare(0, 2, "<|") == 0) s.erase(0, 2);
                while (s.size() >= 2 && s.compare(s.size() - 2, 2, "|>") == 0) s.erase(s.size() - 2);
            }
            int32_t t;
            if (!token(&kv.second, &t))
                return mz_fail(MZ_ERR_ARG, "generation_config.json: %s.%s is not a token id", k, s.c_str());
            names->push_back(s);
            toks->push_back(t);
        }
        return MZ_OK;
    };
    auto ids = [&](const char* k, std::vector<int32_t>* out) {
        const MzJson* j = g.get(k);
        if (!j) return MZ_OK;
        if (j->kind != MzJson::ARR) return mz_fail(MZ_ERR_ARG, "generation_config.json: %s is not a list", k);
        for (auto& v : j->arr) {
            int32_t t;
            if (!token(&v, &t)) return mz_fail(MZ_ERR_ARG, "generation_config.json: %s has an invalid token id", k);
            out->push_back(t);
        }
        return MZ_OK;
    };
    const int L = m->dims.dec_layers, H = m->dims.nh;
    const MzJson* ah = g.get("alignment_heads");
    std::vector<std::pair<int, int>> heads;
    if (!ah) {
        // openai/whisper's default: every head of the second half of the decoder layers
        for (int l = L / 2; l < L; l++)
            for (int h = 0; h < H; h++) heads.emplace_back(l, h);
    } else if (ah->kind == MzJson::ARR) {
        for (auto& p : ah->arr) {
            std::vector<size_t> lh;
            if (!p.uints(&lh) || lh.size() != 2 || lh[0] >= (size_t)L || lh[1] >= (size_t)H)
                return mz_fail(MZ_ERR_ARG,
                               "generation_config.json: alignment_heads must be [layer, head] pairs within the model");
            heads.emplace_back((int)lh[0], (int)lh[1]);
        }
    } else {
        return mz_fail(MZ_ERR_ARG, "generation_config.json: alignment_heads is not a list");
    }
    auto uniq = heads;
    std::sort(uniq.begin(), uniq.end());
    if (heads.empty() || std::unique(uniq.begin(), uniq.end()) != uniq.end())
        return mz_fail(MZ_ERR_ARG, "generation_config.json: alignment_heads is empty or has duplicates");
    const MzJson* ml = g.get("is_multilingual");
    const bool multilingual = ml && ml->kind == MzJson::BOOL ? ml->b : true;
    if (int r = ids("begin_suppress_tokens", &m->begin_suppress)) return r;
    if (m->begin_suppress.size() > 2)
        return mz_fail(MZ_ERR_ARG, "generation_config.json: more than two begin_suppress_tokens are not supported");
    if (multilingual)
        if (int r = map("lang_to_id", true, &m->lang_codes, &m->lang_tokens)) return r;
    if (int r = map("task_to_id", false, &m->task_names, &m->task_tokens)) return r;
    if (multilingual && (m->lang_tokens.empty() || m->task_tokens.empty()))
        return mz_fail(MZ_ERR_ARG, "generation_config.json: a multilingual model needs lang_to_id and task_to_id");
    int r;
    if ((r = id("decoder_start_token_id", &m->sot)) || (r = id("eos_token_id", &m->eos)) ||
        (r = id("no_timestamps_token_id", &m->no_timestamps)) || (r = ids("suppress_tokens", &m->suppress)))
        return r;
    for (auto& p : heads) {
        m->align.push_back(p.first);
        m->align.push_back(p.second);
    }
    return MZ_OK;
}

}  // namespace

extern "C" int mz_model_open(const char* model_dir, mz_model** out) {
    if (!model_dir || !out) return mz_fail(MZ_ERR_ARG, "mz_model_open: null argument");
    *out = nullptr;
    auto m = new mz_model;
    m->dir = model_dir;
    int r = load_dims(m->dir, &m->dims);
    if (!r) r = load_gencfg(m->dir, m);
    if (r) {
        delete m;
        return r;
    }
    *out = m;
    return MZ_OK;
}

extern "C" int mz_model_dims(const mz_model* m, mz_dims* d) {
    if (!m || !d) return mz_fail(MZ_ERR_ARG, "mz_model_dims: null argument");
    *d = m->dims;
    return MZ_OK;
}

extern "C" int mz_model_gencfg(const mz_model* m, mz_gencfg* g) {
    if (!m || !g) return mz_fail(MZ_ERR_ARG, "mz_model_gencfg: null argument");
    g->sot = m->sot;
    g->eos = m->eos;
    g->no_timestamps = m->no_timestamps;
    g->suppress = m->suppress.data();
    g->n_suppress = (int)m->suppress.size();
    g->begin_suppress = m->begin_suppress.data();
    g->n_begin_suppress = (int)m->begin_suppress.size();
    g->lang_tokens = m->lang_tokens.data();
    g->n_langs = (int)m->lang_tokens.size();
    g->align_heads = m->align.data();
    g->n_align = (int)m->align.size() / 2;
    return MZ_OK;
}

extern "C" int mz_model_lang(const mz_model* m, int i, const char** code, int32_t* token) {
    if (!m) return mz_fail(MZ_ERR_ARG, "mz_model_lang: null model");
    if (i < 0 || i >= (int)m->lang_codes.size()) return mz_fail(MZ_ERR_ARG, "mz_model_lang: index %d out of range", i);
    if (code) *code = m->lang_codes[i].c_str();
    if (token) *token = m->lang_tokens[i];
    return MZ_OK;
}

extern "C" int mz_model_task(const mz_model* m, int i, const char** name, int32_t* token) {
    if (!m) return mz_fail(MZ_ERR_ARG, "mz_model_task: null model");
    if (i < 0 || i >= (int)m->task_names.size()) return mz_fail(MZ_ERR_ARG, "mz_model_task: index %d out of range", i);
    if (name) *name = m->task_names[i].c_str();
    if (token) *token = m->task_tokens[i];
    return MZ_OK;
}

extern "C" int mz_model_free(mz_model* m) {
    delete m;
    return MZ_OK;
}

// Every tensor of model.safetensors into the engine (Loader, src/model.rs:200-265), then the completeness check.
extern "C" int mz_engine_load(mz_engine* e, const char* model_dir) {
    if (!e || !model_dir) return mz_fail(MZ_ERR_ARG, "mz_engine_load: null argument");
    const std::string path = std::string(model_dir) + "/model.safetensors";
    mz_st* f = nullptr;
    if (int r = mz_st_open(path.c_str(), &f)) return r;
    int r = MZ_OK;
    for (const auto& t : f->tensors) {
        int dt;
        if (t.dtype == "F16") dt = MZ_DT_F16;
        else if (t.dtype == "F32") dt = MZ_DT_F32;
        else {
            r = mz_fail(MZ_ERR_ARG, "%s: %s is not F16 or F32", t.name.c_str(), t.dtype.c_str());
            break;
        }
        if ((r = mz_engine_put(e, t.name.c_str(), dt, f->bytes + f->start + t.a, t.shape.data(), (int)t.shape.size())))
            break;
    }
    mz_st_close(f);
    if (r) return r;
    return mz_engine_finish(e);
}

extern "C" int mz_engine_open(mz_ctx* c, const char* model_dir, int bmax, int eg, mz_engine** out) {
    if (!c || !model_dir || !out) return mz_fail(MZ_ERR_ARG, "mz_engine_open: null argument");
    *out = nullptr;
    mz_model* m = nullptr;
    if (int r = mz_model_open(model_dir, &m)) return r;
    mz_gencfg g;
    mz_model_gencfg(m, &g);
    mz_engine* e = nullptr;
    int r = mz_engine_new(c, &m->dims, &g, bmax, eg, &e);
    mz_model_free(m);
    if (r) return r;
    if ((r = mz_engine_load(e, model_dir))) {
        mz_engine_free(e);
        return r;
    }
    *out = e;
    return MZ_OK;
}
