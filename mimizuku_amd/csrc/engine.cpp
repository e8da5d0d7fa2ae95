// The Whisper engine behind the C ABI: weight placement, the encoder pass, the decoder step (captured as one graph
// with the position in device memory) and the batch transcription loop. Mirrors src/model.rs (Engine::{new, encode,
// reset, detect, step}) and src/transcribe.rs (transcribe), with its own kernels and data layouts:
//   * the residual streams are fp32 (encoder [clips*1500][d], decoder [bmax][d]); GEMM operands are fp16;
//   * encoder q/k/v and every decoder layer's cross k/v are stored per head as 1536 x 64 tiles, v transposed;
//   * the self-attention cache is per (row, head): k and v both [max_t][64] (one 128-byte row per position).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <map>
#include <set>
#include <atomic>
#include <string>
#include <thread>
#include <vector>

#include "../../include/mimizuku.h"
#include "mz_internal.h"
#include "mz_kernels.h"

namespace {

constexpr int HD = 64, TENC = 1500, TPAD = 1536, NFR = 3000;
constexpr float EPS = 1e-5f;

struct Ln {
    f16 *w = nullptr, *b = nullptr;
};
struct Lin {
    f16 *w = nullptr, *b = nullptr;
};
struct EncLayer {
    Ln ln1, ln2;
    Lin qkv, o, fc1, fc2;
};
struct DecLayer {
    Ln ln1, lnx, ln3;
    Lin qkv, o, xq, xo, fc1, fc2;
};

// where a checkpoint tensor goes: rows [row0, row0 + rows) of a [.][cols] destination
struct Slot {
    f16* dst;
    std::vector<int64_t> shape;
    int kind;  // 0 plain copy, 1 conv weight reordered tap-major into rows of kpad columns
    int kpad;
};

inline int rup(int x, int m) { return (x + m - 1) / m * m; }

}  // namespace

#ifndef MZ_ENC_LANES
#define MZ_ENC_LANES 2  // encoder groups in flight at once in mz_transcribe
#endif

struct EncBufs {
    float* mel;
    f16 *melT, *h1, *hb, *qkvh, *att, *ff, *dd;
    float* ex;
};

// Pinned host staging for uploads (the reference's Arena, src/gpu.rs:289-374, stages weights through two pinned
// buffers): data is written into one buffer while the other's copy to the device is in flight, each buffer's copy
// marked by an event that the next writer of that buffer waits for.
struct Staging {
    static constexpr size_t CAP = (size_t)32 << 20;  // bytes per buffer
    void* buf[2] = {};
    hipEvent_t ev[2] = {};
    int next = 0;
    int init() {
        if (buf[0]) return MZ_OK;
        for (int i = 0; i < 2; i++) {
            if (int r = mz_hip(hipHostMalloc(&buf[i], CAP, hipHostMallocDefault), "hipHostMalloc (staging)")) return r;
            if (int r = mz_hip(hipEventCreateWithFlags(&ev[i], hipEventDisableTiming), "hipEventCreate")) return r;
        }
        return MZ_OK;
    }
    // the buffer the next chunk goes into, once its previous copy has finished
    int acquire(void** p) {
        if (int r = mz_hip(hipEventSynchronize(ev[next]), "staging wait")) return r;
        *p = buf[next];
        return MZ_OK;
    }
    int submit(void* dst, size_t bytes, hipStream_t s) {
        if (int r = mz_hip(hipMemcpyAsync(dst, buf[next], bytes, hipMemcpyHostToDevice, s), "staged upload")) return r;
        if (int r = mz_hip(hipEventRecord(ev[next], s), "hipEventRecord")) return r;
        next ^= 1;
        return MZ_OK;
    }
    void release() {
        for (int i = 0; i < 2; i++) {
            if (ev[i]) {
                hipEventSynchronize(ev[i]);
                hipEventDestroy(ev[i]);
                ev[i] = nullptr;
            }
            if (buf[i]) {
                hipHostFree(buf[i]);
                buf[i] = nullptr;
            }
        }
        next = 0;
    }
};

struct mz_engine {
    mz_ctx* c = nullptr;
    mz_dims dm{};
    int bmax = 0, eg = 0, na = 0;
    int sot = 0, eos = 0, bs1 = -1, bs2 = -1;
    std::vector<int> align_heads;  // pairs
    bool trace_on = false;
    bool capturing = false;  // inside mz_engine_capture: no trace copies go into the graph
    bool loaded = false;

    // weights
    f16* arena = nullptr;
    size_t arena_elems = 0, arena_used = 0;
    std::map<std::string, Slot> slots;
    std::set<std::string> placed;
    Staging wstage;  // weight uploads, until mz_engine_finish
    // host log-mel of a group staged per encoder lane (pinned, allocated at the first host upload), and the event of
    // its last copy
    float* mel_pin[MZ_ENC_LANES] = {};
    hipEvent_t mel_ev[MZ_ENC_LANES] = {};
    EncLayer* enc = nullptr;
    DecLayer* dec = nullptr;
    std::vector<EncLayer> encv;
    std::vector<DecLayer> decv;
    Lin conv1, conv2, xkv;
    Ln eln, dln;
    f16 *epos = nullptr, *emb = nullptr, *dpos = nullptr;
    int k1pad = 0;

    // encoder scratch (eg clips)
    float* mel = nullptr;
    f16 *melT = nullptr, *h1 = nullptr, *hb = nullptr, *qkvh = nullptr, *att = nullptr, *ff = nullptr;
    f16* dd = nullptr;  // out-projection / fc2 output, added to the residual stream by the next add + LayerNorm
    float *ex = nullptr, *trace = nullptr;
    float* dtrace = nullptr;  // decoder residual entering every layer and after the last, [nl + 1][bmax][d]
    // more encoder lanes for batches of several groups: each with its own scratch and stream, so that one group's
    // bandwidth-bound kernels and kernel tails overlap another's products (the groups are independent)
    EncBufs lanes[MZ_ENC_LANES - 1]{};
    hipStream_t ls[MZ_ENC_LANES - 1]{};
    hipEvent_t fork = nullptr, join[MZ_ENC_LANES - 1]{};
    // decoder state (bmax rows)
    f16* xkvbuf = nullptr;
    int *tok = nullptr, *done = nullptr, *ctr = nullptr;
    float *x = nullptr, *part = nullptr, *logits = nullptr;
    f16 *h = nullptr, *datt = nullptr, *dff = nullptr, *kc = nullptr, *vc = nullptr;
    float* align = nullptr;  // alignment-head probabilities [bmax][max_t][na][1500], fp32
    f16* alignh = nullptr;   // the same rows rounded to fp16 (the reference's own buffer, src/model.rs:455)
    int2* amax = nullptr;  // LM head argmax partials [mz_lm_blocks(vocab)][bmax]
    int* aslot = nullptr;
    unsigned char *sup = nullptr, *sup_lang = nullptr;
    size_t part_elems = 0;
    mz_graph* graph = nullptr;
    int graph_b = -1, graph_np = -1;
    // the chunk submitted and not yet collected (mz_transcribe_submit / mz_transcribe_collect): its clip count (0:
    // none) and the host time spent enqueueing its encoder; enc_done marks its encoder done
    int pending_n = 0;
    double pending_enq = 0;
    hipEvent_t enc_done = nullptr;
    // the decode loop's end test: the rows' done flags copied to pinned memory a few steps before they are read
    int* done_pin = nullptr;
    hipEvent_t done_ev = nullptr;
    // kernel timing (mz_engine_profile): events around each encoder launch and each decoder step
    bool prof_on = false;
    struct Rec {
        int id;
        hipEvent_t a, b;
    };
    std::vector<Rec> recs;
    std::vector<hipEvent_t> evpool;
    hipEvent_t ev() {
        if (!evpool.empty()) {
            hipEvent_t x = evpool.back();
            evpool.pop_back();
            return x;
        }
        hipEvent_t x = nullptr;
        if (hipEventCreate(&x) != hipSuccess) return nullptr;
        return x;
    }
    // token timestamps (k_align.hip): per clip (rows, columns), column statistics, DTW cost and trace in
    // anti-diagonal-major order for up to max_t - 1 rows, and the start time of every row
    int2* ts_rc = nullptr;
    float *ts_mean = nullptr, *ts_sd = nullptr, *ts_cost = nullptr, *ts_out = nullptr;
    signed char* ts_trace = nullptr;
    // position of the next step as the host has enqueued it (the device copy is ctr[0]); steps beyond the cache
    // (max_t - 1 of them after a reset) are refused
    int host_pos = 0;

    template <class T>
    int alloc(T** p, size_t n) {
        void* v;
        if (int r = mz_ctx_alloc(c, n * sizeof(T), &v)) return r;
        *p = (T*)v;
        return MZ_OK;
    }
    f16* take(size_t n) {
        f16* p = arena + arena_used;
        arena_used += (n + 127) / 128 * 128;  // 256-byte aligned tensors
        return p;
    }
};

namespace {

size_t weight_elems(const mz_dims& d, int* k1pad) {
    const size_t D = d.d, F = d.ff;
    auto r = [](size_t n) { return (n + 127) / 128 * 128; };
    *k1pad = rup(3 * d.n_mels, 64);
    size_t n = r(D * *k1pad) + r(D) + r(D * 3 * D) + r(D) + r((size_t)TENC * D) + 2 * r(D);
    size_t enc = 4 * r(D) + r(3 * D * D) + r(3 * D) + r(D * D) + r(D) + r(F * D) + r(F) + r(D * F) + r(D);
    size_t dec = 6 * r(D) + r(3 * D * D) + r(3 * D) + 3 * (r(D * D) + r(D)) + r(F * D) + r(F) + r(D * F) + r(D);
    n += d.enc_layers * enc + d.dec_layers * dec;
    n += r((size_t)d.dec_layers * 2 * D * D) + r((size_t)d.dec_layers * 2 * D);
    n += r((size_t)d.vocab * D) + r((size_t)d.max_t * D) + 2 * r(D);
    return n;
}

// one set of cross keys/values: [bmax][dec layers][k|v][heads] tiles of 1536 x 64
size_t xkv_elems(const mz_dims& d, int bmax) { return (size_t)bmax * d.dec_layers * 2 * d.nh * (size_t)TPAD * HD; }

int ksplit_for(int N, int K) {
    // Split K over workgroups until the grid covers most of the 256 CUs, with at most 16 groups of 64 per workgroup
    // (a slice within MZ_DEC_KSLICE, both operands resident in LDS) and at most MZ_MAX_PARTS partials.
    const int tiles = (N + 31) / 32, groups = K / 64;
    int best = 1;
    for (int ks = 1; ks <= std::min(groups, MZ_MAX_PARTS); ks++) {
        if (groups % ks) continue;
        best = ks;
        if (groups / ks <= 16 && (long)tiles * ks >= 192) break;
    }
    return best;
}

// elements of the decoder's split-K partials buffer: the largest ks * rows * n over the decoder products
size_t part_elems(int D, int F, int B) {
    size_t pe = 0;
    for (auto nk : {std::pair<int, int>{D, D}, {D, F}, {3 * D, D}})
        pe = std::max(pe, (size_t)ksplit_for(nk.first, nk.second) * B * nk.first);
    return pe;
}

}  // namespace

extern "C" size_t mz_scratch_bytes(const mz_dims* d, int n_align, int bmax, int eg) {
    if (!d) return 0;
    const size_t D = d->d, F = d->ff, nl = d->dec_layers, nh = d->nh, mt = d->max_t, V = d->vocab;
    const size_t B = bmax, G = eg;
    size_t enc = G * d->n_mels * NFR * 4 + G * NFR * d->n_mels * 2 + G * NFR * D * 2 + G * TENC * D * 4 +
                 G * TENC * D * 2 * 3 + G * 3 * nh * TPAD * HD * 2 + G * TENC * F * 2;
    size_t dec = B * nl * 2 * nh * TPAD * HD * 2 + B * mt * 4 + B * 4 + 16 + B * D * 4 + B * D * 2 * 2 + B * F * 2 +
                 2 * nl * B * nh * mt * HD * 2 + B * V * 4 + B * mt * n_align * TENC * (4 + 2) + (size_t)mz_lm_blocks((int)V) * B * 8 +
                 nl * nh * 4 + 2 * V;
    size_t part = part_elems((int)D, (int)F, (int)B) * 4;
    size_t ts = B * 8 + 2 * B * n_align * TENC * 4 + B * (size_t)mz_ts_diag_stride((int)mt - 1, TENC) * 5 + B * mt * 4;
    return MZ_ENC_LANES * enc + dec + part + ts;
}

extern "C" int mz_engine_new(mz_ctx* c, const mz_dims* d, const mz_gencfg* g, int bmax, int eg, mz_engine** out) {
    if (!c || !d || !g || !out) return mz_fail(MZ_ERR_ARG, "mz_engine_new: null argument");
    *out = nullptr;
    // geometry limits (Dims::load, src/model.rs:47-59) plus the library's own: d % 128 == 0 and d <= 1280 (the decoder's
    // unsplit products, the LM head and the cross-attention's query projection hold a whole row of K in LDS)
    if (d->nh * HD != d->d || d->d % 128 || d->d > MZ_DEC_KSLICE || d->ff % 64 || d->ff <= 0 || d->n_mels % 8 ||
        d->n_mels <= 0 || d->max_t < 16 || d->max_t > 448 || d->max_t % 8 || d->enc_layers < 1 || d->enc_layers > 64 ||
        d->dec_layers < 1 || d->dec_layers > 64 || d->vocab <= 0)
        return mz_fail(MZ_ERR_ARG,
                       "unsupported shape d=%d ff=%d nh=%d n_mels=%d max_t=%d layers=%d/%d: the kernels need 64-wide "
                       "heads, d %% 128 == 0 (<= 1280), ff %% 64 == 0, n_mels %% 8 == 0, max_t %% 8 == 0 in [16, 448]",
                       d->d, d->ff, d->nh, d->n_mels, d->max_t, d->enc_layers, d->dec_layers);
    if (bmax <= 0 || eg <= 0 || eg > bmax) return mz_fail(MZ_ERR_ARG, "bmax %d / enc group %d", bmax, eg);
    if (g->n_begin_suppress > 2) return mz_fail(MZ_ERR_ARG, "more than two begin_suppress tokens are not supported");
    if (g->n_align <= 0) return mz_fail(MZ_ERR_ARG, "alignment_heads is empty");
    std::set<std::pair<int, int>> uniq;
    for (int i = 0; i < g->n_align; i++) {
        int l = g->align_heads[2 * i], hh = g->align_heads[2 * i + 1];
        if (l < 0 || l >= d->dec_layers || hh < 0 || hh >= d->nh)
            return mz_fail(MZ_ERR_ARG, "alignment head (%d, %d) outside the model", l, hh);
        uniq.insert({l, hh});
    }
    if ((int)uniq.size() != g->n_align) return mz_fail(MZ_ERR_ARG, "alignment_heads has duplicates");
    for (int t : {g->sot, g->eos, g->no_timestamps})
        if (t < 0 || t >= d->vocab) return mz_fail(MZ_ERR_ARG, "special token %d out of range", t);

    auto* e = new mz_engine();
    e->c = c;
    e->dm = *d;
    e->bmax = bmax;
    e->eg = eg;
    e->na = g->n_align;
    e->sot = g->sot;
    e->eos = g->eos;
    e->bs1 = g->n_begin_suppress > 0 ? g->begin_suppress[0] : -1;
    e->bs2 = g->n_begin_suppress > 1 ? g->begin_suppress[1] : -1;
    e->align_heads.assign(g->align_heads, g->align_heads + 2 * g->n_align);
    auto fail = [&](int r) {
        mz_engine_free(e);
        return r;
    };

    // pre-flight memory check (src/model.rs:343-357)
    const size_t welems = weight_elems(*d, &e->k1pad);
    const size_t need = welems * 2 + mz_scratch_bytes(d, e->na, bmax, eg);
    size_t fr = 0, tot = 0;
    if (hipMemGetInfo(&fr, &tot) == hipSuccess && need > tot)
        return fail(mz_fail(MZ_ERR_ARG, "not enough GPU memory: about %.1f GB needed for bmax %d / enc group %d, %.1f GB total",
                            need / 1e9, bmax, eg, tot / 1e9));

    if (int r = e->alloc(&e->arena, welems)) return fail(r);
    e->arena_elems = welems;
    const int D = d->d, F = d->ff, nl = d->dec_layers, nh = d->nh, mt = d->max_t, V = d->vocab;
    const int64_t D6 = D;
    auto lin = [&](Lin& L, const std::string& p, int n, int k, bool bias_from_ckpt = true) {
        L.w = e->take((size_t)n * k);
        L.b = e->take(n);
        e->slots[p + ".weight"] = Slot{L.w, {n, k}, 0, 0};
        if (bias_from_ckpt) e->slots[p + ".bias"] = Slot{L.b, {n}, 0, 0};
    };
    auto ln = [&](Ln& L, const std::string& p) {
        L.w = e->take(D);
        L.b = e->take(D);
        e->slots[p + ".weight"] = Slot{L.w, {D6}, 0, 0};
        e->slots[p + ".bias"] = Slot{L.b, {D6}, 0, 0};
    };
    auto qkv = [&](Lin& L, const std::string& p) {  // q, k, v fused into [3D][D]; k has no bias (zeros)
        L.w = e->take((size_t)3 * D * D);
        L.b = e->take(3 * D);
        e->slots[p + ".q_proj.weight"] = Slot{L.w, {D6, D6}, 0, 0};
        e->slots[p + ".k_proj.weight"] = Slot{L.w + (size_t)D * D, {D6, D6}, 0, 0};
        e->slots[p + ".v_proj.weight"] = Slot{L.w + (size_t)2 * D * D, {D6, D6}, 0, 0};
        e->slots[p + ".q_proj.bias"] = Slot{L.b, {D6}, 0, 0};
        e->slots[p + ".v_proj.bias"] = Slot{L.b + 2 * D, {D6}, 0, 0};
    };
    // conv weights [D][cin][3] -> tap-major rows w'[co][tap * cin + ci], K padded to a multiple of 64
    e->conv1.w = e->take((size_t)D * e->k1pad);
    e->conv1.b = e->take(D);
    e->slots["model.encoder.conv1.weight"] = Slot{e->conv1.w, {D6, d->n_mels, 3}, 1, e->k1pad};
    e->slots["model.encoder.conv1.bias"] = Slot{e->conv1.b, {D6}, 0, 0};
    e->conv2.w = e->take((size_t)D * 3 * D);
    e->conv2.b = e->take(D);
    e->slots["model.encoder.conv2.weight"] = Slot{e->conv2.w, {D6, D6, 3}, 1, 3 * D};
    e->slots["model.encoder.conv2.bias"] = Slot{e->conv2.b, {D6}, 0, 0};
    e->epos = e->take((size_t)TENC * D);
    e->slots["model.encoder.embed_positions.weight"] = Slot{e->epos, {TENC, D6}, 0, 0};
    e->encv.resize(d->enc_layers);
    for (int i = 0; i < d->enc_layers; i++) {
        std::string p = "model.encoder.layers." + std::to_string(i);
        EncLayer& L = e->encv[i];
        ln(L.ln1, p + ".self_attn_layer_norm");
        qkv(L.qkv, p + ".self_attn");
        lin(L.o, p + ".self_attn.out_proj", D, D);
        ln(L.ln2, p + ".final_layer_norm");
        lin(L.fc1, p + ".fc1", F, D);
        lin(L.fc2, p + ".fc2", D, F);
    }
    ln(e->eln, "model.encoder.layer_norm");
    e->decv.resize(nl);
    // every decoder layer's cross k/v projection fused: [nl][k|v][D] rows of D, bias [0 | v bias] per layer
    e->xkv.w = e->take((size_t)nl * 2 * D * D);
    e->xkv.b = e->take((size_t)nl * 2 * D);
    for (int i = 0; i < nl; i++) {
        std::string p = "model.decoder.layers." + std::to_string(i);
        DecLayer& L = e->decv[i];
        ln(L.ln1, p + ".self_attn_layer_norm");
        qkv(L.qkv, p + ".self_attn");
        lin(L.o, p + ".self_attn.out_proj", D, D);
        ln(L.lnx, p + ".encoder_attn_layer_norm");
        lin(L.xq, p + ".encoder_attn.q_proj", D, D);
        lin(L.xo, p + ".encoder_attn.out_proj", D, D);
        ln(L.ln3, p + ".final_layer_norm");
        lin(L.fc1, p + ".fc1", F, D);
        lin(L.fc2, p + ".fc2", D, F);
        e->slots[p + ".encoder_attn.k_proj.weight"] = Slot{e->xkv.w + (size_t)(2 * i) * D * D, {D6, D6}, 0, 0};
        e->slots[p + ".encoder_attn.v_proj.weight"] = Slot{e->xkv.w + (size_t)(2 * i + 1) * D * D, {D6, D6}, 0, 0};
        e->slots[p + ".encoder_attn.v_proj.bias"] = Slot{e->xkv.b + (size_t)(2 * i + 1) * D, {D6}, 0, 0};
    }
    e->emb = e->take((size_t)V * D);
    e->slots["model.decoder.embed_tokens.weight"] = Slot{e->emb, {V, D6}, 0, 0};
    e->dpos = e->take((size_t)mt * D);
    e->slots["model.decoder.embed_positions.weight"] = Slot{e->dpos, {mt, D6}, 0, 0};
    ln(e->dln, "model.decoder.layer_norm");
    if (e->arena_used > e->arena_elems) return fail(mz_fail(MZ_ERR_STATE, "weight arena too small"));

    // scratch
    const size_t G = eg, B = bmax;
    int r = 0;
    if ((r = e->alloc(&e->mel, G * d->n_mels * NFR)) || (r = e->alloc(&e->melT, G * NFR * d->n_mels)) ||
        (r = e->alloc(&e->h1, G * NFR * D)) || (r = e->alloc(&e->ex, G * TENC * D)) ||
        (r = e->alloc(&e->hb, G * TENC * D)) || (r = e->alloc(&e->qkvh, G * 3 * nh * (size_t)TPAD * HD)) ||
        (r = e->alloc(&e->att, G * TENC * D)) || (r = e->alloc(&e->ff, G * TENC * F)) ||
        (r = e->alloc(&e->dd, G * TENC * D)))
        return fail(r);
    if ((r = mz_hip(hipEventCreateWithFlags(&e->fork, hipEventDisableTiming), "hipEventCreate"))) return fail(r);
    for (int k = 0; k < MZ_ENC_LANES - 1; k++) {
        EncBufs& l = e->lanes[k];
        if ((r = e->alloc(&l.mel, G * d->n_mels * NFR)) || (r = e->alloc(&l.melT, G * NFR * d->n_mels)) ||
            (r = e->alloc(&l.h1, G * NFR * D)) || (r = e->alloc(&l.ex, G * TENC * D)) ||
            (r = e->alloc(&l.hb, G * TENC * D)) || (r = e->alloc(&l.qkvh, G * 3 * nh * (size_t)TPAD * HD)) ||
            (r = e->alloc(&l.att, G * TENC * D)) || (r = e->alloc(&l.ff, G * TENC * F)) ||
            (r = e->alloc(&l.dd, G * TENC * D)))
            return fail(r);
        // default priority (as the context's stream)
        if ((r = mz_hip(hipStreamCreateWithFlags(&e->ls[k], hipStreamNonBlocking), "hipStreamCreate")) ||
            (r = mz_hip(hipEventCreateWithFlags(&e->join[k], hipEventDisableTiming), "hipEventCreate")))
            return fail(r);
    }
    if ((r = mz_hip(hipEventCreateWithFlags(&e->enc_done, hipEventDisableTiming), "hipEventCreate")) ||
        (r = mz_hip(hipEventCreateWithFlags(&e->done_ev, hipEventDisableTiming), "hipEventCreate")) ||
        (r = mz_hip(hipHostMalloc((void**)&e->done_pin, B * 4, hipHostMallocDefault), "hipHostMalloc (done)")))
        return fail(r);
    if ((r = e->alloc(&e->xkvbuf, xkv_elems(*d, bmax))) || (r = e->alloc(&e->tok, B * mt)) ||
        (r = e->alloc(&e->done, B)) || (r = e->alloc(&e->ctr, 4)) || (r = e->alloc(&e->x, B * D)) ||
        (r = e->alloc(&e->h, B * D)) || (r = e->alloc(&e->datt, B * D)) ||
        (r = e->alloc(&e->dff, B * F)) || (r = e->alloc(&e->kc, (size_t)nl * B * nh * mt * HD)) ||
        (r = e->alloc(&e->vc, (size_t)nl * B * nh * mt * HD)) || (r = e->alloc(&e->logits, B * V)) ||
        (r = e->alloc(&e->align, B * mt * e->na * (size_t)TENC)) ||
        (r = e->alloc(&e->alignh, B * mt * e->na * (size_t)TENC)) ||
        (r = e->alloc(&e->amax, (size_t)mz_lm_blocks(V) * B)) ||
        (r = e->alloc(&e->aslot, (size_t)nl * nh)) || (r = e->alloc(&e->sup, V)) || (r = e->alloc(&e->sup_lang, V)))
        return fail(r);
    const size_t tsd = (size_t)mz_ts_diag_stride(mt - 1, TENC);
    if ((r = e->alloc(&e->ts_rc, B)) || (r = e->alloc(&e->ts_mean, B * e->na * (size_t)TENC)) ||
        (r = e->alloc(&e->ts_sd, B * e->na * (size_t)TENC)) || (r = e->alloc(&e->ts_cost, B * tsd)) ||
        (r = e->alloc(&e->ts_trace, B * tsd)) || (r = e->alloc(&e->ts_out, B * mt)))
        return fail(r);
    const size_t pe = part_elems(D, F, (int)B);
    e->part_elems = pe;
    if ((r = e->alloc(&e->part, pe))) return fail(r);

    // masks and alignment slots (src/model.rs:411-425)
    std::vector<unsigned char> supm(V, 0), langm(V, 1);
    for (int i = 0; i < g->n_suppress; i++) {
        int t = g->suppress[i];
        if (t < 0 || t >= V) return fail(mz_fail(MZ_ERR_ARG, "suppress token %d out of range", t));
        supm[t] = 1;
    }
    for (int i = 0; i < g->n_langs; i++) {
        int t = g->lang_tokens[i];
        if (t < 0 || t >= V) return fail(mz_fail(MZ_ERR_ARG, "language token %d out of range", t));
        langm[t] = 0;
    }
    std::vector<int> sl((size_t)nl * nh, -1);
    for (int s = 0; s < e->na; s++) sl[(size_t)e->align_heads[2 * s] * nh + e->align_heads[2 * s + 1]] = s;
    if ((r = mz_upload(c, (uint64_t)(uintptr_t)e->sup, supm.data(), V)) ||
        (r = mz_upload(c, (uint64_t)(uintptr_t)e->sup_lang, langm.data(), V)) ||
        (r = mz_upload(c, (uint64_t)(uintptr_t)e->aslot, sl.data(), sl.size() * 4)))
        return fail(r);
    *out = e;
    return MZ_OK;
}

extern "C" int mz_engine_put(mz_engine* e, const char* name, int dtype, const void* data, const int64_t* shape,
                             int ndim) {
    if (!e || !name || !data || (!shape && ndim)) return mz_fail(MZ_ERR_ARG, "mz_engine_put: null argument");
    auto it = e->slots.find(name);
    if (it == e->slots.end()) return MZ_OK;  // tensors the engine does not use (e.g. the tied proj_out) are ignored
    const Slot& s = it->second;
    if ((int)s.shape.size() != ndim || !std::equal(s.shape.begin(), s.shape.end(), shape)) {
        std::string want, got;
        for (auto v : s.shape) want += std::to_string(v) + ",";
        for (int i = 0; i < ndim; i++) got += std::to_string(shape[i]) + ",";
        return mz_fail(MZ_ERR_ARG, "%s has shape [%s], expected [%s]", name, got.c_str(), want.c_str());
    }
    if (dtype != MZ_DT_F16 && dtype != MZ_DT_F32) return mz_fail(MZ_ERR_ARG, "%s: unsupported dtype %d", name, dtype);
    // element i of the source as binary16 bits
    const uint16_t* h = (const uint16_t*)data;
    const float* f = (const float*)data;
    auto src = [&](size_t i) { return dtype == MZ_DT_F16 ? h[i] : mz_f2h_host(f[i]); };
    // the destination layout, rows of `cols` halves: the tensor itself (one row), or a conv weight [co][ci][3]
    // reordered tap-major into rows [co][kpad] (column tap * ci + ci_index, zero padding after 3 ci)
    size_t n = 1;
    for (auto v : s.shape) n *= (size_t)v;
    const bool conv = s.kind == 1;
    const size_t ci = conv ? (size_t)s.shape[1] : 0, cols = conv ? (size_t)s.kpad : n, rows = conv ? (size_t)s.shape[0] : 1;
    // converted chunk by chunk into the pinned staging buffers, each chunk's copy in flight while the next is written
    if (int r = e->wstage.init()) return r;
    const size_t per = Staging::CAP / 2;  // halves per chunk
    const size_t total = rows * cols;
    for (size_t o0 = 0; o0 < total; o0 += per) {
        const size_t k = std::min(per, total - o0);
        void* pv;
        if (int r = e->wstage.acquire(&pv)) return r;
        uint16_t* out = (uint16_t*)pv;
        if (!conv) {
            if (dtype == MZ_DT_F16)
                std::memcpy(out, h + o0, k * 2);
            else
                for (size_t i = 0; i < k; i++) out[i] = mz_f2h_host(f[o0 + i]);
        } else {
            for (size_t i = 0; i < k; i++) {
                const size_t o = (o0 + i) / cols, c = (o0 + i) % cols, t = c / ci, cc = c % ci;
                out[i] = t < 3 ? src((o * ci + cc) * 3 + t) : (uint16_t)0;
            }
        }
        if (int r = e->wstage.submit(s.dst + o0, k * 2, e->c->stream)) return r;
    }
    e->placed.insert(name);
    return MZ_OK;
}

extern "C" int mz_engine_finish(mz_engine* e) {
    if (!e) return mz_fail(MZ_ERR_ARG, "mz_engine_finish: null engine");
    for (auto& kv : e->slots)
        if (!e->placed.count(kv.first)) return mz_fail(MZ_ERR_STATE, "model tensor %s was not provided", kv.first.c_str());
    if (int r = mz_sync(e->c)) return r;
    e->wstage.release();  // the staging goes once every weight is in place (Arena::finish)
    e->loaded = true;
    return MZ_OK;
}

extern "C" int mz_engine_set_trace(mz_engine* e, int on) {
    if (!e) return mz_fail(MZ_ERR_ARG, "mz_engine_set_trace: null engine");
    if (on && !e->trace) {
        if (int r = e->alloc(&e->trace, (size_t)e->dm.enc_layers * e->eg * TENC * e->dm.d)) return r;
        if (int r = e->alloc(&e->dtrace, (size_t)(e->dm.dec_layers + 1) * e->bmax * e->dm.d)) return r;
    }
    e->trace_on = on != 0;
    return MZ_OK;
}

#define TRY(expr, what)                                     \
    do {                                                    \
        if (int _r = mz_hip((expr), what)) return _r;       \
    } while (0)

// Times `expr` (one kernel launch) with a pair of events when profiling is on.
#define PROF(id, expr, what)                                                        \
    do {                                                                            \
        hipEvent_t _a = nullptr, _b = nullptr;                                      \
        if (e->prof_on) {                                                           \
            _a = e->ev();                                                           \
            _b = e->ev();                                                           \
            if (!_a || !_b) return mz_fail(MZ_ERR_HIP, "hipEventCreate failed");     \
            TRY(hipEventRecord(_a, s), "hipEventRecord");                          \
        }                                                                           \
        TRY((expr), what);                                                          \
        if (e->prof_on) {                                                           \
            TRY(hipEventRecord(_b, s), "hipEventRecord");                          \
            e->recs.push_back({(id), _a, _b});                                      \
        }                                                                           \
    } while (0)

// One encoder group of n clips into cross k/v slots slot0.. of `xkv`, on stream s with lane `lane`'s scratch and
// pinned staging (lane 0: the engine's own scratch).
static int encode_impl(mz_engine* e, const float* mels, bool on_device, int n, int slot0, int lane, hipStream_t s,
                       f16* xkv) {
    if (!e || !mels) return mz_fail(MZ_ERR_ARG, "mz_engine_encode: null argument");
    if (!e->loaded) return mz_fail(MZ_ERR_STATE, "mz_engine_encode: weights not loaded (mz_engine_finish)");
    if (n <= 0 || n > e->eg || slot0 < 0 || slot0 + n > e->bmax)
        return mz_fail(MZ_ERR_ARG, "mz_engine_encode: %d clips at slot %d (enc group %d, bmax %d)", n, slot0, e->eg, e->bmax);
    if (lane && e->trace_on) return mz_fail(MZ_ERR_STATE, "encoder trace on an extra lane");
    const EncBufs B =
        lane ? e->lanes[lane - 1] : EncBufs{e->mel, e->melT, e->h1, e->hb, e->qkvh, e->att, e->ff, e->dd, e->ex};
    const int D = e->dm.d, nm = e->dm.n_mels, nh = e->dm.nh, F = e->dm.ff, nl = e->dm.dec_layers;
    const int rows = n * TENC;
    const float* src = mels;
    if (!on_device) {
        // through this lane's pinned buffer: the host copy waits only for the lane's previous upload, and the
        // transfer itself is asynchronous (overlapping the other lane's encoder work)
        const size_t bytes = (size_t)n * nm * NFR * 4;
        if (!e->mel_pin[lane]) {
            TRY(hipHostMalloc((void**)&e->mel_pin[lane], (size_t)e->eg * nm * NFR * 4, hipHostMallocDefault),
                "hipHostMalloc (mel)");
            TRY(hipEventCreateWithFlags(&e->mel_ev[lane], hipEventDisableTiming), "hipEventCreate");
        } else {
            TRY(hipEventSynchronize(e->mel_ev[lane]), "mel staging wait");
        }
        std::memcpy(e->mel_pin[lane], mels, bytes);
        TRY(hipMemcpyAsync(B.mel, e->mel_pin[lane], bytes, hipMemcpyHostToDevice, s), "mel upload");
        TRY(hipEventRecord(e->mel_ev[lane], s), "hipEventRecord");
        src = B.mel;
    }
    PROF(MZ_K_MEL, mz_mel_transpose_launch(s, src, B.melT, n, nm), "mel transpose");
    // conv stem as implicit GEMMs (src/model.rs:552-558): GELU(conv1), GELU(conv2, stride 2) + positions
    MzGemm g{};
    g.A = B.melT;
    g.W = e->conv1.w;
    g.bias = e->conv1.b;
    g.M = n * NFR;
    g.N = D;
    g.K = e->k1pad;
    g.conv_cin = nm;
    g.conv_tin = NFR;
    g.conv_tout = NFR;
    g.conv_stride = 1;
    g.out = B.h1;
    g.ldo = D;
    PROF(MZ_K_CONV1, mz_gemm_launch(s, ALOAD_CONV, EPI_GELU_F16, g), "conv1");
    g = MzGemm{};
    g.A = B.h1;
    g.W = e->conv2.w;
    g.bias = e->conv2.b;
    g.M = rows;
    g.N = D;
    g.K = 3 * D;
    g.conv_cin = D;
    g.conv_tin = NFR;
    g.conv_tout = TENC;
    g.conv_stride = 2;
    g.out = B.ex;
    g.ldo = D;
    g.pos = e->epos;
    PROF(MZ_K_CONV2, mz_gemm_launch(s, ALOAD_CONV, EPI_GELU_POS, g), "conv2");
    PROF(MZ_K_LN, mz_layernorm_launch(s, B.ex, D, e->encv[0].ln1.w, e->encv[0].ln1.b, B.hb, D, rows, D, EPS), "ln");
    for (int i = 0; i < e->dm.enc_layers; i++) {
        const EncLayer& L = e->encv[i];
        if (e->trace_on)
            TRY(hipMemcpyAsync(e->trace + (size_t)i * e->eg * TENC * D, B.ex, (size_t)rows * D * 4,
                               hipMemcpyDeviceToDevice, s),
                "trace");
        g = MzGemm{};
        g.A = B.hb;
        g.lda = D;
        g.W = L.qkv.w;
        g.bias = L.qkv.b;
        g.M = rows;
        g.N = 3 * D;
        g.K = D;
        g.heads = B.qkvh;
        g.blocks_per_clip = 3 * nh;
        g.nh = nh;
        g.kind = 3;
        PROF(MZ_K_QKV, mz_gemm_launch(s, ALOAD_PLAIN, EPI_HEADS, g), "qkv");
        PROF(MZ_K_ATTN, mz_enc_attention_launch(s, B.qkvh, B.att, n, nh), "attention");
        g = MzGemm{};
        g.A = B.att;
        g.lda = D;
        g.W = L.o.w;
        g.bias = L.o.b;
        g.M = rows;
        g.N = D;
        g.K = D;
        g.out = B.dd;
        g.ldo = D;
        // the projection's output is rounded to fp16 once (as the reference's linear outputs) and added to the fp32
        // residual stream by the streaming add + LayerNorm, which also normalises for fc1
        PROF(MZ_K_OPROJ, mz_gemm_launch(s, ALOAD_PLAIN, EPI_F16, g), "out-proj");
        PROF(MZ_K_LN, mz_add_layernorm_launch(s, B.ex, B.dd, L.ln2.w, L.ln2.b, B.hb, rows, D, EPS), "add+ln2");
        g.A = B.hb;
        g.W = L.fc1.w;
        g.bias = L.fc1.b;
        g.N = F;
        g.out = B.ff;
        g.ldo = F;
        PROF(MZ_K_FC1, mz_gemm_launch(s, ALOAD_PLAIN, EPI_GELU_F16, g), "fc1");
        g.A = B.ff;
        g.lda = F;
        g.W = L.fc2.w;
        g.bias = L.fc2.b;
        g.N = D;
        g.K = F;
        g.out = B.dd;
        g.ldo = D;
        PROF(MZ_K_FC2, mz_gemm_launch(s, ALOAD_PLAIN, EPI_F16, g), "fc2");
        const Ln& nx = i + 1 < e->dm.enc_layers ? e->encv[i + 1].ln1 : e->eln;  // the last one is the final LN
        PROF(MZ_K_LN, mz_add_layernorm_launch(s, B.ex, B.dd, nx.w, nx.b, B.hb, rows, D, EPS), "add+ln");
    }
    // cross k/v of every decoder layer for the clips' slots (src/model.rs:614-623)
    g = MzGemm{};
    g.A = B.hb;
    g.lda = D;
    g.W = e->xkv.w;
    g.bias = e->xkv.b;
    g.M = rows;
    g.N = nl * 2 * D;
    g.K = D;
    g.heads = xkv;
    g.blocks_per_clip = nl * 2 * nh;
    g.nh = nh;
    g.kind = 2;
    g.slot0 = slot0;
    PROF(MZ_K_XKV, mz_gemm_launch(s, ALOAD_PLAIN, EPI_HEADS, g), "cross k/v");
    return MZ_OK;
}

extern "C" int mz_engine_encode(mz_engine* e, const float* mels, int n, int slot0) {
    if (!e) return mz_fail(MZ_ERR_ARG, "mz_engine_encode: null engine");
    return encode_impl(e, mels, false, n, slot0, 0, e->c->stream, e->xkvbuf);
}

extern "C" int mz_engine_encode_device(mz_engine* e, uint64_t mels, int n, int slot0) {
    if (!e) return mz_fail(MZ_ERR_ARG, "mz_engine_encode: null engine");
    return encode_impl(e, (const float*)(uintptr_t)mels, true, n, slot0, 0, e->c->stream, e->xkvbuf);
}

extern "C" int mz_engine_profile(mz_engine* e, int on) {
    if (!e) return mz_fail(MZ_ERR_ARG, "mz_engine_profile: null engine");
    if (int r = mz_sync(e->c)) return r;
    for (auto& r : e->recs) {
        e->evpool.push_back(r.a);
        e->evpool.push_back(r.b);
    }
    e->recs.clear();
    e->prof_on = on != 0;
    return MZ_OK;
}

extern "C" int mz_engine_profile_read(mz_engine* e, int id, double* total_ms, int* count) {
    if (!e || !total_ms || !count) return mz_fail(MZ_ERR_ARG, "mz_engine_profile_read: null argument");
    if (int r = mz_sync(e->c)) return r;
    double t = 0;
    int n = 0;
    for (auto& r : e->recs)
        if (r.id == id) {
            float ms = 0;
            if (int rc = mz_hip(hipEventElapsedTime(&ms, r.a, r.b), "hipEventElapsedTime")) return rc;
            t += ms;
            n++;
        }
    *total_ms = t;
    *count = n;
    return MZ_OK;
}

extern "C" int mz_engine_reset(mz_engine* e, const int32_t* prompts, int n, int prompt_len) {
    if (!e || !prompts) return mz_fail(MZ_ERR_ARG, "mz_engine_reset: null argument");
    if (n <= 0 || n > e->bmax || prompt_len <= 0 || prompt_len >= e->dm.max_t)
        return mz_fail(MZ_ERR_ARG, "mz_engine_reset: %d rows, prompt of %d", n, prompt_len);
    const int mt = e->dm.max_t;
    std::vector<int32_t> t((size_t)n * mt, 0);
    for (int b = 0; b < n; b++)
        for (int i = 0; i < prompt_len; i++) {
            int v = prompts[(size_t)b * prompt_len + i];
            if (v < 0 || v >= e->dm.vocab) return mz_fail(MZ_ERR_ARG, "prompt token %d out of range", v);
            t[(size_t)b * mt + i] = v;
        }
    std::vector<int32_t> zeros(std::max(n, 4), 0);
    if (int r = mz_upload(e->c, (uint64_t)(uintptr_t)e->tok, t.data(), t.size() * 4)) return r;
    if (int r = mz_upload(e->c, (uint64_t)(uintptr_t)e->done, zeros.data(), (size_t)n * 4)) return r;
    if (int r = mz_upload(e->c, (uint64_t)(uintptr_t)e->ctr, zeros.data(), 16)) return r;
    e->host_pos = 0;
    return MZ_OK;
}

static int take_position(mz_engine* e) {
    if (e->host_pos >= e->dm.max_t - 1)
        return mz_fail(MZ_ERR_STATE, "decoder position %d: the cache holds %d positions (reset first)", e->host_pos,
                       e->dm.max_t);
    e->host_pos++;
    return MZ_OK;
}

static int step_impl(mz_engine* e, int b, int lang, int prompt_len) {
    hipStream_t s = e->c->stream;
    const int D = e->dm.d, F = e->dm.ff, nh = e->dm.nh, nl = e->dm.dec_layers, mt = e->dm.max_t, V = e->dm.vocab;
    const long blk = (long)TPAD * HD;
    PROF(MZ_K_DEC_EMBED,
         mz_dec_embed_ln_launch(s, e->tok, e->ctr, e->emb, e->dpos, e->x, e->decv[0].ln1.w, e->decv[0].ln1.b, e->h, b,
                                D, mt, EPS),
         "embed");
    // with the trace on (eager steps only): the residual entering layer l, l = 0 .. nl (nl: after the last layer)
    const bool dtr = e->trace_on && e->dtrace && !e->capturing;
    auto dtrace = [&](int l) {
        return hipMemcpyAsync(e->dtrace + (size_t)l * e->bmax * D, e->x, (size_t)b * D * 4, hipMemcpyDeviceToDevice, s);
    };
    if (dtr) TRY(dtrace(0), "decoder trace");
    // the projection weights stay in the memory-side cache between steps when all layers' fit it with room to spare
    // (large-v3-turbo: 183 MB of 256) and the batch has two rows or more; otherwise they stream nontemporally
    const bool w_cached = (size_t)nl * (6 * (size_t)D * D + 2 * (size_t)D * F) * 2 <= ((size_t)200 << 20) && b >= 2;
    auto gemm = [&](int epi, const f16* x, int ldx, const Lin& L, int N, int K, int ks, void* out, long ldo) {
        MzDec g{};
        g.w_nt = w_cached ? 0 : 1;
        g.x = x;
        g.ldx = ldx;
        g.W = L.w;
        g.bias = L.b;
        g.M = b;
        g.N = N;
        g.K = K;
        g.ksplit = ks;
        g.out = out;
        g.ldo = ldo;
        g.ctr = e->ctr;
        return mz_dec_gemm_launch(s, epi, g);
    };
    auto attn_args = [&](const float* q, int nq, const f16* wq, const f16* qbias, const f16* k, const f16* v, long kv_b,
                         int L, const int* aslot) {
        MzDecAttn a{};
        a.q = q;
        a.nq = nq;
        a.qstride = (long)b * D;
        a.qbias = qbias;
        a.xin = wq ? e->h : nullptr;
        a.wq = wq;
        a.k = k;
        a.v = v;
        a.kv_b = kv_b;
        a.kv_h = L > 0 ? blk : (long)mt * HD;
        a.L = L;
        a.ctr = e->ctr;
        a.done = e->done;
        a.out = e->datt;
        a.B = b;
        a.nh = nh;
        a.d = D;
        a.maxT = mt;
        a.aslot = aslot;
        a.align = e->align;
        a.na = e->na;
        return a;
    };
    const int ks_dd = ksplit_for(D, D), ks_df = ksplit_for(D, F), ks_qkv = ksplit_for(3 * D, D);
    const f16* xkv = e->xkvbuf;
    for (int i = 0; i < nl; i++) {
        const DecLayer& L = e->decv[i];
        f16* kc = e->kc + (size_t)i * e->bmax * nh * mt * HD;
        f16* vc = e->vc + (size_t)i * e->bmax * nh * mt * HD;
        // q/k/v as split-K partials; the self-attention sums them for its (row, head), adds the bias and writes the
        // step's key and value into the cache
        PROF(MZ_K_DEC_QKV, gemm(DEPI_PARTIAL, e->h, D, L.qkv, 3 * D, D, ks_qkv, e->part, 3 * D), "dec qkv");
        {
            MzDecAttn a = attn_args(e->part, ks_qkv, nullptr, L.qkv.b, kc, vc, (long)nh * mt * HD, -1, nullptr);
            a.qstride = (long)b * 3 * D;
            a.qrow = 3 * D;
            a.kw = kc;
            a.vw = vc;
            a.kvbias = L.qkv.b + D;
            PROF(MZ_K_DEC_SELF, mz_dec_attn_launch(s, a), "self attention");
        }
        PROF(MZ_K_DEC_OPROJ, gemm(DEPI_PARTIAL, e->datt, D, L.o, D, D, ks_dd, e->part, D), "dec out-proj");
        PROF(MZ_K_DEC_ADDLN,
             mz_dec_add_ln_launch(s, e->x, e->x, e->part, ks_dd, (long)b * D, L.o.b, L.lnx.w, L.lnx.b, e->h, b, D,
                                  EPS),
             "add+ln");
        // the cross-attention projects its own query from the layer-norm output
        {
            MzDecCross c{};
            c.xin = e->h;
            c.wq = L.xq.w;
            c.qbias = L.xq.b;
            c.k = xkv + (size_t)(2 * i) * nh * blk;
            c.v = xkv + (size_t)(2 * i + 1) * nh * blk;
            c.kv_b = (long)nl * 2 * nh * blk;
            c.kv_h = blk;
            c.ctr = e->ctr;
            c.done = e->done;
            c.out = e->datt;
            c.B = b;
            c.nh = nh;
            c.d = D;
            c.maxT = mt;
            c.aslot = e->aslot + (size_t)i * nh;
            c.align = e->align;
            c.alignh = e->alignh;
            c.na = e->na;
            PROF(MZ_K_DEC_CROSS, mz_dec_cross_launch(s, c), "cross attention");
        }
        PROF(MZ_K_DEC_XO, gemm(DEPI_PARTIAL, e->datt, D, L.xo, D, D, ks_dd, e->part, D), "dec cross out-proj");
        PROF(MZ_K_DEC_ADDLN,
             mz_dec_add_ln_launch(s, e->x, e->x, e->part, ks_dd, (long)b * D, L.xo.b, L.ln3.w, L.ln3.b, e->h, b, D,
                                  EPS),
             "add+ln");
        PROF(MZ_K_DEC_FC1, gemm(DEPI_GELU_F16, e->h, D, L.fc1, F, D, 1, e->dff, F), "dec fc1");
        PROF(MZ_K_DEC_FC2, gemm(DEPI_PARTIAL, e->dff, F, L.fc2, D, F, ks_df, e->part, D), "dec fc2");
        const Ln& nx = i + 1 < nl ? e->decv[i + 1].ln1 : e->dln;
        PROF(MZ_K_DEC_ADDLN,
             mz_dec_add_ln_launch(s, e->x, e->x, e->part, ks_df, (long)b * D, L.fc2.b, nx.w, nx.b, e->h, b, D, EPS),
             "add+ln");
        if (dtr) TRY(dtrace(i + 1), "decoder trace");
    }
    // tied LM head with the masked per-workgroup argmax, then the greedy choice, which advances the position
    {
        MzDec g{};
        g.x = e->h;
        g.ldx = D;
        g.W = e->emb;
        g.M = b;
        g.N = V;
        g.K = D;
        g.ksplit = 1;
        g.out = e->logits;
        g.ldo = V;
        g.ctr = e->ctr;
        g.sup = lang ? e->sup_lang : e->sup;
        g.bs1 = lang ? -1 : e->bs1;
        g.bs2 = lang ? -1 : e->bs2;
        g.prompt_len = prompt_len;
        g.amax = e->amax;
        PROF(MZ_K_DEC_LM, mz_dec_gemm_launch(s, DEPI_LOGITS, g), "lm head");
    }
    PROF(MZ_K_DEC_ARGMAX,
         mz_dec_argmax_launch(s, e->amax, mz_lm_blocks(V), e->tok, e->done, e->ctr, b, mt, prompt_len, e->eos),
         "argmax");
    return MZ_OK;
}

extern "C" int mz_engine_step(mz_engine* e, int b, int lang, int prompt_len) {
    if (!e) return mz_fail(MZ_ERR_ARG, "mz_engine_step: null engine");
    if (!e->loaded) return mz_fail(MZ_ERR_STATE, "mz_engine_step: weights not loaded");
    if (b <= 0 || b > e->bmax) return mz_fail(MZ_ERR_ARG, "mz_engine_step: %d rows (bmax %d)", b, e->bmax);
    if (int r = take_position(e)) return r;
    return step_impl(e, b, lang, prompt_len);
}

extern "C" int mz_engine_detect(mz_engine* e, int b, int32_t* langs) {
    if (!e || !langs) return mz_fail(MZ_ERR_ARG, "mz_engine_detect: null argument");
    if (int r = mz_engine_step(e, b, 1, 1)) return r;
    const int mt = e->dm.max_t;
    std::vector<int32_t> t((size_t)b * mt);
    if (int r = mz_download(e->c, t.data(), (uint64_t)(uintptr_t)e->tok, t.size() * 4)) return r;
    for (int i = 0; i < b; i++) langs[i] = t[(size_t)i * mt + 1];
    return MZ_OK;
}

extern "C" int mz_engine_capture(mz_engine* e, int b, int prompt_len) {
    if (!e) return mz_fail(MZ_ERR_ARG, "mz_engine_capture: null engine");
    if (!e->loaded) return mz_fail(MZ_ERR_STATE, "mz_engine_capture: weights not loaded");
    if (b <= 0 || b > e->bmax) return mz_fail(MZ_ERR_ARG, "mz_engine_capture: %d rows", b);
    if (e->graph) {
        mz_graph_free(e->graph);
        e->graph = nullptr;
    }
    if (int r = mz_graph_begin(e->c)) return r;
    const bool prof = e->prof_on;
    e->prof_on = false;  // events are not recorded into the graph
    e->capturing = true;
    int rs = step_impl(e, b, 0, prompt_len);
    e->capturing = false;
    e->prof_on = prof;
    mz_graph* g = nullptr;
    int re = mz_graph_end(e->c, &g);
    if (rs) {
        mz_graph_free(g);
        return rs;
    }
    if (re) return re;
    e->graph = g;
    e->graph_b = b;
    e->graph_np = prompt_len;
    return MZ_OK;
}

extern "C" int mz_engine_replay(mz_engine* e) {
    if (!e || !e->graph) return mz_fail(MZ_ERR_STATE, "mz_engine_replay: no captured step");
    if (int r = take_position(e)) return r;
    hipStream_t s = e->c->stream;
    PROF(MZ_K_STEP, mz_graph_launch(e->c, e->graph) ? hipErrorUnknown : hipSuccess, "hipGraphLaunch");
    return MZ_OK;
}

extern "C" int mz_engine_buffer(mz_engine* e, int which, uint64_t* dptr, size_t* bytes) {
    if (!e || !dptr || !bytes) return mz_fail(MZ_ERR_ARG, "mz_engine_buffer: null argument");
    const size_t D = e->dm.d, B = e->bmax, mt = e->dm.max_t, G = e->eg;
    void* p = nullptr;
    size_t n = 0;
    switch (which) {
        case MZ_BUF_TOK: p = e->tok, n = B * mt * 4; break;
        case MZ_BUF_DONE: p = e->done, n = B * 4; break;
        case MZ_BUF_CTR: p = e->ctr, n = 16; break;
        case MZ_BUF_ALIGN: p = e->align, n = B * mt * e->na * TENC * 4; break;
        case MZ_BUF_ALIGN_H: p = e->alignh, n = B * mt * e->na * TENC * 2; break;
        case MZ_BUF_ENC_OUT: p = e->hb, n = G * TENC * D * 2; break;
        case MZ_BUF_LOGITS: p = e->logits, n = B * e->dm.vocab * 4; break;
        case MZ_BUF_TRACE:
            if (!e->trace) return mz_fail(MZ_ERR_STATE, "trace not enabled");
            p = e->trace, n = (size_t)e->dm.enc_layers * G * TENC * D * 4;
            break;
        case MZ_BUF_XKV: p = e->xkvbuf, n = xkv_elems(e->dm, e->bmax) * 2; break;
        case MZ_BUF_DEC_X: p = e->x, n = B * D * 4; break;
        case MZ_BUF_ENC_X: p = e->ex, n = G * TENC * D * 4; break;
        case MZ_BUF_DEC_TRACE:
            if (!e->dtrace) return mz_fail(MZ_ERR_STATE, "trace not enabled");
            p = e->dtrace, n = (size_t)(e->dm.dec_layers + 1) * B * D * 4;
            break;
        case MZ_BUF_SELF_K: p = e->kc, n = (size_t)e->dm.dec_layers * B * e->dm.nh * e->dm.max_t * HD * 2; break;
        case MZ_BUF_SELF_V: p = e->vc, n = (size_t)e->dm.dec_layers * B * e->dm.nh * e->dm.max_t * HD * 2; break;
        default: return mz_fail(MZ_ERR_ARG, "unknown engine buffer %d", which);
    }
    *dptr = (uint64_t)(uintptr_t)p;
    *bytes = n;
    return MZ_OK;
}

extern "C" int mz_engine_read(mz_engine* e, int which, void* dst, size_t offset, size_t bytes) {
    uint64_t p;
    size_t n;
    if (int r = mz_engine_buffer(e, which, &p, &n)) return r;
    if (offset + bytes > n) return mz_fail(MZ_ERR_ARG, "mz_engine_read: %zu bytes at %zu of %zu", bytes, offset, n);
    return mz_download(e->c, dst, p + offset, bytes);
}

extern "C" int mz_engine_free(mz_engine* e) {
    if (!e) return MZ_OK;
    if (e->graph) mz_graph_free(e->graph);
    hipStreamSynchronize(e->c->stream);
    if (e->enc_done) hipEventDestroy(e->enc_done);
    if (e->done_ev) hipEventDestroy(e->done_ev);
    if (e->done_pin) hipHostFree(e->done_pin);
    for (auto& r : e->recs) {
        hipEventDestroy(r.a);
        hipEventDestroy(r.b);
    }
    for (hipEvent_t x : e->evpool) hipEventDestroy(x);
    e->wstage.release();
    for (int k = 0; k < MZ_ENC_LANES; k++) {
        if (e->mel_ev[k]) {
            hipEventSynchronize(e->mel_ev[k]);
            hipEventDestroy(e->mel_ev[k]);
        }
        if (e->mel_pin[k]) hipHostFree(e->mel_pin[k]);
    }
    if (e->fork) hipEventDestroy(e->fork);
    for (int k = 0; k < MZ_ENC_LANES - 1; k++) {
        if (e->ls[k]) {
            hipStreamSynchronize(e->ls[k]);
            hipStreamDestroy(e->ls[k]);
        }
        if (e->join[k]) hipEventDestroy(e->join[k]);
        const EncBufs& l = e->lanes[k];
        for (void* p : {(void*)l.mel, (void*)l.melT, (void*)l.h1, (void*)l.hb, (void*)l.qkvh, (void*)l.att, (void*)l.ff,
                        (void*)l.dd, (void*)l.ex})
            if (p) mz_free(e->c, (uint64_t)(uintptr_t)p);
    }
    for (void* p : {(void*)e->ts_rc, (void*)e->ts_mean, (void*)e->ts_sd, (void*)e->ts_cost, (void*)e->ts_trace,
                    (void*)e->ts_out})
        if (p) mz_free(e->c, (uint64_t)(uintptr_t)p);
    for (void* p : {(void*)e->arena, (void*)e->mel, (void*)e->melT, (void*)e->h1, (void*)e->ex, (void*)e->hb, (void*)e->dd,
                    (void*)e->qkvh, (void*)e->att, (void*)e->ff, (void*)e->trace, (void*)e->dtrace, (void*)e->xkvbuf, (void*)e->tok,
                    (void*)e->done, (void*)e->ctr, (void*)e->x, (void*)e->h, (void*)e->datt,
                    (void*)e->dff, (void*)e->kc, (void*)e->vc, (void*)e->logits, (void*)e->align, (void*)e->alignh, (void*)e->amax,
                    (void*)e->aslot, (void*)e->sup, (void*)e->sup_lang,
                    (void*)e->part})
        if (p) mz_free(e->c, (uint64_t)(uintptr_t)p);
    delete e;
    return MZ_OK;
}

// ------------------------------------------------------------------ batch transcription (src/transcribe.rs:104-167)

using clk = std::chrono::steady_clock;
static double since(clk::time_point a) { return std::chrono::duration<double>(clk::now() - a).count(); }

// Enqueues the encoder of a chunk of n clips and returns (the first half of transcribe, src/transcribe.rs:107-116):
// its groups go round-robin over the encoder lanes (the main stream and the engine's other streams, each with its
// own scratch), and one event marks them all done. One chunk at a time: collect it before submitting the next.
static int submit_impl(mz_engine* e, const float* mels, bool on_device, int n) {
    if (!e || !mels) return mz_fail(MZ_ERR_ARG, "mz_transcribe_submit: null argument");
    if (!e->loaded) return mz_fail(MZ_ERR_STATE, "mz_transcribe_submit: weights not loaded (mz_engine_finish)");
    if (n <= 0 || n > e->bmax) return mz_fail(MZ_ERR_ARG, "mz_transcribe_submit: %d clips (bmax %d)", n, e->bmax);
    if (e->pending_n) return mz_fail(MZ_ERR_STATE, "mz_transcribe_submit: a chunk is pending; collect it first");
    const auto t0 = clk::now();
    const int nm = e->dm.n_mels, ngroups = (n + e->eg - 1) / e->eg;
    const int nlanes = e->trace_on ? 1 : std::min(ngroups, MZ_ENC_LANES);
    hipStream_t st[MZ_ENC_LANES];  // lane 0: the engine's stream; lane k: its own stream ls[k - 1]
    st[0] = e->c->stream;
    for (int k = 1; k < MZ_ENC_LANES; k++) st[k] = e->ls[k - 1];
    if (nlanes > 1) {
        TRY(hipEventRecord(e->fork, st[0]), "hipEventRecord");
        for (int k = 1; k < nlanes; k++) TRY(hipStreamWaitEvent(st[k], e->fork, 0), "hipStreamWaitEvent");
    }
    for (int g0 = 0, gi = 0; g0 < n; g0 += e->eg, gi++) {
        const int gn = std::min(e->eg, n - g0), k = gi % nlanes;
        if (int r = encode_impl(e, mels + (size_t)g0 * nm * NFR, on_device, gn, g0, k, st[k], e->xkvbuf)) return r;
    }
    for (int k = 1; k < nlanes; k++) {
        TRY(hipEventRecord(e->join[k - 1], st[k]), "hipEventRecord");
        TRY(hipStreamWaitEvent(st[0], e->join[k - 1], 0), "hipStreamWaitEvent");
    }
    TRY(hipEventRecord(e->enc_done, st[0]), "hipEventRecord");
    e->pending_n = n;
    e->pending_enq = since(t0);
    return MZ_OK;
}

static int check_frames(const int32_t* frames, int n, const char* who) {
    for (int c = 0; c < n; c++)
        if (frames[c] < 0 || frames[c] > NFR)
            return mz_fail(MZ_ERR_ARG, "%s: clip %d has %d frames (0..%d)", who, c, frames[c], NFR);
    return MZ_OK;
}

// Decodes the oldest submitted chunk and computes its token timestamps (the rest of transcribe,
// src/transcribe.rs:118-167). times->enc is the host's enqueue time at submission plus its wait here for the encoder.
static int collect_impl(mz_engine* e, const int32_t* frames, int n, const int32_t* prompt, int prompt_len, int detect,
                        int use_graph, int max_new, int half_align, int32_t* seq, int32_t* seq_len, float* ts,
                        int32_t* langs, mz_times* times) {
    if (!e || !frames || !prompt || !seq || !seq_len || !ts || !langs)
        return mz_fail(MZ_ERR_ARG, "mz_transcribe_collect: null argument");
    if (!e->pending_n) return mz_fail(MZ_ERR_STATE, "mz_transcribe_collect: no chunk submitted");
    if (n != e->pending_n)
        return mz_fail(MZ_ERR_ARG, "mz_transcribe_collect: %d clips, the submitted chunk has %d", n, e->pending_n);
    if (prompt_len <= 0 || prompt_len >= e->dm.max_t)
        return mz_fail(MZ_ERR_ARG, "mz_transcribe_collect: prompt of %d", prompt_len);
    if (int r = check_frames(frames, n, "mz_transcribe_collect")) return r;
    e->pending_n = 0;
    const int mt = e->dm.max_t, eos = e->eos, np = prompt_len;
    auto sec = since;
    mz_times tm{};

    auto t0 = clk::now();
    TRY(hipEventSynchronize(e->enc_done), "encoder wait");
    tm.enc = e->pending_enq + sec(t0);

    t0 = clk::now();
    std::vector<int32_t> pr((size_t)n * np);
    for (int b = 0; b < n; b++)
        for (int i = 0; i < np; i++) pr[(size_t)b * np + i] = prompt[i];
    if (int r = mz_engine_reset(e, pr.data(), n, np)) return r;
    std::vector<int32_t> lg(n, np > 1 ? prompt[1] : -1);
    int steps = 0;
    if (detect) {
        if (int r = mz_engine_detect(e, n, lg.data())) return r;
        steps = 1;
    }
    const int limit = max_new > 0 ? std::min(mt - 1, np - 1 + max_new) : mt - 1;
    if (use_graph) {
        if (!e->graph || e->graph_b != n || e->graph_np != np)
            if (int r = mz_engine_capture(e, n, np)) return r;
    }
    // Every 8 steps the loop ends if every row is done. The flags it reads were copied (asynchronously, into pinned
    // memory) DONE_LAG steps earlier, so the steps enqueued since keep the device busy while the host waits for
    // the copy and tests it: the queue never drains. A batch that finishes runs at most 8 + DONE_LAG - 1 steps
    // more than it needs (finished rows skip their attention and keep eos).
    constexpr int DONE_LAG = 2;
    bool copied = false;
    while (steps < limit) {
        if (int r = use_graph ? mz_engine_replay(e) : mz_engine_step(e, n, 0, np)) return r;
        steps++;
        if (steps + DONE_LAG >= np && (steps + DONE_LAG) % 8 == 0) {
            TRY(hipMemcpyAsync(e->done_pin, e->done, (size_t)n * 4, hipMemcpyDeviceToHost, e->c->stream), "done flags");
            TRY(hipEventRecord(e->done_ev, e->c->stream), "hipEventRecord");
            copied = true;
        }
        if (copied && steps % 8 == 0) {
            TRY(hipEventSynchronize(e->done_ev), "done flags wait");
            copied = false;
            if (std::all_of(e->done_pin, e->done_pin + n, [](int v) { return v != 0; })) break;
        }
    }
    if (int r = mz_sync(e->c)) return r;
    tm.dec = sec(t0);
    tm.steps = steps;

    t0 = clk::now();
    std::vector<int32_t> toks((size_t)n * mt);
    if (int r = mz_download(e->c, toks.data(), (uint64_t)(uintptr_t)e->tok, toks.size() * 4)) return r;
    const size_t row = (size_t)e->na * TENC;
    // sequence lengths; the token rows of clip c are the positions np .. n_seq - 2 (the last token is eos or the
    // step limit) and their alignment rows start at align[c][np]
    std::vector<int> nseq(n), nrows(n);
    std::vector<int2> rc(n);
    int rmax = 0;
    for (int c = 0; c < n; c++) {
        const int32_t* t = &toks[(size_t)c * mt];
        int n_seq = std::min(steps + 1, mt);
        for (int k = np; k < mt; k++)
            if (t[k] == eos) {
                n_seq = std::min(k + 1, mt);
                break;
            }
        n_seq = std::min(n_seq, steps + 1);
        nseq[c] = n_seq;
        nrows[c] = std::max(n_seq - 1 - np, 0);
        rc[c] = int2{nrows[c], frames[c] / 2};
        rmax = std::max(rmax, nrows[c]);
    }
    // token timestamps on the device (median filter + DTW per clip, k_align.hip); only the times come back
    std::vector<float> jt((size_t)n * mt);
    if (rmax > 0) {
        TRY(hipMemcpyAsync(e->ts_rc, rc.data(), (size_t)n * sizeof(int2), hipMemcpyHostToDevice, e->c->stream),
            "upload");
        MzTs p{};
        p.w = e->align + (size_t)np * row;
        p.clip_stride = (long)mt * row;
        p.heads = e->na;
        p.cols_full = TENC;
        p.width = 7;
        p.half = half_align;
        p.rmax = rmax;
        p.rc = e->ts_rc;
        p.mean = e->ts_mean;
        p.sd = e->ts_sd;
        p.cost = e->ts_cost;
        p.trace = e->ts_trace;
        p.diag_stride = mz_ts_diag_stride(rmax, TENC);
        p.ldd = mz_ts_ldd(rmax);
        p.out = e->ts_out;
        p.out_stride = mt;
        TRY(mz_ts_launch(e->c->stream, p, n), "timestamp kernels");
        TRY(hipMemcpyAsync(jt.data(), e->ts_out, jt.size() * 4, hipMemcpyDeviceToHost, e->c->stream),
            "timestamp download");
        if (int r = mz_sync(e->c)) return r;
    }
    for (int c = 0; c < n; c++) {
        const int32_t* t = &toks[(size_t)c * mt];
        const int n_seq = nseq[c];
        for (int k = 0; k < mt; k++) seq[(size_t)c * mt + k] = k < n_seq ? t[k] : 0;
        seq_len[c] = n_seq;
        float* tc = ts + (size_t)c * mt;
        std::fill(tc, tc + mt, 0.f);
        const int rows = nrows[c];
        if (rows > 0) {
            const float* j = &jt[(size_t)c * mt];
            for (int k = 0; k < rows; k++) tc[np + k] = j[k];
            tc[n_seq - 1] = j[rows - 1];
        }
        langs[c] = lg[c];
    }
    tm.post = sec(t0);
    if (times) *times = tm;
    return MZ_OK;
}

static int transcribe_impl(mz_engine* e, const float* mels, bool on_device, const int32_t* frames, int n,
                           const int32_t* prompt, int prompt_len, int detect, int use_graph, int max_new,
                           int half_align, int32_t* seq, int32_t* seq_len, float* ts, int32_t* langs,
                           mz_times* times) {
    if (!e || !mels || !frames || !prompt || !seq || !seq_len || !ts || !langs)
        return mz_fail(MZ_ERR_ARG, "mz_transcribe: null argument");
    if (e->pending_n) return mz_fail(MZ_ERR_STATE, "mz_transcribe: a submitted chunk is not collected");
    if (n <= 0 || n > e->bmax) return mz_fail(MZ_ERR_ARG, "mz_transcribe: %d clips (bmax %d)", n, e->bmax);
    if (prompt_len <= 0 || prompt_len >= e->dm.max_t)
        return mz_fail(MZ_ERR_ARG, "mz_transcribe: prompt of %d", prompt_len);
    if (int r = check_frames(frames, n, "mz_transcribe")) return r;
    if (int r = submit_impl(e, mels, on_device, n)) return r;
    return collect_impl(e, frames, n, prompt, prompt_len, detect, use_graph, max_new, half_align, seq, seq_len, ts,
                        langs, times);
}

extern "C" int mz_transcribe_submit(mz_engine* e, const float* mels, int n) {
    return submit_impl(e, mels, false, n);
}

extern "C" int mz_transcribe_submit_device(mz_engine* e, uint64_t mels, int n) {
    return submit_impl(e, (const float*)(uintptr_t)mels, true, n);
}

extern "C" int mz_transcribe_collect(mz_engine* e, const int32_t* frames, int n, const int32_t* prompt,
                                     int prompt_len, int detect, int use_graph, int max_new, int half_align,
                                     int32_t* seq, int32_t* seq_len, float* ts, int32_t* langs, mz_times* times) {
    return collect_impl(e, frames, n, prompt, prompt_len, detect, use_graph, max_new, half_align, seq, seq_len, ts,
                        langs, times);
}

extern "C" int mz_transcribe(mz_engine* e, const float* mels, const int32_t* frames, int n, const int32_t* prompt,
                             int prompt_len, int detect, int use_graph, int max_new, int half_align, int32_t* seq,
                             int32_t* seq_len, float* ts, int32_t* langs, mz_times* times) {
    return transcribe_impl(e, mels, false, frames, n, prompt, prompt_len, detect, use_graph, max_new, half_align, seq,
                           seq_len, ts, langs, times);
}

extern "C" int mz_transcribe_device(mz_engine* e, uint64_t mels, const int32_t* frames, int n, const int32_t* prompt,
                                    int prompt_len, int detect, int use_graph, int max_new, int half_align,
                                    int32_t* seq, int32_t* seq_len, float* ts, int32_t* langs, mz_times* times) {
    return transcribe_impl(e, (const float*)(uintptr_t)mels, true, frames, n, prompt, prompt_len, detect, use_graph,
                           max_new, half_align, seq, seq_len, ts, langs, times);
}
