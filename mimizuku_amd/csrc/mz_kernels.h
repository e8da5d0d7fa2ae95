// Host-side launchers of the gfx950 kernels (internal to libmimizuku_amd; the C ABI is include/mimizuku.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

typedef _Float16 f16;

// ---------------------------------------------------------------- tiled MFMA GEMM (encoder sizes)
// C[m][n] = sum_k A[m][k] W[n][k] (+ bias[n]), fp16 operands, fp32 accumulation, K a multiple of 64.
enum MzALoad { ALOAD_PLAIN = 0, ALOAD_CONV = 1 };
enum MzEpi {
    EPI_F16 = 0,        // out f16 [M][ldo] = acc + bias
    EPI_GELU_F16 = 1,   // out f16 [M][ldo] = gelu(acc + bias)
    EPI_RESID_F32 = 2,  // out f32 [M][ldo] += acc + bias        (residual add fused into the producing GEMM)
    EPI_GELU_POS = 3,   // out f32 [M][ldo] = gelu(acc + bias) + pos[m % 1500][n]   (conv2 -> residual stream)
    EPI_HEADS = 4,      // head-major scatter into [1536][64] tiles (encoder v transposed [64][1536])
};

struct MzGemm {
    const f16* A;
    long lda;
    const f16* W;  // [N][K] row-major
    const f16* bias;  // [N] or null
    int M, N, K;
    // ALOAD_CONV: A[g * tout + t][tap * cin + ci] = src[(g * tin + stride * t + tap - 1) * cin + ci], zero outside
    int conv_cin, conv_tin, conv_tout, conv_stride;
    // epilogues
    void* out;
    long ldo;
    const f16* pos;
    // EPI_HEADS: column n belongs to 64-wide block blk = n / 64 and row m = g * 1500 + t to clip g; the block's
    // 1536 x 64 tile lives at heads + ((slot0 + g) * blocks_per_clip + blk) * 1536 * 64. kind 3: blocks ordered
    // [q|k|v][head] (encoder self-attention; q stored multiplied by log2(e) / 8, the attention's exponent scale, and
    // v transposed [64][1536] for the P.V matrix product), kind 2: [layer][k|v][head] (decoder cross-attention;
    // every tile row-major [1536][64]).
    f16* heads;
    int blocks_per_clip, nh, kind, slot0;
};
hipError_t mz_gemm_launch(hipStream_t s, int aload, int epi, const MzGemm& g);

// ---------------------------------------------------------------- encoder attention
// qkvh: [G][3][nh] tiles of 1536 x 64 halves (q, k row-major [t][64]; v transposed [64][t]; t >= 1500 zero);
// out: [G * 1500][nh * 64]
hipError_t mz_enc_attention_launch(hipStream_t s, const f16* qkvh, f16* out, int G, int nh);

// ---------------------------------------------------------------- norms and small encoder kernels
// y[r] = LN(x[r]) (fp32 in, fp16 out), rows of dim (dim % 128 == 0, dim <= 2048)
hipError_t mz_layernorm_launch(hipStream_t s, const float* x, long ldx, const f16* w, const f16* b, f16* y, long ldy,
                               int rows, int dim, float eps);
// x[r] += d[r] (f16), then y[r] = LN(x[r])
hipError_t mz_add_layernorm_launch(hipStream_t s, float* x, const f16* d, const f16* w, const f16* b, f16* y, int rows,
                                   int dim, float eps);
// mel f32 [G][nm][3000] -> melT f16 [G][3000][nm]
hipError_t mz_mel_transpose_launch(hipStream_t s, const float* mel, f16* melT, int G, int nm);

// ---------------------------------------------------------------- decoder step
// Position: ctr[0] = position of the next step; the step's first kernel (embed) copies it to ctr[1], the later
// kernels read ctr[1], the last one (argmax) writes ctr[0] = ctr[1] + 1.
#define MZ_MAX_PARTS 16  // split-K partials summed by dec_add_ln
#define MZ_DEC_KSLICE 1280  // largest K slice of one skinny-GEMM workgroup (both operands resident in 160 KB of LDS)

// skinny GEMM for decode batches: rows m < M of x (f16, row stride ldx % 8 == 0, M <= 32 per m-tile) times W[N][K];
// K / ksplit <= MZ_DEC_KSLICE
enum MzDecEpi {
    DEPI_PARTIAL = 0,  // part[ks][m][n] (f32), ks = blockIdx.y (split-K)
    DEPI_GELU_F16 = 1, // out f16 [m][ldo] = gelu(acc + bias)
    DEPI_LOGITS = 2,   // out f32 [m][ldo] = acc, and amax[wg][m] = masked (max, lowest id) of each workgroup's ids
                       // (mz_lm_blocks(N) workgroups per 32-row block; K <= MZ_DEC_KSLICE)
    DEPI_F16 = 4,      // out f16 [m][ldo] = acc + bias
};
struct MzDec {
    const f16* x;
    long ldx;
    const f16* W;
    const f16* bias;
    int M, N, K, ksplit;
    void* out;
    long ldo;
    const int* ctr;
    // DEPI_LOGITS: mask (nonzero = never chosen), begin-suppressed ids at the first generated position, partials
    const unsigned char* sup;
    int bs1, bs2, prompt_len;
    void* amax;  // int2 {float bits, id} [mz_lm_blocks(N)][M]
    int w_nt;    // projections: W read nontemporally (1) or with the default policy (0); the LM head always streams
};
hipError_t mz_dec_gemm_launch(hipStream_t s, int epi, const MzDec& g);
// LM head workgroups (each with one argmax partial per row) and vocabulary tiles of 16 per workgroup
int mz_lm_blocks(int N);
int mz_lm_tiles_per_block(int N);

struct MzDecAttn {
    // query: sum over nq slices of q[s * qstride + b * qrow + head * 64 + i] (+ qbias), scaled by 1/8 (qrow 0: d);
    // or, when wq is set, the projection xin[b] . wq[head * 64 + i] (+ qbias) computed in the kernel
    // (d <= MZ_DEC_KSLICE)
    const float* q;
    int nq;
    long qstride, qrow;
    const f16* qbias;
    // self-attention only, when kw is set: the slices also hold the step's key and value at columns d + head * 64 + i
    // and 2d + head * 64 + i of each row; summed with kvbias (k then v, [2d]), rounded to fp16, they are written to
    // the caches kw / vw (laid out as k / v) at the step's position and stand in for that position's key and value
    f16* kw;
    f16* vw;
    const f16* kvbias;
    const f16* xin;  // [B][d]
    const f16* wq;   // [d][d], row = output feature
    // keys and values of (b, head): rows of 64 halves at k + b * kv_b + head * kv_h (v likewise)
    const f16* k;
    const f16* v;
    long kv_b, kv_h;
    int L;             // keys (cross, <= 1536) or -1: position + 1 (self)
    const int* ctr;
    const int* done;
    f16* out;          // [B][d]
    int B, nh, d;
    int maxT;
    // alignment-head capture (cross only, may be null): slot of each head of this layer or -1
    const int* aslot;
    float* align;      // [bmax][maxT][na][1500]
    f16* alignh;       // the same rows rounded to fp16 (may be null)
    int na;
};
hipError_t mz_dec_attn_launch(hipStream_t s, const MzDecAttn& a);

// Cross-attention of one query per (row, head) over the encoder's 1500 keys with its own query projection
// (kernels/whisper.cu:355-449, 309-317): q = wq[head rows] . xin[b] + qbias, xin the row's LayerNorm output. The keys
// and values of (b, head) are 1500 rows of 64 halves at k + b * kv_b + head * kv_h (v likewise). Batches of at most
// 256 / nh rows run a variant that keeps more of each workgroup's stream in flight; both give the same bits.
struct MzDecCross {
    const f16* xin;  // [B][d]
    const f16* wq;   // [d][d], row = output feature
    const f16* qbias;
    const f16* k;
    const f16* v;
    long kv_b, kv_h;
    const int* ctr;
    const int* done;
    f16* out;        // [B][d]
    int B, nh, d, maxT;
    const int* aslot;  // alignment slot of each head of this layer or -1 (may be null)
    float* align;      // [bmax][maxT][na][1500]
    f16* alignh;       // the same rows rounded to fp16 (may be null)
    int na;
};
hipError_t mz_dec_cross_launch(hipStream_t s, const MzDecCross& a);

// x[b] = xin[b] + sum_s parts[s][b] + bias; y[b] = LN(x[b])  (the residual add fused with the next layer norm;
// xin may be x)
hipError_t mz_dec_add_ln_launch(hipStream_t s, const float* xin, float* x, const float* parts, int nparts,
                                long part_stride, const f16* bias, const f16* w, const f16* b, f16* y, int rows,
                                int dim, float eps);
// ctr[1] = ctr[0]; x[b] = emb[tok[b * maxT + p]] + pe[p] (fp32); y[b] = LN(x[b])
hipError_t mz_dec_embed_ln_launch(hipStream_t s, const int* tok, int* ctr, const f16* emb, const f16* pe, float* x,
                                  const f16* w, const f16* b, f16* y, int rows, int dim, int maxT, float eps);
// greedy choice of token p + 1 (kernels/whisper.cu:451-493 semantics) from the LM head partials; ctr[0] = p + 1
hipError_t mz_dec_argmax_launch(hipStream_t s, const int2* amax, int nblk, int* tok, int* done, int* ctr, int B,
                                int maxT, int prompt_len, int eos);

// ---------------------------------------------------------------- token timestamps
// Alignment rows of clip c: w + c * clip_stride floats, rc[c].x rows of heads x cols_full floats, of which the first
// rc[c].y columns are used. Scratch per clip: mean and sd [heads][cols_full]; cost (f32) and trace (i8) in
// anti-diagonal-major order [rmax + cols_full + 1][ldd], ldd = mz_ts_ldd(rmax), diag_stride elements apart.
#define MZ_TS_MAX_WIDTH 15
struct MzTs {
    const float* w;
    long clip_stride;
    int heads, cols_full, width, half, rmax;
    const int2* rc;
    float* mean;
    float* sd;
    float* cost;
    signed char* trace;
    long diag_stride;
    int ldd;
    float* out;  // out[c * out_stride + k], k < rc[c].x: start time in seconds of row k's token
    long out_stride;
};
// floats per diagonal: rows 0 .. rmax rounded up to a multiple of 4, so every diagonal starts 16-byte aligned and a
// 4-row group never straddles two diagonals
inline int mz_ts_ldd(int rmax) { return (rmax + 4) & ~3; }
// scratch elements per clip for cost / trace
inline long mz_ts_diag_stride(int rmax, int cols_full) { return (long)(rmax + cols_full + 1) * mz_ts_ldd(rmax); }
hipError_t mz_ts_launch(hipStream_t s, const MzTs& p, int n);
// the static scratch of mz_jump_times_device_noalloc (64 MiB per device) and the clips it takes per pass
#define MZ_TS_SCRATCH_BYTES (64u << 20)
#define MZ_TS_NOALLOC_CHUNK 64
// looks up that scratch's address on `device` (which must be current) once; mz_init calls it
int mz_ts_scratch_setup(int device);

// ---------------------------------------------------------------- log-mel features (Mel::features, src/audio.rs)
#define MZ_MEL_NFFT 400
#define MZ_MEL_HOP 160
#define MZ_MEL_BINS 201          // MZ_MEL_NFFT / 2 + 1
#define MZ_MEL_NSAMPLES 480000   // 30 s at 16 kHz
#define MZ_NFR_HOST 3000         // log-mel frames of 30 s
// audio [n][480000] f32 (samples at or past ns[c] read as zero), tables from mz_mel_tables (cosb / sinb
// [400][201] windowed DFT basis, filt [201][n_mels]); pow [n][3000][201] and mx [n] are scratch;
// mel [n][n_mels][3000] the normalised log-mel
struct MzMel {
    const float* audio;
    const int* ns;
    const double* cosb;
    const double* sinb;
    const float* filt;
    float* pow;
    float* mx;
    float* mel;
    int n, n_mels;
};
hipError_t mz_log_mel_launch(hipStream_t s, const MzMel& p);
