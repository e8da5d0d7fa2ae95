// Decoder-step kernels: one greedy step for B rows (kernels/whisper.cu:301-567). The step is HBM-bound, and every
// kernel here is written to keep its whole operand stream in flight at once and to need no communication between
// workgroups of one launch: on a part with one L2 per XCD, a device-scope fence costs an L2 write-back, so the
// split-key attention of the reference (three kernels) and any last-block combine are replaced by one workgroup per
// (row, head) that merges its own partial softmaxes in LDS.
//
// Position: ctr[0] is the position of the next step (what the host resets and reads back); the step's first kernel
// copies it to ctr[1], every later kernel of the step reads ctr[1], and the step's last kernel writes ctr[0] =
// ctr[1] + 1. No kernel writes a slot that another workgroup of the same launch reads, so one captured graph replays
// every step (the reference's device-resident position, whisper.cu:7-8).
//
//   dec_embed_ln  token + position embedding fused with the first LayerNorm (whisper.cu:303-307, 65-69)
//   dec_gemm      skinny GEMM for M <= 32 rows per tile on the matrix cores: both operands of a K slice loaded
//                 straight into LDS at once, W rows the 32x32x16 MFMA A operand and x rows the B operand; split-K
//                 over workgroups (grid.y) and over the 4 waves of a workgroup. Epilogues: fp32 split-K partials,
//                 GELU -> fp16, fp16, or logits with a masked per-workgroup argmax (gemv_* + cuBLAS + fill_bias,
//                 whisper.cu:92-97, 309-317, 497-567)
//   dec_attn      attention of one query per (row, head) over a run of keys: self-attention over the cache, which
//                 sums the q/k/v projection's split-K partials for its (row, head), adds the bias and writes the
//                 step's key and value into the cache (kv_write + whisper.cu:319-353), and cross-attention over the
//                 encoder keys/values, which projects its own query from the row's LayerNorm output and records the
//                 alignment-head probabilities (whisper.cu:355-449)
//   dec_add_ln    residual add of the split-K partials + bias, fused with the next LayerNorm (whisper.cu:71-82)
//   dec_argmax    greedy choice from the per-workgroup argmax partials; advances the position (whisper.cu:451-495)
#include "mz_common.h"
#include "mz_kernels.h"

namespace {

// LayerNorm of one row held as v = x[4t .. 4t + 3] by thread t (threads with 4t >= dim hold zeros), written as fp16;
// gamma / beta come in already loaded. Each wave takes the mean and the sum of squared deviations of its own
// elements (two passes over registers), and one exchange through LDS combines the waves' pairs (Chan et al.'s
// pairwise update): one barrier per row. The workgroup is at most 16 waves; red holds 16 pairs.
__device__ __forceinline__ void ln_row4(float4 v, bool on, int dim, f16x4 wv, f16x4 bv, f16* __restrict__ y,
                                       float eps, float2* red) {
    const int c = 4 * threadIdx.x, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const float nk = (float)min(256, dim - 256 * wave);  // elements of this wave (every wave holds at least 4)
    const float mk = wave_sum(on ? v.x + v.y + v.z + v.w : 0.f) / nk;
    const float ex = v.x - mk, ey = v.y - mk, ez = v.z - mk, ew = v.w - mk;
    const float qk = wave_sum(on ? ex * ex + ey * ey + ez * ez + ew * ew : 0.f);
    if ((threadIdx.x & 63) == 0) red[wave] = make_float2(mk, qk);
    __syncthreads();
    float mean = 0.f;
    for (int i = 0; i < nw; i++) mean += (float)min(256, dim - 256 * i) * red[i].x;
    mean /= dim;
    float m2 = 0.f;
    for (int i = 0; i < nw; i++) {
        const float d = red[i].x - mean;
        m2 += red[i].y + (float)min(256, dim - 256 * i) * d * d;
    }
    const float rstd = rsqrtf(m2 / dim + eps);
    if (on) {
        const float dx = v.x - mean, dy = v.y - mean, dz = v.z - mean, dw = v.w - mean;
        st4(y + c, dx * rstd * (float)wv[0] + (float)bv[0], dy * rstd * (float)wv[1] + (float)bv[1],
            dz * rstd * (float)wv[2] + (float)bv[2], dw * rstd * (float)wv[3] + (float)bv[3]);
    }
}

// ---------------------------------------------------------------- row kernels (one workgroup per row)

__global__ void __launch_bounds__(512) dec_add_ln_kernel(const float* xin, float* x, const float* __restrict__ parts,
                                                         int nparts, long part_stride, const f16* __restrict__ bias,
                                                         const f16* __restrict__ w, const f16* __restrict__ b,
                                                         f16* __restrict__ y, int dim, float eps) {
    __shared__ float2 red[16];
    const int row = blockIdx.x, c = 4 * threadIdx.x;
    const bool on = c < dim;
    float4 v = {0.f, 0.f, 0.f, 0.f};
    f16x4 wv = {}, bv = {};
    if (on) {
        // every load of the row is issued before the first use
        const long idx = (long)row * dim + c;
        float4 pp[MZ_MAX_PARTS];
#pragma unroll
        for (int s = 0; s < MZ_MAX_PARTS; s++)
            if (s < nparts) pp[s] = *(const float4*)(parts + s * part_stride + idx);
        v = *(const float4*)(xin + idx);
        const f16x4 bb = bias ? *(const f16x4*)(bias + c) : f16x4{};
        wv = *(const f16x4*)(w + c);
        bv = *(const f16x4*)(b + c);
#pragma unroll
        for (int s = 0; s < MZ_MAX_PARTS; s++)
            if (s < nparts) {
                v.x += pp[s].x;
                v.y += pp[s].y;
                v.z += pp[s].z;
                v.w += pp[s].w;
            }
        v.x += (float)bb[0];
        v.y += (float)bb[1];
        v.z += (float)bb[2];
        v.w += (float)bb[3];
        *(float4*)(x + idx) = v;
    }
    ln_row4(v, on, dim, wv, bv, y + (long)row * dim, eps, red);
}

// LayerNorm of one row held by one wave, NC float4 per lane (v[i] = x[4 (lane + 64 i) ..]), written to y as fp16:
// two-pass statistics over the wave through DPP and lane reads (no LDS, no barrier)
template <int NC>
__device__ __forceinline__ void ln_wave(const f32x4 (&v)[NC], const f16x4 (&wv)[NC], const f16x4 (&bv)[NC],
                                        f16* __restrict__ y, float eps) {
    constexpr int dim = 256 * NC;
    const int lane = threadIdx.x & 63;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NC; i++) sum += (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]);
    const float mean = wave_sum(sum) / dim;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NC; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float d = v[i][e] - mean;
            q = fmaf(d, d, q);
        }
    const float rstd = rsqrtf(wave_sum(q) / dim + eps);
#pragma unroll
    for (int i = 0; i < NC; i++) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; e++) o[e] = (v[i][e] - mean) * rstd * (float)wv[i][e] + (float)bv[i][e];
        st4(y + (lane + 64 * i) * 4, o[0], o[1], o[2], o[3]);
    }
}

// dec_add_ln_kernel's work with one wave per row for NC float4 per lane (dim = 256 NC) and NP partials: every load of
// the row (residual, partials, bias, gamma, beta: 6 NC + 3 NC requests per lane) is issued before the first use, the
// residual is summed in dec_add_ln_kernel's order (the same x), and the LayerNorm statistics are two-pass sums over
// the wave through DPP and lane reads, so no barrier and no LDS are needed.
template <int NC, int NP>
__global__ void __launch_bounds__(64) dec_add_ln_wave_kernel(const float* xin, float* x, const float* __restrict__ parts,
                                                              long part_stride, const f16* __restrict__ bias,
                                                              const f16* __restrict__ w, const f16* __restrict__ b,
                                                              f16* __restrict__ y, float eps) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int dim = 256 * NC;
    const int row = blockIdx.x, lane = threadIdx.x;
    const long r0 = (long)row * dim;
    f32x4 v[NC], pp[NP][NC];
    f16x4 bb[NC], wv[NC], bv[NC];
#pragma unroll
    for (int i = 0; i < NC; i++) v[i] = *(const f32x4*)(xin + r0 + (lane + 64 * i) * 4);
#pragma unroll
    for (int s = 0; s < NP; s++)
#pragma unroll
        for (int i = 0; i < NC; i++) pp[s][i] = *(const f32x4*)(parts + s * part_stride + r0 + (lane + 64 * i) * 4);
    const __amdgpu_buffer_rsrc_t rB = rsrc(bias, bias ? (unsigned)dim * 2u : 0u);
#pragma unroll
    for (int i = 0; i < NC; i++) {
        const unsigned o = (unsigned)(lane + 64 * i) * 8u;
        bb[i] = __builtin_bit_cast(f16x4, __builtin_amdgcn_raw_buffer_load_b64(rB, o, 0, 0));
        wv[i] = *(const f16x4*)(w + (lane + 64 * i) * 4);
        bv[i] = *(const f16x4*)(b + (lane + 64 * i) * 4);
    }
    __builtin_amdgcn_sched_barrier(0);  // every request above is issued before anything waits for data
#pragma unroll
    for (int i = 0; i < NC; i++) {
#pragma unroll
        for (int s = 0; s < NP; s++) v[i] += pp[s][i];
#pragma unroll
        for (int e = 0; e < 4; e++) v[i][e] += (float)bb[i][e];
        *(f32x4*)(x + r0 + (lane + 64 * i) * 4) = v[i];
    }
    ln_wave<NC>(v, wv, bv, y + r0, eps);
#endif
}

__global__ void __launch_bounds__(512) dec_embed_ln_kernel(const int* __restrict__ tok, int* __restrict__ ctr,
                                                           const f16* __restrict__ emb, const f16* __restrict__ pe,
                                                           float* __restrict__ x, const f16* __restrict__ w,
                                                           const f16* __restrict__ b, f16* __restrict__ y, int dim,
                                                           int maxT, float eps) {
    __shared__ float2 red[16];
    const int row = blockIdx.x, c = 4 * threadIdx.x;
    const bool on = c < dim;
    f16x4 wv = {}, bv = {};
    if (on) {
        wv = *(const f16x4*)(w + c);
        bv = *(const f16x4*)(b + c);
    }
    const int p = min(ctr[0], maxT - 1);
    if (row == 0 && threadIdx.x == 0) ctr[1] = p;  // the position of this step, for its later kernels
    float4 v = {0.f, 0.f, 0.f, 0.f};
    if (on) {
        const int t = tok[(long)row * maxT + p];
        const f16x4 e = *(const f16x4*)(emb + (long)t * dim + c), q = *(const f16x4*)(pe + (long)p * dim + c);
        v = {(float)e[0] + (float)q[0], (float)e[1] + (float)q[1], (float)e[2] + (float)q[2], (float)e[3] + (float)q[3]};
        *(float4*)(x + (long)row * dim + c) = v;
    }
    ln_row4(v, on, dim, wv, bv, y + (long)row * dim, eps, red);
}

// ---------------------------------------------------------------- skinny GEMM

typedef __attribute__((address_space(3))) void lds_void;
#define LDSP(q) ((lds_void*)(q))

// s_waitcnt operand that waits until at most n vector memory operations of this wave are outstanding (n < 64)
constexpr int vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }


// Cache policy of the decoder's streams. The cross keys / values (983 MB per 32-row turbo step) and the LM head's
// tied embedding (133 MB) are read nontemporally. The projection weights are read with the default policy when the
// caller sets w_nt = 0 (the engine does when all layers' projections fit the 256 MB memory-side cache with room to
// spare, as large-v3-turbo's 183 MB do, and the batch has at least two rows): they then stay in that cache from one
// step to the next while the nontemporal streams pass through, and the latency-bound projections wait less for
// memory (32-row turbo step 415.1 -> 399.7 us). large-v3's 1.47 GB cannot stay, and there, as at one row, the
// nontemporal loads are faster (3.07 -> 2.98 ms and 248 -> 245 us per step).
constexpr int MZ_NT = 2;  // cache-policy bit of a buffer load: nontemporal

// One workgroup per (32 output columns, K slice, 32 rows): both operands of its K slice (<= MZ_DEC_KSLICE) go from
// memory straight into LDS with every load issued at once (buffer_load ... lds, 16 bytes per lane), in 1 KB blocks of
// 8 rows x 64 halves: lane i of a load writes block bytes 16 i, so one load reads 8 whole 128-byte rows (full cache
// lines; a 32-row MFMA fragment read straight from memory touches 32 lines per instruction and runs at a quarter of
// the rate). Block (g, rg) of an operand holds rows 8 rg .. 8 rg + 7, k = 64 g .. 64 g + 63, its row r chunk c at
// 16-byte position c ^ r ^ (rg & 1): the fragment reads of 16 consecutive lanes (8 rows of two blocks) hit distinct
// banks. The 4 waves split the K groups; their 32x32 products are summed in LDS. Every operand of the epilogue (bias,
// mask, position) is requested at entry with the loads, so the kernel makes a single round trip to memory.
// KS: the largest K slice of the launch (LDS sized to it: a workgroup asks for no more than it uses)
template <int EPI, int KS>
__global__ void __launch_bounds__(256) dec_gemm_kernel(const MzDec p) {
#if defined(__HIP_DEVICE_COMPILE__)  // the buffer-resource type exists only in the device pass
    constexpr int NC = 4;  // output columns per epilogue thread
    static_assert(KS <= MZ_DEC_KSLICE && 64 * KS * 2 >= 4 * 32 * 33 * 4, "LDS holds the operands and the reduction");
    __shared__ __attribute__((aligned(16))) f16 lds[64 * KS];
    f16* const sw = lds;
    f16* const sx = lds + 32 * KS;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 31, lh = lane >> 5;
    const int n0 = blockIdx.x * 32, ks = blockIdx.y, m0 = blockIdx.z * 32;
    const int ksl = p.K / p.ksplit, kb = ks * ksl, G = ksl >> 6;
    const int ml = tid >> 3, nl = (tid & 7) * NC, m = m0 + ml;

    // direct loads: x rows m0.., W rows n0.. (rows past M or N read zeros through the descriptor's range check)
    const int r8 = lane >> 3, q8 = lane & 7;
    // 32-bit offsets throughout (the operands are far below 4 GB)
    const unsigned ldx2 = (unsigned)p.ldx * 2u, mrows = (unsigned)min(p.M - m0, 32);
    const __amdgpu_buffer_rsrc_t rX = rsrc(p.x + (long)m0 * p.ldx, mrows * ldx2);
    const __amdgpu_buffer_rsrc_t rW = rsrc(p.W, (unsigned)p.N * (unsigned)p.K * 2u);
    for (int i = wave; i < 4 * G; i += 4) {
        const int g = i >> 2, rg = i & 3, c = q8 ^ r8 ^ (rg & 1);
        const unsigned col = (unsigned)(kb + g * 64 + c * 8) * 2;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rX, LDSP(sx + i * 512), 16, (unsigned)(rg * 8 + r8) * ldx2 + col, 0, 0,
                                                 0);
        const unsigned ow = (unsigned)(n0 + rg * 8 + r8) * (unsigned)p.K * 2u + col;
        if (p.w_nt)  // (the policy is an immediate of the instruction: one load per branch, a uniform branch)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rW, LDSP(sw + i * 512), 16, ow, 0, 0, MZ_NT);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rW, LDSP(sw + i * 512), 16, ow, 0, 0, 0);
    }
    // epilogue operands
    float bv[NC];
    bool msk[NC];
#pragma unroll
    for (int e = 0; e < NC; e++) {
        const int n = min(n0 + nl + e, p.N - 1);
        bv[e] = (EPI != DEPI_PARTIAL && p.bias) ? (float)p.bias[n] : 0.f;
        msk[e] = EPI == DEPI_LOGITS ? p.sup[n] != 0 : false;
    }
    const int pos = EPI == DEPI_LOGITS ? p.ctr[1] : 0;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // W rows are the MFMA A operand, x rows the B operand; wave w takes K groups w, w + 4, ...
    f32x16 acc = f32x16{};
    const int rgx = lr >> 3, rr = lr & 7;
    for (int g = wave; g < G; g += 4) {
        const f16* bw = sw + (g * 4 + rgx) * 512 + rr * 64;
        const f16* bx = sx + (g * 4 + rgx) * 512 + rr * 64;
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const int off = ((2 * st + lh) ^ rr ^ (rgx & 1)) << 3;
            acc = mfma32(*(const f16x8*)(bw + off), *(const f16x8*)(bx + off), acc);
        }
    }
    __syncthreads();  // every wave is done with the operand blocks: the LDS holds the partial products next
    float(*red)[32][33] = (float(*)[32][33])lds;
    // accumulator element r: n = n0 + 8 (r / 4) + 4 lh + r % 4, m = m0 + lr
#pragma unroll
    for (int r = 0; r < 16; r++) red[wave][8 * (r >> 2) + 4 * lh + (r & 3)][lr] = acc[r];
    __syncthreads();
    float v[NC];
#pragma unroll
    for (int e = 0; e < NC; e++)
        v[e] = red[0][nl + e][ml] + red[1][nl + e][ml] + red[2][nl + e][ml] + red[3][nl + e][ml];

    if (EPI == DEPI_LOGITS) {
        // logits, and the largest unmasked one of this workgroup's columns per row (lowest id on ties)
        const bool first = pos + 1 == p.prompt_len;
        float best = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int e = 0; e < NC; e++) {
            const int n = n0 + nl + e;
            if (m < p.M && n < p.N) {
                ((float*)p.out)[(long)m * p.ldo + n] = v[e];
                const bool masked = msk[e] || (first && (n == p.bs1 || n == p.bs2));
                if (!masked && (v[e] > best || (v[e] == best && n < bi))) {
                    best = v[e];
                    bi = n;
                }
            }
        }
        group8_argmax(best, bi);  // the 8 lanes of one row are adjacent in the wave
        if ((tid & 7) == 0 && m < p.M) {
            int2 r;
            r.x = __float_as_int(best);
            r.y = bi;
            ((int2*)p.amax)[(long)blockIdx.x * p.M + m] = r;
        }
        return;
    }
    if (m >= p.M) return;
#pragma unroll
    for (int e = 0; e < NC; e++) {
        const int n = n0 + nl + e;
        if (n >= p.N) continue;
        if (EPI == DEPI_PARTIAL) {
            ((float*)p.out)[((long)ks * p.M + m) * p.ldo + n] = v[e];
            continue;
        }
        const float a = v[e] + bv[e];
        if (EPI == DEPI_GELU_F16) {
            ((f16*)p.out)[(long)m * p.ldo + n] = (f16)gelu_erf_h(a);
        } else if (EPI == DEPI_F16) {
            ((f16*)p.out)[(long)m * p.ldo + n] = (f16)a;
        }
    }
#endif
}

// ---------------------------------------------------------------- LM head

// Logits of 32 rows (row block blockIdx.y) over the whole vocabulary, with each workgroup's masked argmax per row. The
// workgroup keeps its rows' x in registers (the B operands of 16x16x32 products, its quarter of K per wave) and streams a contiguous
// run of 16-column weight tiles through a 3-deep LDS ring (direct loads, two tiles in flight), so x is read once per
// workgroup and the weight stream never waits for a round trip per tile. Ids and the argmax rules as dec_gemm's.
constexpr int LM_TILE = 16;                          // vocabulary ids per tile
constexpr int LM_TB = LM_TILE * MZ_DEC_KSLICE * 2;   // bytes of one weight tile in LDS
constexpr int LM_XG = MZ_DEC_KSLICE / 64 / 4;        // K groups of 64 per wave

__global__ void __launch_bounds__(256) dec_lmhead_kernel(const MzDec p, int T) {
#if defined(__HIP_DEVICE_COMPILE__)
    __shared__ __attribute__((aligned(16))) f16 lds[3 * LM_TB / 2 + 4 * 32 * (LM_TILE + 1) * 2];
    float(*red)[32][LM_TILE + 1] = (float(*)[32][LM_TILE + 1])(lds + 3 * LM_TB / 2);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, lq = lane >> 4;
    const int G = p.K >> 6, ntiles = (p.N + LM_TILE - 1) / LM_TILE;
    const int t0 = blockIdx.x * T, nt = min(T, ntiles - t0), m0 = blockIdx.y * 32;
    const int r8 = lane >> 3, q8 = lane & 7;
    const int pos = p.ctr[1];
    const bool first = pos + 1 == p.prompt_len;
    const int em = tid >> 3, ec = (tid & 7) * 2;  // epilogue thread: row em, ids n0 + ec, n0 + ec + 1 of each tile
    // the suppression mask of this thread's ids in every tile, requested before any other load (bit 2 t + e)
    unsigned smask = 0;
    {
        unsigned char sv[32];  // all 32 byte loads in flight together (clamped ids, no branches), then combined
#pragma unroll
        for (int k = 0; k < 32; k++) sv[k] = p.sup[min((t0 + (k >> 1)) * LM_TILE + ec + (k & 1), p.N - 1)];
#pragma unroll
        for (int k = 0; k < 32; k++) {
            const int t = k >> 1, n = (t0 + t) * LM_TILE + ec + (k & 1);
            smask |= (t < nt && n < p.N && sv[k] ? 1u : 0u) << k;
        }
    }

    // x rows (32 x K) through LDS into this wave's fragments: groups g = wave + 4 i, halves s of 32 k, row halves h
    // rows past M read zeros through the descriptor's range check
    const __amdgpu_buffer_rsrc_t rX = rsrc(p.x + (long)m0 * p.ldx, (unsigned)min(p.M - m0, 32) * (unsigned)p.ldx * 2u);
    for (int i = wave; i < 4 * G; i += 4) {
        const int g = i >> 2, rg = i & 3, c = q8 ^ r8 ^ (rg & 1);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rX, LDSP(lds + i * 512), 16,
                                                 (unsigned)(rg * 8 + r8) * (unsigned)p.ldx * 2u +
                                                     (unsigned)(g * 64 + c * 8) * 2u,
                                                 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    f16x8 xf[LM_XG][2][2];
#pragma unroll
    for (int i = 0; i < LM_XG; i++) {
        const int g = wave + 4 * i;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int row = 16 * h + l16, rg = row >> 3, rr = row & 7;
#pragma unroll
            for (int st = 0; st < 2; st++) {
                const int c = 4 * st + lq;
                xf[i][st][h] = g < G ? *(const f16x8*)(lds + (g * 4 + rg) * 512 + rr * 64 + ((c ^ rr ^ (rg & 1)) << 3))
                                     : f16x8{};
            }
        }
    }
    __syncthreads();  // the x staging area becomes the weight ring

    const __amdgpu_buffer_rsrc_t rW = rsrc(p.W, (unsigned)p.N * (unsigned)p.K * 2u);
    auto issue = [&](int t) {  // tile t of this workgroup into ring slot t % 3: 2 G blocks of 8 rows x 64 k
        f16* dst = lds + (t % 3) * (LM_TB / 2);
        const int n0 = (t0 + t) * LM_TILE;
        for (int i = wave; i < 2 * G; i += 4) {
            const int g = i >> 1, rg = i & 1, c = q8 ^ r8 ^ rg;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rW, LDSP(dst + i * 512), 16,
                                                     (unsigned)(n0 + rg * 8 + r8) * (unsigned)p.K * 2u +
                                                         (unsigned)(g * 64 + c * 8) * 2u,
                                                     0, 0, MZ_NT);
        }
    };
    if (nt > 0) issue(0);
    if (nt > 1) issue(1);

    // running best of this thread's row over the workgroup's tiles
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int t = 0; t < nt; t++) {
        // tile t landed (at most the next tile's loads, issued after it, still in flight); every wave is done with
        // the slot the next issue overwrites and with the previous tile's partial sums
        // (the count is exact for K = MZ_DEC_KSLICE: 10 weight loads per wave per tile; loads complete in order, so
        // with 10 or fewer operations outstanding none of tile t's loads is)
        static_assert(2 * MZ_DEC_KSLICE / 64 / 4 == 10, "10 weight loads per wave per tile at the full K");
        if (t + 1 < nt && G == MZ_DEC_KSLICE / 64)
            __builtin_amdgcn_s_waitcnt((10 & 15) | (7 << 4) | (15 << 8));
        else
            __builtin_amdgcn_s_waitcnt(0);
        lds_barrier();
        if (t + 2 < nt) issue(t + 2);
        const f16* wt = lds + (t % 3) * (LM_TB / 2);
        f32x4 acc0 = f32x4{}, acc1 = f32x4{};
        const int rg = l16 >> 3, rr = l16 & 7;
#pragma unroll
        for (int i = 0; i < LM_XG; i++) {
            const int g = wave + 4 * i;
            if (g < G) {
#pragma unroll
                for (int st = 0; st < 2; st++) {
                    const int c = 4 * st + lq;
                    const f16x8 wf = *(const f16x8*)(wt + (g * 2 + rg) * 512 + rr * 64 + ((c ^ rr ^ rg) << 3));
                    acc0 = mfma16(wf, xf[i][st][0], acc0);
                    acc1 = mfma16(wf, xf[i][st][1], acc1);
                }
            }
        }
        // element r of lane l: id n0 + 4 (l / 16) + r, row l % 16 (+ 16 for acc1)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            red[wave][l16][4 * lq + r] = acc0[r];
            red[wave][16 + l16][4 * lq + r] = acc1[r];
        }
        lds_barrier();
        const int n0 = (t0 + t) * LM_TILE;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int n = n0 + ec + e;
            const float v = red[0][em][ec + e] + red[1][em][ec + e] + red[2][em][ec + e] + red[3][em][ec + e];
            if (m0 + em < p.M && n < p.N) {
                ((float*)p.out)[(long)(m0 + em) * p.ldo + n] = v;
                const bool masked = ((smask >> (2 * t + e)) & 1u) || (first && (n == p.bs1 || n == p.bs2));
                if (!masked && (v > best || (v == best && n < bi))) {
                    best = v;
                    bi = n;
                }
            }
        }
    }
    group8_argmax(best, bi);  // the 8 threads of one row are adjacent lanes
    if ((tid & 7) == 0 && m0 + em < p.M) {
        int2 r;
        r.x = __float_as_int(best);
        r.y = bi;
        ((int2*)p.amax)[(long)blockIdx.x * p.M + m0 + em] = r;
    }
#endif
}

// ---------------------------------------------------------------- attention of one query per (row, head)

// One workgroup per (row, head): AG groups of 8 lanes stream the keys round-robin (a lane holds 8 of the 64 dims),
// loading each key's k and v rows together, and keep a private online softmax; the groups merge in LDS. Scores are
// in the log2 domain (log2(e) / 8 folded into q), all arithmetic fp32. The alignment heads' probabilities are
// written for position ctr[1] from the scores kept in LDS.
// AG groups of 8 lanes per workgroup, AU keys in flight per group: 32 x 8 (every (row, head) workgroup of a 32-row
// batch resident at once, 64 KB in flight each; one pass over a self-attention cache of up to 256 positions; 64 x 4
// was 3 us per step slower there, its merge over twice the groups included).
// The cross-attention's query projection runs in the same workgroup (wq set): its head's 64 rows of wq (read by the
// 32 rows' workgroups of that head, so from L2 after the first) against the row's layer-norm output staged in LDS,
// 8 lanes per weight row over whole 128-byte lines, with the first keys and values in flight behind them.
template <int AG, int AU, bool CROSS>
__global__ void __launch_bounds__(AG * 8) dec_attn_kernel(const MzDecAttn a) {
    __shared__ float qs[MZ_HD];
    __shared__ __attribute__((aligned(16))) f16 xs[MZ_DEC_KSLICE];
    __shared__ float sc[MZ_TPAD];
    __shared__ float gm[AG], gl[AG];
    __shared__ float gacc[AG][MZ_HD + 1];
    __shared__ float tot[2];
    __shared__ __attribute__((aligned(16))) f16 kvn[2][MZ_HD];  // the step's own key and value (self, kw set)

    const int bh = blockIdx.x, b = bh / a.nh, head = bh - b * a.nh;
    const int tid = threadIdx.x, grp = tid >> 3, sub = tid & 7;
    // the row's done flag, the position and the alignment slot: the self-attention reads them first (its keys'
    // count needs the position); the cross-attention (L given), whose keys do not depend on the step, once its
    // first requests are issued
    bool done = false;
    int pos = 0, slot = -1;
    auto step_scalars = [&] {
        done = a.done[b] != 0;
        pos = a.ctr[1];
        slot = CROSS && a.aslot ? a.aslot[head] : -1;
    };
    if (!CROSS) {
        step_scalars();
        if (done) return;
    }
    const int L = CROSS ? a.L : min(pos + 1, a.maxT);

    // the first batch of keys and values is requested before the query, which arrives in the same round trip
    const f16* kb = a.k + (long)b * a.kv_b + (long)head * a.kv_h + sub * 8;
    const f16* vb = a.v + (long)b * a.kv_b + (long)head * a.kv_h + sub * 8;
    // keys and values are streamed once per step: nontemporal loads (about 10% more HBM throughput than cached ones)
    f16x8 kk[AU], vv[AU];
    auto fetch = [&](int j0) {
#pragma unroll
        for (int u = 0; u < AU; u++) {
            const int j = j0 + u * AG;
            kk[u] = j < L ? __builtin_nontemporal_load((const f16x8*)(kb + (long)j * MZ_HD)) : f16x8{};
            vv[u] = j < L ? __builtin_nontemporal_load((const f16x8*)(vb + (long)j * MZ_HD)) : f16x8{};
        }
    };
    constexpr float QS = 0.125f * 1.4426950408889634f;  // 1/8 and log2(e)
    if (CROSS && AG * 8 == 256 && a.wq) {
        // q[i] = xin[b] . wq[head * 64 + i] + qbias: lane (r8, q8) of wave w takes rows 8 w + r8 and 32 + 8 w + r8,
        // 16-byte chunks q8, q8 + 8, ... of each (nj per row); 8 lanes sum one row through DPP
        const int w = tid >> 6, r8 = (tid >> 3) & 7, q8 = tid & 7, nj = a.d >> 6;
        constexpr int NJ = MZ_DEC_KSLICE / 64;
        // in issue order, with no wait between them (range-checked buffer loads, zeros past the range, so no load
        // sits behind a branch): the row (one chunk per thread, d / 8 <= 160), the first 32 weight rows, this
        // thread's two query biases, the first keys and values; each wait below then covers only what it needs.
        // Chunks j >= nj of a weight row read the next row or zeros and are never used.
        const bool xl = tid < (a.d >> 3);
        const __amdgpu_buffer_rsrc_t rX = rsrc(a.xin + (long)b * a.d, (unsigned)a.d * 2u);
        const __amdgpu_buffer_rsrc_t rW = rsrc(a.wq + (long)head * MZ_HD * a.d, (unsigned)(MZ_HD * a.d) * 2u);
        const __amdgpu_buffer_rsrc_t rQB = rsrc(a.qbias, a.qbias ? (unsigned)a.d * 2u : 0u);
        const unsigned wo = (unsigned)(((8 * w + r8) * a.d + q8 * 8) * 2);
        const f16x8 xv0 = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rX, (unsigned)tid * 16u, 0, 0));
        f16x8 wv[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++)
            wv[j] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rW, wo + j * 128u, 0, 0));
        const unsigned short qb[2] = {
            __builtin_amdgcn_raw_buffer_load_b16(rQB, (unsigned)(head * MZ_HD + 8 * w + r8) * 2u, 0, 0),
            __builtin_amdgcn_raw_buffer_load_b16(rQB, (unsigned)(head * MZ_HD + 32 + 8 * w + r8) * 2u, 0, 0)};
#pragma unroll
        for (int u = 0; u < AU; u++) {  // the first batch: keys grp + 32 u < 256 <= L (checked at launch)
            kk[u] = __builtin_nontemporal_load((const f16x8*)(kb + (long)(grp + u * AG) * MZ_HD));
            vv[u] = __builtin_nontemporal_load((const f16x8*)(vb + (long)(grp + u * AG) * MZ_HD));
        }
        __builtin_amdgcn_sched_barrier(0);  // every request above is issued before anything waits for data
        step_scalars();
        if (done) {  // a finished row: no attention
            __builtin_amdgcn_s_waitcnt(vm_wait(0));
            return;
        }
        if (xl) *(f16x8*)&xs[tid * 8] = xv0;
        lds_barrier();  // the row in LDS; the weight rows, keys and values stay in flight
#pragma unroll
        for (int half = 0; half < 2; half++) {
            float t = 0.f;
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                if (j < nj) {
                    const f16x8 xv = *(const f16x8*)&xs[(q8 + 8 * j) * 8];
#pragma unroll
                    for (int e = 0; e < 8; e += 2)
                        t = __builtin_amdgcn_fdot2(f16x2{wv[j][e], wv[j][e + 1]}, f16x2{xv[e], xv[e + 1]}, t, false);
                }
            }
            if (half == 0) {  // the second 32 rows, requested once the first ones are consumed
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    wv[j] = __builtin_bit_cast(
                        f16x8, __builtin_amdgcn_raw_buffer_load_b128(rW, wo + (unsigned)(32 * a.d * 2) + j * 128u, 0, 0));
            }
            t = group8_sum(t);
            const int i = 32 * half + 8 * w + r8;
            if (q8 == 0) qs[i] = (t + (a.qbias ? (float)__builtin_bit_cast(f16, qb[half]) : 0.f)) * QS;
        }
    } else {
        if (CROSS) step_scalars();  // (the cross-attention without its query projection)
        if (done) return;
        fetch(grp);
        // thread 64 w + i takes dim i of q (w = 0) or, with kw set, of the step's key (1) or value (2)
        const long qrow = a.qrow ? a.qrow : a.d;
        if (tid < ((!CROSS && a.kw) ? 3 : 1) * MZ_HD) {
            const int which = tid >> 6, i = tid & 63, col = which * a.d + head * MZ_HD + i;
            const f16* bias = which == 0 ? a.qbias : a.kvbias ? a.kvbias + (which - 1) * a.d : nullptr;
            float v = bias ? (float)bias[head * MZ_HD + i] : 0.f;
            for (int s = 0; s < a.nq; s++) v += a.q[s * a.qstride + (long)b * qrow + col];
            if (which == 0) {
                qs[i] = v * QS;
            } else {
                const f16 h = (f16)v;
                kvn[which - 1][i] = h;
                if (pos < a.maxT)
                    (which == 1 ? a.kw : a.vw)[(long)b * a.kv_b + (long)head * a.kv_h + (long)pos * MZ_HD + i] = h;
            }
        }
    }
    __syncthreads();
    // with kw set the step's position is read from kvn, never from the cache this workgroup has just written
    const bool own = !CROSS && a.kw != nullptr;
    float q8[8];
#pragma unroll
    for (int e = 0; e < 8; e++) q8[e] = qs[sub * 8 + e];

    float m = -INFINITY, l = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j0 = grp; j0 < L; j0 += AG * AU) {
        if (j0 != grp) fetch(j0);
        if (own) {
#pragma unroll
            for (int u = 0; u < AU; u++)
                if (j0 + u * AG == pos) {
                    kk[u] = *(const f16x8*)&kvn[0][sub * 8];
                    vv[u] = *(const f16x8*)&kvn[1][sub * 8];
                }
        }
        float s[AU];
#pragma unroll
        for (int u = 0; u < AU; u++) {
            float t = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) t = fmaf(q8[e], (float)kk[u][e], t);
            t = group8_sum(t);
            const int j = j0 + u * AG;
            s[u] = j < L ? t : -INFINITY;
            if (slot >= 0 && sub == 0 && j < L) sc[j] = t;
        }
        float mx = s[0];  // key j0 < L: finite
#pragma unroll
        for (int u = 1; u < AU; u++) mx = fmaxf(mx, s[u]);
        const float mn = fmaxf(m, mx);
        const float cr = __builtin_amdgcn_exp2f(m - mn);
        l *= cr;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] *= cr;
#pragma unroll
        for (int u = 0; u < AU; u++) {
            const float pe = __builtin_amdgcn_exp2f(s[u] - mn);
            l += pe;
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e] = fmaf(pe, (float)vv[u][e], acc[e]);
        }
        m = mn;
    }
    if (sub == 0) {
        gm[grp] = m;  // -inf for a group that saw no key
        gl[grp] = l;
    }
#pragma unroll
    for (int e = 0; e < 8; e++) gacc[grp][sub * 8 + e] = acc[e];
    __syncthreads();
    if (tid < MZ_HD) {
        float M = gm[0];
        for (int g = 1; g < AG; g++) M = fmaxf(M, gm[g]);
        float lt = 0.f, o = 0.f;
        for (int g = 0; g < AG; g++) {
            const float w = __builtin_amdgcn_exp2f(gm[g] - M);
            lt = fmaf(gl[g], w, lt);
            o = fmaf(gacc[g][tid], w, o);
        }
        a.out[(long)b * a.d + head * MZ_HD + tid] = (f16)(o / lt);
        if (tid == 0) {
            tot[0] = M;
            tot[1] = lt;
        }
    }
    if (slot < 0 || pos >= a.maxT) return;
    __syncthreads();
    const float M = tot[0], inv = 1.f / tot[1];
    const long ao = (((long)b * a.maxT + pos) * a.na + slot) * MZ_TENC;
    float* al = a.align + ao;
    f16* alh = a.alignh ? a.alignh + ao : nullptr;
    for (int j = tid; j < L; j += blockDim.x) {
        const float pj = __builtin_amdgcn_exp2f(sc[j] - M) * inv;
        al[j] = pj;
        if (alh) alh[j] = (f16)pj;
    }
}

// ---------------------------------------------------------------- cross-attention for small batches

// dec_attn_kernel<32, 8, true>'s arithmetic for batches of at most 256 / nh rows, where every (row, head) workgroup
// has a CU to itself: with only B x nh workgroups streaming, one workgroup's bytes in flight set the rate (a
// workgroup of the 32-row kernel keeps one batch, 64 KB, in flight). Here the row, all 64 query rows of wq (160
// registers per lane) and batch 0 are requested together, and batches 1 and 2 straight into LDS (buffer_load ...
// lds): ~350 KB in flight from the start, and the query projection waits only for its own operands (vmcnt counts
// in issue order, so they are issued first). Then batches 3 (registers), 4 and 5 (refilling the two LDS slots as they
// are read) follow. Same groups, key order, per-batch online-softmax updates, projection order and merge as
// dec_attn_kernel: the same bits.
__global__ void __launch_bounds__(256, 1) dec_cross_wide_kernel(const MzDecCross a) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int AG = 32, AU = 8, BK = AG * AU, NB = (MZ_TENC + BK - 1) / BK, L = MZ_TENC;
    static_assert(NB == 6, "the staging schedule below is written for 6 batches");
    constexpr int NJ = MZ_DEC_KSLICE / 64;
    __shared__ __attribute__((aligned(16))) f16x8 kvs[2][2][AU][256];  // [slot][k|v][key u][thread]
    __shared__ __attribute__((aligned(16))) f16 xs[MZ_DEC_KSLICE];
    __shared__ float qs[MZ_HD];
    __shared__ float sc[MZ_TPAD];
    __shared__ float gm[AG], gl[AG];
    __shared__ float gacc[AG][MZ_HD + 1];
    __shared__ float tot[2];

    const int bh = blockIdx.x, b = bh / a.nh, head = bh - b * a.nh;
    const int tid = threadIdx.x, grp = tid >> 3, sub = tid & 7, wave = tid >> 6;
    const int r8 = (tid >> 3) & 7, q8 = tid & 7, nj = a.d >> 6;
    // scalars first (scalar loads, waited for only where used)
    const int pos = a.ctr[1];
    const int slot = a.aslot ? a.aslot[head] : -1;
    const bool done = a.done[b] != 0;
    const f16* kb = a.k + (long)b * a.kv_b + (long)head * a.kv_h;
    const f16* vb = a.v + (long)b * a.kv_b + (long)head * a.kv_h;
    const __amdgpu_buffer_rsrc_t rK = rsrc(kb, L * MZ_HD * 2), rV = rsrc(vb, L * MZ_HD * 2);
    f16x8 kk[AU], vv[AU];
    auto fetch = [&](int i) {  // batch i of this group into registers
#pragma unroll
        for (int u = 0; u < AU; u++) {
            const int j = i * BK + grp + u * AG;
            kk[u] = j < L ? __builtin_nontemporal_load((const f16x8*)(kb + (long)j * MZ_HD + sub * 8)) : f16x8{};
            vv[u] = j < L ? __builtin_nontemporal_load((const f16x8*)(vb + (long)j * MZ_HD + sub * 8)) : f16x8{};
        }
    };
    // batch i of every group into LDS slot s_: 2 AU loads per wave, lane l of wave w writing the 16 bytes thread
    // 64 w + l reads back; keys past L read zeros through the range check
    auto stage = [&](int i, int s_) {
#pragma unroll
        for (int u = 0; u < AU; u++) {
            const unsigned o = (unsigned)((i * BK + grp + u * AG) * MZ_HD + sub * 8) * 2u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rK, LDSP(&kvs[s_][0][u][wave * 64]), 16, o, 0, 0, MZ_NT);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rV, LDSP(&kvs[s_][1][u][wave * 64]), 16, o, 0, 0, MZ_NT);
        }
    };

    // in issue order: the row (one 16-byte chunk per thread), this thread's 40 chunks of wq (rows 8 w + r8 and
    // 32 + 8 w + r8, chunks q8, q8 + 8, ... of each), its two query biases, batch 0, batches 1 and 2 into LDS
    const bool xl = tid < (a.d >> 3);
    const f16x8 xv0 = xl ? *(const f16x8*)(a.xin + (long)b * a.d + tid * 8) : f16x8{};
    const f16* wr = a.wq + (long)(head * MZ_HD + 8 * wave + r8) * a.d + q8 * 8;
    f16x8 wv[2][NJ];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int j = 0; j < NJ; j++) wv[h][j] = j < nj ? *(const f16x8*)(wr + 32L * h * a.d + j * 64) : f16x8{};
    const __amdgpu_buffer_rsrc_t rQB = rsrc(a.qbias, a.qbias ? (unsigned)a.d * 2u : 0u);
    const unsigned short qb[2] = {__builtin_amdgcn_raw_buffer_load_b16(rQB, (unsigned)(head * MZ_HD + 8 * wave + r8) * 2u, 0, 0),
                         __builtin_amdgcn_raw_buffer_load_b16(rQB, (unsigned)(head * MZ_HD + 32 + 8 * wave + r8) * 2u,
                                                              0, 0)};
    fetch(0);
    stage(1, 0);
    stage(2, 1);
    __builtin_amdgcn_sched_barrier(0);  // every request above is issued before anything waits for data
    if (done) {  // a finished row: no attention (the staged loads land before the LDS is released)
        __builtin_amdgcn_s_waitcnt(vm_wait(0));
        return;
    }
    if (xl) *(f16x8*)&xs[tid * 8] = xv0;
    lds_barrier();  // the row in LDS; wq, the biases and the stream stay in flight

    // q[i] = xin[b] . wq[head * 64 + i] + qbias, the two halves of rows in the order of dec_attn_kernel
    constexpr float QS = 0.125f * 1.4426950408889634f;  // 1/8 and log2(e)
#pragma unroll
    for (int h = 0; h < 2; h++) {
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            if (j < nj) {
                const f16x8 xq = *(const f16x8*)&xs[(q8 + 8 * j) * 8];
#pragma unroll
                for (int e = 0; e < 8; e += 2)
                    t = __builtin_amdgcn_fdot2(f16x2{wv[h][j][e], wv[h][j][e + 1]}, f16x2{xq[e], xq[e + 1]}, t, false);
            }
        }
        t = group8_sum(t);
        const int i = 32 * h + 8 * wave + r8;
        if (q8 == 0) qs[i] = (t + (a.qbias ? (float)__builtin_bit_cast(f16, qb[h]) : 0.f)) * QS;
    }
    lds_barrier();
    float q8v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) q8v[e] = qs[sub * 8 + e];

    float m = -INFINITY, l = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int i, const f16x8(&K)[AU], const f16x8(&V)[AU]) {
        const int j0 = i * BK + grp;
        float s[AU];
#pragma unroll
        for (int u = 0; u < AU; u++) {
            float t = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) t = fmaf(q8v[e], (float)K[u][e], t);
            t = group8_sum(t);
            const int j = j0 + u * AG;
            s[u] = j < L ? t : -INFINITY;
            if (slot >= 0 && sub == 0 && j < L) sc[j] = t;
        }
        float mx = s[0];  // key j0 < L: finite
#pragma unroll
        for (int u = 1; u < AU; u++) mx = fmaxf(mx, s[u]);
        const float mn = fmaxf(m, mx);
        const float cr = __builtin_amdgcn_exp2f(m - mn);
        l *= cr;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] *= cr;
#pragma unroll
        for (int u = 0; u < AU; u++) {
            const float pe = __builtin_amdgcn_exp2f(s[u] - mn);
            l += pe;
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e] = fmaf(pe, (float)V[u][e], acc[e]);
        }
        m = mn;
    };
    // a slot's keys into (K, V) once its staged loads have landed (this wave's: the vmcnt wait before the call;
    // every wave's: the barrier)
    auto unstage = [&](int s_, f16x8(&K)[AU], f16x8(&V)[AU]) {
        lds_barrier();
#pragma unroll
        for (int u = 0; u < AU; u++) {
            K[u] = kvs[s_][0][u][tid];
            V[u] = kvs[s_][1][u][tid];
        }
    };
    // batches 0, 3 in registers; 1, 4 through slot 0; 2, 5 through slot 1 (2 AU vector memory operations per batch)
    f16x8 ks[AU], vs[AU];
    compute(0, kk, vv);
    fetch(3);
    __builtin_amdgcn_s_waitcnt(vm_wait(2 * AU));  // all but batch 3: batches 1 and 2 have landed
    unstage(0, ks, vs);
    lds_barrier();  // every wave has read slot 0
    stage(4, 0);
    compute(1, ks, vs);
    __builtin_amdgcn_s_waitcnt(vm_wait(4 * AU));  // all but batches 3 and 4
    unstage(1, ks, vs);
    lds_barrier();
    stage(5, 1);
    compute(2, ks, vs);
    compute(3, kk, vv);
    __builtin_amdgcn_s_waitcnt(vm_wait(2 * AU));  // all but batch 5
    unstage(0, ks, vs);
    compute(4, ks, vs);
    __builtin_amdgcn_s_waitcnt(vm_wait(0));
    unstage(1, ks, vs);
    compute(5, ks, vs);

    if (sub == 0) {
        gm[grp] = m;
        gl[grp] = l;
    }
#pragma unroll
    for (int e = 0; e < 8; e++) gacc[grp][sub * 8 + e] = acc[e];
    __syncthreads();
    if (tid < MZ_HD) {
        float M = gm[0];
        for (int g = 1; g < AG; g++) M = fmaxf(M, gm[g]);
        float lt = 0.f, o = 0.f;
        for (int g = 0; g < AG; g++) {
            const float w = __builtin_amdgcn_exp2f(gm[g] - M);
            lt = fmaf(gl[g], w, lt);
            o = fmaf(gacc[g][tid], w, o);
        }
        a.out[(long)b * a.d + head * MZ_HD + tid] = (f16)(o / lt);
        if (tid == 0) {
            tot[0] = M;
            tot[1] = lt;
        }
    }
    if (slot < 0 || pos >= a.maxT) return;
    __syncthreads();
    const float M = tot[0], inv = 1.f / tot[1];
    const long ao = (((long)b * a.maxT + pos) * a.na + slot) * MZ_TENC;
    float* al = a.align + ao;
    f16* alh = a.alignh ? a.alignh + ao : nullptr;
    for (int j = tid; j < L; j += 256) {
        const float pj = __builtin_amdgcn_exp2f(sc[j] - M) * inv;
        al[j] = pj;
        if (alh) alh[j] = (f16)pj;
    }
#endif
}

// ---------------------------------------------------------------- greedy choice

// Token p + 1 of row b from the LM head's per-workgroup partials (value, id) (kernels/whisper.cu:451-493 rules:
// the prompt positions stay; a finished row, or one whose every id is masked, gets eos). Workgroup 0 advances the
// position for the next step.
__global__ void __launch_bounds__(64) dec_argmax_kernel(const int2* __restrict__ amax, int nblk, int* __restrict__ tok,
                                                        int* __restrict__ done, int* __restrict__ ctr, int B, int maxT,
                                                        int prompt_len, int eos) {
    // one wave per row: lane l takes partials l, l + 64, ... (all of one batch of 8 in flight together), then the
    // wave's reduction; the lowest id wins ties, so the choice does not depend on the order
    const int b = blockIdx.x, tid = threadIdx.x;
    const int p = ctr[1];
    if (b == 0 && tid == 0) ctr[0] = p + 1;
    if (p + 1 < prompt_len || p + 1 >= maxT) return;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int i0 = tid; i0 < nblk; i0 += 64 * 8) {
        int2 r[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + 64 * u;
            r[u] = i < nblk ? amax[(long)i * B + b] : make_int2(__float_as_int(-INFINITY), 0x7fffffff);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float v = __int_as_float(r[u].x);
            if (v > best || (v == best && r[u].y < bi)) {
                best = v;
                bi = r[u].y;
            }
        }
    }
    wave_argmax(best, bi);
    if (tid == 0) {
        const int t = (done[b] || bi == 0x7fffffff) ? eos : bi;
        tok[(long)b * maxT + p + 1] = t;
        if (t == eos) done[b] = 1;
    }
}

}  // namespace

int mz_lm_tiles_per_block(int N) {
    const int ntiles = (N + LM_TILE - 1) / LM_TILE;
    return (ntiles + 255) / 256;  // at most 16 for N <= 65536 (the per-thread mask holds 2 bits per tile)
}
int mz_lm_blocks(int N) {
    const int ntiles = (N + LM_TILE - 1) / LM_TILE, T = mz_lm_tiles_per_block(N);
    return (ntiles + T - 1) / T;
}

hipError_t mz_dec_gemm_launch(hipStream_t s, int epi, const MzDec& g) {
    if (g.K % 64 != 0 || g.M <= 0 || g.N <= 0 || g.ksplit <= 0 || (g.K / 64) % g.ksplit != 0 ||
        g.K / g.ksplit > MZ_DEC_KSLICE || g.ldx % 8 != 0)
        return hipErrorInvalidValue;
    if (epi == DEPI_LOGITS && (!g.sup || !g.amax || !g.ctr || g.N > 65536 || g.K > MZ_DEC_KSLICE)) return hipErrorInvalidValue;
    if (epi != DEPI_PARTIAL && g.ksplit != 1) return hipErrorInvalidValue;
    const dim3 grid((g.N + 31) / 32, g.ksplit, (g.M + 31) / 32);
    const int ksl = g.K / g.ksplit;
    switch (epi) {
        case DEPI_PARTIAL:
            if (ksl <= 256) hipLaunchKernelGGL((dec_gemm_kernel<DEPI_PARTIAL, 256>), grid, dim3(256), 0, s, g);
            else if (ksl <= 512) hipLaunchKernelGGL((dec_gemm_kernel<DEPI_PARTIAL, 512>), grid, dim3(256), 0, s, g);
            else if (ksl <= 640) hipLaunchKernelGGL((dec_gemm_kernel<DEPI_PARTIAL, 640>), grid, dim3(256), 0, s, g);
            else if (ksl <= 1024) hipLaunchKernelGGL((dec_gemm_kernel<DEPI_PARTIAL, 1024>), grid, dim3(256), 0, s, g);
            else hipLaunchKernelGGL((dec_gemm_kernel<DEPI_PARTIAL, MZ_DEC_KSLICE>), grid, dim3(256), 0, s, g);
            break;
        case DEPI_GELU_F16:
            hipLaunchKernelGGL((dec_gemm_kernel<DEPI_GELU_F16, MZ_DEC_KSLICE>), grid, dim3(256), 0, s, g);
            break;
        case DEPI_F16: hipLaunchKernelGGL((dec_gemm_kernel<DEPI_F16, MZ_DEC_KSLICE>), grid, dim3(256), 0, s, g); break;
        case DEPI_LOGITS: {
            const int T = mz_lm_tiles_per_block(g.N);
            hipLaunchKernelGGL(dec_lmhead_kernel, dim3(mz_lm_blocks(g.N), (g.M + 31) / 32), dim3(256), 0, s, g, T);
            break;
        }
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t mz_dec_attn_launch(hipStream_t s, const MzDecAttn& a) {
    if (a.maxT <= 0 || a.B <= 0 || a.nh <= 0 || a.L > MZ_TPAD || (a.L <= 0 && a.maxT > MZ_TPAD)) return hipErrorInvalidValue;
    if (a.aslot && (!a.align || a.na <= 0 || (a.L > 0 && a.L != MZ_TENC))) return hipErrorInvalidValue;
    // the fused query projection: cross-attention only, whole 64-half chunks per lane group, the row in LDS
    // (and at least one whole first batch of keys, L >= 256, which the kernel requests without a range check)
    if (a.wq && (a.L < 32 * 8 || !a.xin || a.d % 64 != 0 || a.d > MZ_DEC_KSLICE)) return hipErrorInvalidValue;
    // two instances (the query projection compiled only into the cross one), also told apart by name in traces
    if (a.L > 0)
        hipLaunchKernelGGL((dec_attn_kernel<32, 8, true>), dim3(a.B * a.nh), dim3(32 * 8), 0, s, a);
    else
        hipLaunchKernelGGL((dec_attn_kernel<32, 8, false>), dim3(a.B * a.nh), dim3(32 * 8), 0, s, a);
    return hipGetLastError();
}

hipError_t mz_dec_cross_launch(hipStream_t s, const MzDecCross& a) {
    if (a.maxT <= 0 || a.B <= 0 || a.nh <= 0 || a.d % 64 != 0 || a.d > MZ_DEC_KSLICE || a.d != a.nh * MZ_HD || !a.xin ||
        !a.wq)
        return hipErrorInvalidValue;
    if (a.aslot && (!a.align || a.na <= 0)) return hipErrorInvalidValue;
    if (a.B * a.nh <= 256) {  // one workgroup per CU, all at once
        hipLaunchKernelGGL(dec_cross_wide_kernel, dim3(a.B * a.nh), dim3(256), 0, s, a);
        return hipGetLastError();
    }
    MzDecAttn c{};
    c.qbias = a.qbias;
    c.xin = a.xin;
    c.wq = a.wq;
    c.k = a.k;
    c.v = a.v;
    c.kv_b = a.kv_b;
    c.kv_h = a.kv_h;
    c.L = MZ_TENC;
    c.ctr = a.ctr;
    c.done = a.done;
    c.out = a.out;
    c.B = a.B;
    c.nh = a.nh;
    c.d = a.d;
    c.maxT = a.maxT;
    c.aslot = a.aslot;
    c.align = a.align;
    c.alignh = a.alignh;
    c.na = a.na;
    return mz_dec_attn_launch(s, c);
}

static int row_threads(int dim) { return (dim / 4 + 63) / 64 * 64; }

hipError_t mz_dec_add_ln_launch(hipStream_t s, const float* xin, float* x, const float* parts, int nparts,
                                long part_stride, const f16* bias, const f16* w, const f16* b, f16* y, int rows,
                                int dim, float eps) {
    if (dim % 4 != 0 || dim > 2048 || rows <= 0 || nparts < 0 || nparts > MZ_MAX_PARTS) return hipErrorInvalidValue;
    // one wave per row for the decoder width of large-v3 and large-v3-turbo with its five split-K partials
    if (dim == 1280 && nparts == 5) {
        hipLaunchKernelGGL((dec_add_ln_wave_kernel<5, 5>), dim3(rows), dim3(64), 0, s, xin, x, parts, part_stride, bias,
                           w, b, y, eps);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(dec_add_ln_kernel, dim3(rows), dim3(row_threads(dim)), 0, s, xin, x, parts, nparts, part_stride,
                       bias, w, b, y, dim, eps);
    return hipGetLastError();
}

hipError_t mz_dec_embed_ln_launch(hipStream_t s, const int* tok, int* ctr, const f16* emb, const f16* pe, float* x,
                                  const f16* w, const f16* b, f16* y, int rows, int dim, int maxT, float eps) {
    if (dim % 4 != 0 || dim > 2048 || rows <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dec_embed_ln_kernel, dim3(rows), dim3(row_threads(dim)), 0, s, tok, ctr, emb, pe, x, w, b, y, dim,
                       maxT, eps);
    return hipGetLastError();
}

hipError_t mz_dec_argmax_launch(hipStream_t s, const int2* amax, int nblk, int* tok, int* done, int* ctr, int B,
                                int maxT, int prompt_len, int eos) {
    if (B <= 0 || nblk <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dec_argmax_kernel, dim3(B), dim3(64), 0, s, amax, nblk, tok, done, ctr, B, maxT, prompt_len,
                       eos);
    return hipGetLastError();
}
