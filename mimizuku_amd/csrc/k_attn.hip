// Encoder self-attention for head_dim 64 on the gfx950 matrix cores (non-causal, 1500 keys, scale 1/8), replacing
// kernels/whisper.cu:168-299 (enc_flash). softmax(Q K^T / 8) V with fp32 scores and online softmax, P rounded to
// fp16 for the P.V product, O / l rounded to fp16 (the SDPA arithmetic the reference follows, whisper.cu:3-4).
//
// Work: one block per (256 queries, head, clip) = 4 waves x 2 sets of 32 queries. K and V^T tiles of 64 keys are
// staged in LDS (double buffered, register prefetch) and shared by the 4 waves. Scores are computed transposed,
// S^T = K Q^T (32x32x16 MFMA), so each lane owns one query column: the running max and the rescale of O are per
// lane, and the only cross-lane step is one swap with lane l ^ 32. K rows are stored in LDS with bits 2 and 3 of the
// key index swapped, which makes each lane's 16 scores two runs of 8 consecutive keys: the probabilities, rounded to
// fp16, are directly the B operand of O^T = V^T P^T, and V^T (written transposed by the QKV GEMM) is read with
// 16-byte LDS loads.
//
// On this part the vector ALU and the matrix cores of a SIMD do not overlap (an MFMA and the vector instructions
// around it take the sum of their times), so every vector instruction per score counts: the running max is raised
// only when a block's scores exceed it by more than 2^8 (p = exp2(s - m) <= 256 is exact enough in fp16 and keeps
// the rescale of O rare), the row sums add the fp16 probabilities two per dot2 instruction, and the key mask of the
// padded last tile is applied in that tile only.
#include <type_traits>

#include "mz_common.h"
#include "mz_kernels.h"

namespace {

constexpr int KP = 72;  // LDS row pitch in halves (144 B): conflict-free 16-byte fragment reads
constexpr int QB = 256; // queries per block
constexpr int NT = MZ_TPAD / 64;  // key tiles (the last one holds keys 1472..1535, valid < 1500)

__device__ __forceinline__ int swap23(int x) { return (x & ~12) | ((x & 4) << 1) | ((x & 8) >> 1); }

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) enc_attn_kernel(const f16* __restrict__ qkvh, f16* __restrict__ out, int nh, int G) {
    __shared__ __attribute__((aligned(16))) f16 sK[2][64 * KP];
    __shared__ __attribute__((aligned(16))) f16 sV[2][64 * KP];

    // workgroup i runs on XCD i % 8: XCD x takes (clip, head) pairs x, x + 8, ... and all six query blocks of a pair,
    // so a pair's K and V tiles are fetched into one L2 only
    const int xcd = blockIdx.x & 7, li = blockIdx.x >> 3, npq = (MZ_TENC + QB - 1) / QB;
    const int pair = (li / npq) * 8 + xcd, qb = li % npq;
    if (pair >= nh * G) return;
    const int head = pair % nh, g = pair / nh;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 31, lh = lane >> 5;
    const long blk = (long)MZ_TPAD * MZ_HD;
    const f16* Q = qkvh + ((long)g * 3 * nh + head) * blk;
    const f16* K = Q + (long)nh * blk;
    const f16* Vt = Q + 2L * nh * blk;
    const int d = nh * MZ_HD;

    // query fragments (B operand of S^T): query row, dims 16c + 8 lh .. + 8
    const float cs = 0.125f * 1.4426950408889634f;  // scale * log2(e)
    const int q0 = qb * QB + wave * 64;
    f16x8 qf[2][4];
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int c = 0; c < 4; c++) qf[s][c] = ld8(Q + (long)(q0 + s * 32 + lr) * MZ_HD + 16 * c + 8 * lh);

    // this thread's two K chunks and two V^T chunks of a tile
    const int c0 = tid, c1 = tid + 256;
    const int kr0 = c0 >> 3, kr1 = c1 >> 3, cc = (tid & 7) * 8;
    f16x8 pk0, pk1, pv0, pv1;
    auto gload = [&](int kt) {
        pk0 = ld8(K + (long)(kt * 64 + kr0) * MZ_HD + cc);
        pk1 = ld8(K + (long)(kt * 64 + kr1) * MZ_HD + cc);
        pv0 = ld8(Vt + (long)kr0 * MZ_TPAD + kt * 64 + cc);
        pv1 = ld8(Vt + (long)kr1 * MZ_TPAD + kt * 64 + cc);
    };
    auto lstore = [&](int buf) {
        *(f16x8*)&sK[buf][swap23(kr0) * KP + cc] = pk0;
        *(f16x8*)&sK[buf][swap23(kr1) * KP + cc] = pk1;
        *(f16x8*)&sV[buf][kr0 * KP + cc] = pv0;
        *(f16x8*)&sV[buf][kr1 * KP + cc] = pv1;
    };

    constexpr float TAU = 8.f;  // log2 of the largest unnormalised probability before O is rescaled
    float m[2] = {0.f, 0.f};    // running max of the scaled scores (per query column); set by the first block
    float l[2] = {0.f, 0.f};
    f32x16 o[2][2];
#pragma unroll
    for (int s = 0; s < 2; s++) o[s][0] = o[s][1] = f32x16{};

    gload(0);
    lstore(0);
    __syncthreads();
    // one 64-key tile; LAST masks the keys past 1500 of the padded last tile
    auto tile = [&](int kt, auto last) {
        constexpr bool LAST = decltype(last)::value;
        const int buf = kt & 1;
        if (!LAST) gload(kt + 1);
#pragma unroll
        for (int ss = 0; ss < 2; ss++) {  // 32-key halves of the tile
            f16x8 kf[4], vf[2][2];
#pragma unroll
            for (int c = 0; c < 4; c++) kf[c] = *(const f16x8*)&sK[buf][(32 * ss + lr) * KP + 16 * c + 8 * lh];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int c = 0; c < 2; c++)
                    vf[t][c] = *(const f16x8*)&sV[buf][(32 * t + lr) * KP + 32 * ss + 16 * c + 8 * lh];
#pragma unroll
            for (int qs = 0; qs < 2; qs++) {
                f32x16 sc = {};
#pragma unroll
                for (int c = 0; c < 4; c++) sc = mfma32(kf[c], qf[qs][c], sc);
                if (LAST) {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int key = kt * 64 + 32 * ss + 16 * (r >> 3) + 8 * lh + (r & 7);
                        if (key >= MZ_TENC) sc[r] = -INFINITY;
                    }
                }
                float mx = fmaxf(fmaxf(sc[0], sc[1]), sc[2]);
#pragma unroll
                for (int r = 3; r < 15; r += 2) mx = fmaxf(fmaxf(mx, sc[r]), sc[r + 1]);
                mx = fmaxf(mx, sc[15]);
                mx = pair32_max(mx) * cs - m[qs];  // block max over the running max
                // first block: the max becomes this block's max; later: raised only past TAU (wave-uniform branch)
                const bool first = kt == 0 && ss == 0;
                if (__ballot(first || mx > TAU)) {
                    const float dm = (first || mx > TAU) ? mx : 0.f;
                    const float corr = __builtin_amdgcn_exp2f(-dm);
                    m[qs] += dm;
                    l[qs] *= corr;
#pragma unroll
                    for (int t = 0; t < 2; t++)
#pragma unroll
                        for (int r = 0; r < 16; r++) o[qs][t][r] *= corr;
                }
                f16x8 pf[2];
#pragma unroll
                for (int r = 0; r < 16; r++) pf[r >> 3][r & 7] = (f16)__builtin_amdgcn_exp2f(fmaf(sc[r], cs, -m[qs]));
                // row sum of the fp16 probabilities (the ones that weight V), two per dot2 with fp32 accumulation
#pragma unroll
                for (int r = 0; r < 16; r += 2)
                    l[qs] = __builtin_amdgcn_fdot2(f16x2{pf[r >> 3][r & 7], pf[r >> 3][(r & 7) + 1]}, f16x2{1, 1}, l[qs],
                                                   false);
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (int c = 0; c < 2; c++) o[qs][t] = mfma32(vf[t][c], pf[c], o[qs][t]);
            }
        }
        if (!LAST) lstore(buf ^ 1);
        __syncthreads();
    };
    for (int kt = 0; kt < NT - 1; kt++) tile(kt, std::false_type{});
    tile(NT - 1, std::true_type{});

#pragma unroll
    for (int qs = 0; qs < 2; qs++) {
        const float lt = pair32_sum(l[qs]);
        const float inv = 1.f / lt;
        const int q = q0 + qs * 32 + lr;
        if (q >= MZ_TENC) continue;
        f16* dst = out + ((long)g * MZ_TENC + q) * d + head * MZ_HD;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) {
                const int dim = 32 * t + 8 * r4 + 4 * lh;
                st4(dst + dim, o[qs][t][4 * r4] * inv, o[qs][t][4 * r4 + 1] * inv, o[qs][t][4 * r4 + 2] * inv,
                    o[qs][t][4 * r4 + 3] * inv);
            }
    }
}

}  // namespace

hipError_t mz_enc_attention_launch(hipStream_t s, const f16* qkvh, f16* out, int G, int nh) {
    if (G <= 0 || nh <= 0) return hipErrorInvalidValue;
    // 1-D grid: 8 XCDs x ceil(pairs / 8) pairs x 6 query blocks
    const int npq = (MZ_TENC + QB - 1) / QB, pairs = G * nh;
    hipLaunchKernelGGL(enc_attn_kernel, dim3(8 * ((pairs + 7) / 8) * npq), dim3(256), 0, s, qkvh, out, nh, G);
    return hipGetLastError();
}
