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
// Vector work hides only in part under the matrix cores (a wave's own vector instructions overlap about two thirds
// of their time with its independent products, the other wave of the SIMD covers more), so every vector instruction
// per score counts: the running max is set by the first block and later blocks compute no max at all; a block is recomputed against its own max (and O
// rescaled) only when the sum of its probabilities reaches 2^12, i.e. some p = exp2(s - m) could leave the range
// where fp16 holds it exactly enough; the probabilities are rounded two per packed conversion and summed two per
// dot2 instruction, and the key mask of the padded last tile is applied in that tile only.
#include <type_traits>

#include "mz_common.h"
#include "mz_kernels.h"

namespace {

constexpr int KP = 72;  // LDS row pitch in halves (144 B): conflict-free 16-byte fragment reads
constexpr int QB = 256; // queries per block
constexpr int NT = MZ_TPAD / 64;  // key tiles (the last one holds keys 1472..1535, valid < 1500)

__device__ __forceinline__ int swap23(int x) { return (x & ~12) | ((x & 4) << 1) | ((x & 8) >> 1); }

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float block_max(const f32x16& sc) {
    float mx = fmaxf(fmaxf(sc[0], sc[1]), sc[2]);
#pragma unroll
    for (int r = 3; r < 15; r += 2) mx = fmaxf(fmaxf(mx, sc[r]), sc[r + 1]);
    return fmaxf(mx, sc[15]);
}

// p = exp2(sc) (the scores already in log2 units and relative to the running max) rounded to fp16 two at a time (one
// packed conversion per pair, each pair one dword of the P.V operand), and the sum of the rounded values (the ones
// that weight V) through dot2 in fp32
__device__ __forceinline__ float probs(const f32x16& sc, unsigned (&pw)[2][4]) {
    float lb = 0.f;
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
        const f32x2 e = {__builtin_amdgcn_exp2f(sc[r]), __builtin_amdgcn_exp2f(sc[r + 1])};
        const f16x2 h = __builtin_convertvector(e, f16x2);
        lb = __builtin_amdgcn_fdot2(h, f16x2{1, 1}, lb, false);
        pw[r >> 3][(r & 7) >> 1] = __builtin_bit_cast(unsigned, h);
    }
    return lb;
}

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

    // query fragments (B operand of S^T): query row, dims 16c + 8 lh .. + 8; the QKV product stores q multiplied by
    // log2(e) / 8, so the products are the scores in log2 units
    const int q0 = qb * QB + wave * 64;
    f16x8 qf[2][4];
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int c = 0; c < 4; c++) qf[s][c] = ld8(Q + (long)(q0 + s * 32 + lr) * MZ_HD + 16 * c + 8 * lh);

    // this thread's two K chunks and two V^T chunks of a tile: buffer loads with a fixed per-lane offset and the tile
    // step in the scalar offset (no address arithmetic per tile; every offset lies within the padded head block)
    const int c0 = tid, c1 = tid + 256;
    const int kr0 = c0 >> 3, kr1 = c1 >> 3, cc = (tid & 7) * 8;
    const __amdgpu_buffer_rsrc_t rK = rsrc(K, MZ_TPAD * MZ_HD * 2), rV = rsrc(Vt, MZ_HD * MZ_TPAD * 2);
    const unsigned ok0 = (kr0 * MZ_HD + cc) * 2, ok1 = (kr1 * MZ_HD + cc) * 2;
    const unsigned ov0 = (kr0 * MZ_TPAD + cc) * 2, ov1 = (kr1 * MZ_TPAD + cc) * 2;
    f16x8 pk0, pk1, pv0, pv1;
    auto gload = [&](int kt) {
        const int sk = kt * 64 * MZ_HD * 2, sv = kt * 64 * 2;
        pk0 = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rK, ok0, sk, 0));
        pk1 = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rK, ok1, sk, 0));
        pv0 = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rV, ov0, sv, 0));
        pv1 = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rV, ov1, sv, 0));
    };
    auto lstore = [&](int buf) {
        *(f16x8*)&sK[buf][swap23(kr0) * KP + cc] = pk0;
        *(f16x8*)&sK[buf][swap23(kr1) * KP + cc] = pk1;
        *(f16x8*)&sV[buf][kr0 * KP + cc] = pv0;
        *(f16x8*)&sV[buf][kr1 * KP + cc] = pv1;
    };

    // running max of the scores (per query column), set by the first block, kept as -m in all 16 elements of the C
    // input of each block's first product: the scores come out of the matrix core relative to it
    float m[2] = {0.f, 0.f};
    f32x16 cm[2] = {f32x16{}, f32x16{}};
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
                f32x16 sc = mfma32(kf[0], qf[qs][0], cm[qs]);
#pragma unroll
                for (int c = 1; c < 4; c++) sc = mfma32(kf[c], qf[qs][c], sc);
                if (LAST) {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int key = kt * 64 + 32 * ss + 16 * (r >> 3) + 8 * lh + (r & 7);
                        if (key >= MZ_TENC) sc[r] = -INFINITY;
                    }
                }
                // the first block sets the running max (l and o are still zero)
                const bool first = kt == 0 && ss == 0;
                if (first) {
                    m[qs] = pair32_max(block_max(sc));
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        sc[r] -= m[qs];
                        cm[qs][r] = -m[qs];
                    }
                }
                unsigned pw[2][4];
                float lb = probs(sc, pw);
                // later blocks raise it only when their probabilities get large: a block sum of 2^12 or more (some
                // score more than 8 above the running max, or an fp16 overflow) recomputes the block against its
                // own max; below that every probability is < 2^12, exact enough in fp16 (wave-uniform branch)
                if (!first && __ballot(!(lb < 4096.f))) {
                    const float mx = pair32_max(block_max(sc));
                    const float dm = mx > 0.f ? mx : 0.f;
                    const float corr = __builtin_amdgcn_exp2f(-dm);
                    m[qs] += dm;
                    l[qs] *= corr;
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        sc[r] -= dm;
                        cm[qs][r] = -m[qs];
                    }
#pragma unroll
                    for (int t = 0; t < 2; t++)
#pragma unroll
                        for (int r = 0; r < 16; r++) o[qs][t][r] *= corr;
                    lb = probs(sc, pw);
                }
                l[qs] += lb;
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (int c = 0; c < 2; c++)
                        o[qs][t] = mfma32(vf[t][c], __builtin_bit_cast(f16x8, u32x4{pw[c][0], pw[c][1], pw[c][2], pw[c][3]}),
                                          o[qs][t]);
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
