// Tiled fp16 GEMM on the gfx950 matrix cores for the encoder-sized products (M = clips x 1500 or x 3000):
// QKV (head-major scatter), out-proj and fc2 (residual add into the fp32 stream), fc1 (GELU), the conv stem as an
// implicit GEMM (no im2col buffer), and the cross-attention K/V of every decoder layer. Replaces the reference's
// cuBLAS calls with a bias prefill (src/gpu.rs:208-236, 254-286; kernels/whisper.cu:92-104, 106-139).
//
// Block tile BM x BN x 64 with 4 waves in a 2 x 2 grid; each wave owns a (BM/2) x (BN/2) tile of 32x32x16 MFMA
// products. Both operands are K-contiguous, staged through LDS with an XOR swizzle of the 16-byte chunks (conflict
// free ds_read_b128 for the operand fragments), double buffered with register prefetch of the next K tile.
// The W tile is the MFMA A operand and the activation tile the B operand, so a lane's accumulators hold one token
// row and 4-wide runs of output columns: epilogues store 8-byte runs, and transposed (V) stores are coalesced
// across lanes.
#include "mz_common.h"
#include "mz_kernels.h"

namespace {

template <int BM, int BN>
struct Tile {
    static constexpr int WM = BM / 2, WN = BN / 2;
    static constexpr int TM = WM / 32, TN = WN / 32;
    static constexpr int AL = BM * 8 / 256;  // 16-byte chunks of the A tile per thread per K tile
    static constexpr int WL = BN * 8 / 256;
};

// Map the launch index to a tile so that the blocks one XCD receives (block i runs on XCD i % 8) form a contiguous
// run of tiles, ordered with N fastest: concurrently resident blocks of an XCD share activation rows in its L2.
__device__ __forceinline__ int xcd_tile(int bid, int nblocks) {
    int per = nblocks >> 3;
    return (bid & 7) * per + (bid >> 3);
}

template <int BM, int BN, int ALOAD, int EPI>
__global__ void __launch_bounds__(256) gemm_kernel(const MzGemm p) {
    using T = Tile<BM, BN>;
    __shared__ __attribute__((aligned(16))) f16 sA[2][BM * 64];
    __shared__ __attribute__((aligned(16))) f16 sW[2][BN * 64];

    const int nbn = (p.N + BN - 1) / BN, nbm = (p.M + BM - 1) / BM;
    const int tile = xcd_tile(blockIdx.x, gridDim.x);
    if (tile >= nbm * nbn) return;
    const int bm = tile / nbn, bn = tile % nbn;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, lh = lane >> 5;
    const int nk = p.K >> 6;
    const int chunk = tid & 7;

    // global sources of this thread's chunks
    const f16* gW[T::WL];
#pragma unroll
    for (int r = 0; r < T::WL; r++) {
        int row = min(bn * BN + (tid >> 3) + 32 * r, p.N - 1);
        gW[r] = p.W + (long)row * p.K + chunk * 8;
    }
    const f16* gA[T::AL];
    int cg[T::AL], ct[T::AL];  // conv: clip and output time of the row
#pragma unroll
    for (int r = 0; r < T::AL; r++) {
        int row = min(bm * BM + (tid >> 3) + 32 * r, p.M - 1);
        if (ALOAD == ALOAD_PLAIN) {
            gA[r] = p.A + (long)row * p.lda + chunk * 8;
        } else {
            cg[r] = row / p.conv_tout;
            ct[r] = row - cg[r] * p.conv_tout;
            gA[r] = p.A;
        }
    }

    f16x8 ra[T::AL], rw[T::WL];
    auto gload = [&](int kt) {
#pragma unroll
        for (int r = 0; r < T::WL; r++) rw[r] = ld8(gW[r] + kt * 64);
        if (ALOAD == ALOAD_PLAIN) {
#pragma unroll
            for (int r = 0; r < T::AL; r++) ra[r] = ld8(gA[r] + kt * 64);
        } else {
            int k0 = kt * 64 + chunk * 8;
            int tap = k0 / p.conv_cin, ci = k0 - tap * p.conv_cin;
#pragma unroll
            for (int r = 0; r < T::AL; r++) {
                int tt = p.conv_stride * ct[r] + tap - 1;
                bool ok = tap < 3 && tt >= 0 && tt < p.conv_tin;
                f16x8 z = {};
                ra[r] = ok ? ld8(p.A + ((long)cg[r] * p.conv_tin + tt) * p.conv_cin + ci) : z;
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int r = 0; r < T::AL; r++) {
            int row = (tid >> 3) + 32 * r;
            *(f16x8*)&sA[buf][row * 64 + ((chunk ^ (row & 7)) << 3)] = ra[r];
        }
#pragma unroll
        for (int r = 0; r < T::WL; r++) {
            int row = (tid >> 3) + 32 * r;
            *(f16x8*)&sW[buf][row * 64 + ((chunk ^ (row & 7)) << 3)] = rw[r];
        }
    };

    f32x16 acc[T::TM][T::TN];
#pragma unroll
    for (int i = 0; i < T::TM; i++)
#pragma unroll
        for (int j = 0; j < T::TN; j++) acc[i][j] = f32x16{};

    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const int sw = (((2 * kk + lh) ^ (lr & 7)) << 3);
            f16x8 fa[T::TM], fw[T::TN];
#pragma unroll
            for (int i = 0; i < T::TM; i++) fa[i] = *(const f16x8*)&sA[buf][(wm * T::WM + i * 32 + lr) * 64 + sw];
#pragma unroll
            for (int j = 0; j < T::TN; j++) fw[j] = *(const f16x8*)&sW[buf][(wn * T::WN + j * 32 + lr) * 64 + sw];
#pragma unroll
            for (int i = 0; i < T::TM; i++)
#pragma unroll
                for (int j = 0; j < T::TN; j++) acc[i][j] = mfma32(fw[j], fa[i], acc[i][j]);
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

    // epilogue: lane holds row m and columns n0 + {0..3} for each (i, j, q)
#pragma unroll
    for (int i = 0; i < T::TM; i++) {
        const int m = bm * BM + wm * T::WM + i * 32 + lr;
        if (m >= p.M) continue;
#pragma unroll
        for (int j = 0; j < T::TN; j++) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int n = bn * BN + wn * T::WN + j * 32 + 8 * q + 4 * lh;
                if (n >= p.N) continue;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = acc[i][j][4 * q + e] + (p.bias ? (float)p.bias[n + e] : 0.f);
                if (EPI == EPI_F16) {
                    st4((f16*)p.out + (long)m * p.ldo + n, v[0], v[1], v[2], v[3]);
                } else if (EPI == EPI_GELU_F16) {
                    st4((f16*)p.out + (long)m * p.ldo + n, gelu_erf(v[0]), gelu_erf(v[1]), gelu_erf(v[2]),
                        gelu_erf(v[3]));
                } else if (EPI == EPI_RESID_F32) {
                    float4* o = (float4*)((float*)p.out + (long)m * p.ldo + n);
                    float4 r = *o;
                    r.x += v[0];
                    r.y += v[1];
                    r.z += v[2];
                    r.w += v[3];
                    *o = r;
                } else if (EPI == EPI_GELU_POS) {
                    const f16* ps = p.pos + (long)(m % MZ_TENC) * p.N + n;
                    float4 r;
                    r.x = gelu_erf(v[0]) + (float)ps[0];
                    r.y = gelu_erf(v[1]) + (float)ps[1];
                    r.z = gelu_erf(v[2]) + (float)ps[2];
                    r.w = gelu_erf(v[3]) + (float)ps[3];
                    *(float4*)((float*)p.out + (long)m * p.ldo + n) = r;
                } else if (EPI == EPI_HEADS) {
                    const int g = m / MZ_TENC, t = m - g * MZ_TENC;
                    const int blk = n >> 6, dim = n & 63;
                    f16* base = p.heads + ((long)(p.slot0 + g) * p.blocks_per_clip + blk) * (MZ_TPAD * MZ_HD);
                    if (p.kind == 3 && blk / p.nh == 2) {  // encoder v: transposed for the P.V product
#pragma unroll
                        for (int e = 0; e < 4; e++) base[(long)(dim + e) * MZ_TPAD + t] = (f16)v[e];
                    } else {
                        st4(base + (long)t * MZ_HD + dim, v[0], v[1], v[2], v[3]);
                    }
                }
            }
        }
    }
}

template <int BM, int BN, int ALOAD, int EPI>
hipError_t launch(hipStream_t s, const MzGemm& g) {
    int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
    int grid = (tiles + 7) & ~7;
    hipLaunchKernelGGL((gemm_kernel<BM, BN, ALOAD, EPI>), dim3(grid), dim3(256), 0, s, g);
    return hipGetLastError();
}

template <int ALOAD, int EPI>
hipError_t pick(hipStream_t s, const MzGemm& g) {
    // 256 x 256 tiles once there are enough of them to fill 256 CUs; 256 x 128 (or 128 x 128) below that
    long t256 = (long)((g.M + 255) / 256) * ((g.N + 255) / 256);
    if (t256 >= 512) return launch<256, 256, ALOAD, EPI>(s, g);
    long t128 = (long)((g.M + 255) / 256) * ((g.N + 127) / 128);
    if (t128 >= 256) return launch<256, 128, ALOAD, EPI>(s, g);
    return launch<128, 128, ALOAD, EPI>(s, g);
}

}  // namespace

hipError_t mz_gemm_launch(hipStream_t s, int aload, int epi, const MzGemm& g) {
    if (g.K % 64 != 0 || g.M <= 0 || g.N <= 0 || g.K <= 0 || g.N % 4 != 0) return hipErrorInvalidValue;
    if (epi == EPI_HEADS && g.N % 64 != 0) return hipErrorInvalidValue;
    if (aload == ALOAD_CONV) {
        if (g.conv_cin % 8 != 0 || g.conv_tout <= 0) return hipErrorInvalidValue;
        if (epi == EPI_GELU_F16) return pick<ALOAD_CONV, EPI_GELU_F16>(s, g);
        if (epi == EPI_GELU_POS) return pick<ALOAD_CONV, EPI_GELU_POS>(s, g);
        return hipErrorInvalidValue;
    }
    switch (epi) {
        case EPI_F16: return pick<ALOAD_PLAIN, EPI_F16>(s, g);
        case EPI_GELU_F16: return pick<ALOAD_PLAIN, EPI_GELU_F16>(s, g);
        case EPI_RESID_F32: return pick<ALOAD_PLAIN, EPI_RESID_F32>(s, g);
        case EPI_HEADS: return pick<ALOAD_PLAIN, EPI_HEADS>(s, g);
    }
    return hipErrorInvalidValue;
}
