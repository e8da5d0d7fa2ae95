// Row LayerNorm kernels over the fp32 residual stream, and the log-mel layout change for the conv stem.
// LayerNorm follows kernels/whisper.cu:48-82 (two-pass fp32 statistics, eps 1e-5, biased variance) with one wave64
// per row: the row is held in registers (dim / 256 float4 per lane), so it is read from HBM once.
#include "mz_common.h"
#include "mz_kernels.h"

namespace {

constexpr int MAXC = 8;  // float4 chunks per lane: dim <= 2048

// LayerNorm of one row held as v[i] = x[4 (lane + 64 i) .. + 4] (chunks past dim / 4 hold zeros and are not
// stored), written to y as fp16. Two-pass statistics (mean, then the centred second moment) as the reference. The
// kernels request gamma and beta (ln_params) together with the row, so they cost no round trip of their own.
__device__ __forceinline__ void ln_params(int nc, int lane, const f16* __restrict__ w, const f16* __restrict__ b,
                                          f16x4 (&wv)[MAXC], f16x4 (&bv)[MAXC]) {
#pragma unroll
    for (int i = 0; i < MAXC; i++)
        if (lane + 64 * i < nc) {
            wv[i] = *(const f16x4*)(w + (lane + 64 * i) * 4);
            bv[i] = *(const f16x4*)(b + (lane + 64 * i) * 4);
        }
}
__device__ __forceinline__ void ln_store_wb(const float4 (&v)[MAXC], int nc, int lane, const f16x4 (&wv)[MAXC],
                                            const f16x4 (&bv)[MAXC], f16* __restrict__ y, int dim, float eps) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < MAXC; i++)
        if (lane + 64 * i < nc) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    const float mean = wave_sum(s) / dim;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < MAXC; i++)
        if (lane + 64 * i < nc) {
            const float a = v[i].x - mean, c = v[i].y - mean, e = v[i].z - mean, f = v[i].w - mean;
            q += (a * a + c * c) + (e * e + f * f);
        }
    const float rstd = rsqrtf(wave_sum(q) / dim + eps);
#pragma unroll
    for (int i = 0; i < MAXC; i++)
        if (lane + 64 * i < nc) {
            const int idx = (lane + 64 * i) * 4;
            const f16x4 o = {(f16)((v[i].x - mean) * rstd * (float)wv[i][0] + (float)bv[i][0]),
                             (f16)((v[i].y - mean) * rstd * (float)wv[i][1] + (float)bv[i][1]),
                             (f16)((v[i].z - mean) * rstd * (float)wv[i][2] + (float)bv[i][2]),
                             (f16)((v[i].w - mean) * rstd * (float)wv[i][3] + (float)bv[i][3])};
            __builtin_nontemporal_store(o, (f16x4*)(y + idx));
        }
}

// one wave per row, 4 rows per workgroup; every load of the row is issued before the reductions
__global__ void __launch_bounds__(256) ln_kernel(const float* __restrict__ x, long ldx, const f16* __restrict__ w,
                                                 const f16* __restrict__ b, f16* __restrict__ y, long ldy, int rows,
                                                 int dim, float eps) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int nc = dim / 4;
    const float* xr = x + (long)row * ldx;
    float4 v[MAXC];
    f16x4 wv[MAXC], bv[MAXC];
    ln_params(nc, lane, w, b, wv, bv);
#pragma unroll
    for (int i = 0; i < MAXC; i++) v[i] = lane + 64 * i < nc ? *(const float4*)(xr + (lane + 64 * i) * 4) : float4{};
    ln_store_wb(v, nc, lane, wv, bv, y + (long)row * ldy, dim, eps);
}

// x[r] += d[r] (fp16) in place, then y[r] = LN(x[r])
__global__ void __launch_bounds__(256) add_ln_kernel(float* __restrict__ x, const f16* __restrict__ d,
                                                     const f16* __restrict__ w, const f16* __restrict__ b,
                                                     f16* __restrict__ y, int rows, int dim, float eps) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int nc = dim / 4;
    float* xr = x + (long)row * dim;
    const f16* dr = d + (long)row * dim;
    float4 v[MAXC];
    f16x4 dv[MAXC], wv[MAXC], bv[MAXC];
    ln_params(nc, lane, w, b, wv, bv);  // gamma and beta in flight with the row, not a round trip after it
    // the residual and the delta are streamed once: nontemporal loads and stores
#pragma unroll
    for (int i = 0; i < MAXC; i++) {
        const bool on = lane + 64 * i < nc;
        const f32x4 t = on ? __builtin_nontemporal_load((const f32x4*)(xr + (lane + 64 * i) * 4)) : f32x4{};
        v[i] = float4{t[0], t[1], t[2], t[3]};
        dv[i] = on ? __builtin_nontemporal_load((const f16x4*)(dr + (lane + 64 * i) * 4)) : f16x4{};
    }
#pragma unroll
    for (int i = 0; i < MAXC; i++)
        if (lane + 64 * i < nc) {
            v[i].x += (float)dv[i][0];
            v[i].y += (float)dv[i][1];
            v[i].z += (float)dv[i][2];
            v[i].w += (float)dv[i][3];
            __builtin_nontemporal_store(f32x4{v[i].x, v[i].y, v[i].z, v[i].w}, (f32x4*)(xr + (lane + 64 * i) * 4));
        }
    ln_store_wb(v, nc, lane, wv, bv, y + (long)row * dim, dim, eps);
}

// mel f32 [G][nm][3000] -> f16 [G][3000][nm], 64 x 64 tiles through LDS
__global__ void __launch_bounds__(256) mel_t_kernel(const float* mel, f16* melT, int nm) {
    __shared__ float t[64][65];
    const int g = blockIdx.z, c0 = blockIdx.y * 64, t0 = blockIdx.x * 64;
    const float* src = mel + (long)g * nm * MZ_NFR;
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
        int c = i >> 6, tt = i & 63;
        t[c][tt] = (c0 + c < nm && t0 + tt < MZ_NFR) ? src[(long)(c0 + c) * MZ_NFR + t0 + tt] : 0.f;
    }
    __syncthreads();
    f16* dst = melT + (long)g * MZ_NFR * nm;
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
        int tt = i >> 6, c = i & 63;
        if (c0 + c < nm && t0 + tt < MZ_NFR) dst[(long)(t0 + tt) * nm + c0 + c] = (f16)t[c][tt];
    }
}

}  // namespace

hipError_t mz_layernorm_launch(hipStream_t s, const float* x, long ldx, const f16* w, const f16* b, f16* y, long ldy,
                               int rows, int dim, float eps) {
    if (dim % 4 != 0 || dim > 256 * MAXC || rows <= 0 || ldx % 4 != 0 || ldy % 4 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(ln_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, ldx, w, b, y, ldy, rows, dim, eps);
    return hipGetLastError();
}

hipError_t mz_add_layernorm_launch(hipStream_t s, float* x, const f16* d, const f16* w, const f16* b, f16* y, int rows,
                                   int dim, float eps) {
    if (dim % 4 != 0 || dim > 256 * MAXC || rows <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(add_ln_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, d, w, b, y, rows, dim, eps);
    return hipGetLastError();
}

hipError_t mz_mel_transpose_launch(hipStream_t s, const float* mel, f16* melT, int G, int nm) {
    if (G <= 0 || nm <= 0) return hipErrorInvalidValue;
    dim3 grid((MZ_NFR + 63) / 64, (nm + 63) / 64, G);
    hipLaunchKernelGGL(mel_t_kernel, grid, dim3(256), 0, s, mel, melT, nm);
    return hipGetLastError();
}
