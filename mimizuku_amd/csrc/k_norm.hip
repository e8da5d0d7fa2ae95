// Row LayerNorm kernels over the fp32 residual stream, and the log-mel layout change for the conv stem.
// LayerNorm follows kernels/whisper.cu:48-82 (two-pass fp32 statistics, eps 1e-5, biased variance) with one wave64
// per row: the row is held in registers (dim / 128 float2 per lane), so it is read from HBM once.
#include "mz_common.h"
#include "mz_kernels.h"

namespace {

constexpr int MAXV = 16;  // float2 per lane: dim <= 2048

// LayerNorm of one row held as v[i] = x[(lane + 64 i) * 2 .. + 2], written to y as fp16.
__device__ __forceinline__ void ln_store(const float2 (&v)[MAXV], int nv, int lane, const f16* w, const f16* b, f16* y,
                                         int dim, float eps) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < MAXV; i++)
        if (i < nv) s += v[i].x + v[i].y;
    const float mean = wave_sum(s) / dim;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < MAXV; i++)
        if (i < nv) {
            float a = v[i].x - mean, c = v[i].y - mean;
            q += a * a + c * c;
        }
    const float rstd = rsqrtf(wave_sum(q) / dim + eps);
#pragma unroll
    for (int i = 0; i < MAXV; i++)
        if (i < nv) {
            int idx = (lane + 64 * i) * 2;
            f16x2 wv = *(const f16x2*)(w + idx), bv = *(const f16x2*)(b + idx);
            f16x2 o = {(f16)((v[i].x - mean) * rstd * (float)wv[0] + (float)bv[0]),
                       (f16)((v[i].y - mean) * rstd * (float)wv[1] + (float)bv[1])};
            *(f16x2*)(y + idx) = o;
        }
}

__global__ void __launch_bounds__(256) ln_kernel(const float* x, long ldx, const f16* w, const f16* b, f16* y, long ldy,
                                                 int rows, int dim, float eps) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int nv = dim / 128;
    const float* xr = x + (long)row * ldx;
    float2 v[MAXV];
#pragma unroll
    for (int i = 0; i < MAXV; i++)
        if (i < nv) v[i] = *(const float2*)(xr + (lane + 64 * i) * 2);
    ln_store(v, nv, lane, w, b, y + (long)row * ldy, dim, eps);
}

__global__ void __launch_bounds__(256) add_ln_kernel(float* x, const f16* d, const f16* w, const f16* b, f16* y,
                                                     int rows, int dim, float eps) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int nv = dim / 128;
    float* xr = x + (long)row * dim;
    const f16* dr = d + (long)row * dim;
    float2 v[MAXV];
#pragma unroll
    for (int i = 0; i < MAXV; i++)
        if (i < nv) {
            int idx = (lane + 64 * i) * 2;
            float2 a = *(const float2*)(xr + idx);
            f16x2 c = *(const f16x2*)(dr + idx);
            a.x += (float)c[0];
            a.y += (float)c[1];
            *(float2*)(xr + idx) = a;
            v[i] = a;
        }
    ln_store(v, nv, lane, w, b, y + (long)row * dim, dim, eps);
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
    if (dim % 128 != 0 || dim > 128 * MAXV || rows <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(ln_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, ldx, w, b, y, ldy, rows, dim, eps);
    return hipGetLastError();
}

hipError_t mz_add_layernorm_launch(hipStream_t s, float* x, const f16* d, const f16* w, const f16* b, f16* y, int rows,
                                   int dim, float eps) {
    if (dim % 128 != 0 || dim > 128 * MAXV || rows <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(add_ln_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, d, w, b, y, rows, dim, eps);
    return hipGetLastError();
}

hipError_t mz_mel_transpose_launch(hipStream_t s, const float* mel, f16* melT, int G, int nm) {
    if (G <= 0 || nm <= 0) return hipErrorInvalidValue;
    dim3 grid((MZ_NFR + 63) / 64, (nm + 63) / 64, G);
    hipLaunchKernelGGL(mel_t_kernel, grid, dim3(256), 0, s, mel, melT, nm);
    return hipGetLastError();
}
