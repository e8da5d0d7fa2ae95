// Shared device-side definitions for the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define MZ_HD 64      // head size of every Whisper model
#define MZ_TENC 1500  // encoder positions (30 s)
#define MZ_TPAD 1536  // encoder positions padded to a multiple of 64 in every per-head buffer
#define MZ_NFR 3000   // log-mel frames (30 s)

// Wave64 matrix-core products. The operand k-order inside a lane is arbitrary as long as both operands use the same
// one; rows/columns follow the CDNA3/CDNA4 layouts: 32x32: operand lane l holds row (l % 32) and 8 k values chosen by
// l / 32; accumulator element r of lane l is (row 8 * (r / 4) + 4 * (l / 32) + r % 4, column l % 32).
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
// 16x16: operand lane l holds row (l % 16) and 8 k values chosen by l / 16; accumulator element r of lane l is
// (row 4 * (l / 16) + r, column l % 16).
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// Exact (erf) GELU, as nn.GELU(): 0.5 v (1 + erf(v / sqrt 2)). erff is the ROCm device library's.
__device__ __forceinline__ float gelu_erf(float v) { return 0.5f * v * (1.f + erff(v * 0.70710678118654752f)); }

__device__ __forceinline__ f16x8 ld8(const f16* p) { return *(const f16x8*)p; }
__device__ __forceinline__ void st4(f16* p, float a, float b, float c, float d) {
    f16x4 v = {(f16)a, (f16)b, (f16)c, (f16)d};
    *(f16x4*)p = v;
}
