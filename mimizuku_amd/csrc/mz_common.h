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

// Cross-lane moves through DPP: a vector-ALU operand modifier of a few cycles, where __shfl_xor becomes an LDS
// permute (a round trip through the LDS pipeline). Controls (GCN / CDNA): quad_perm [1,0,3,2] = 0xB1 (lane ^ 1),
// [2,3,0,1] = 0x4E (lane ^ 2), row_half_mirror = 0x141 (lane i of 8 reads 7 - i), row_mirror = 0x140 (lane i of 16
// reads 15 - i). Every lane of the groups involved must be active.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}
// sum over each aligned group of 8 lanes, in every lane of the group
__device__ __forceinline__ float group8_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    return v + dpp_f<0x141>(v);
}
// sum / max over the wave, in every lane: 16-lane rows through DPP, then the four row values through lane reads
__device__ __forceinline__ float wave_sum(float v) {
    v = group8_sum(v);
    v += dpp_f<0x140>(v);
    const int b = __builtin_bit_cast(int, v);
    return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
           (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    const int b = __builtin_bit_cast(int, v);
    return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)),
                       __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))),
                 fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)),
                       __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48))));
}
// lanes i and i ^ 32 combined, in both: v_permlane32_swap with both operands v returns (low half, high half) of v in
// every lane, so no selection by lane is needed
__device__ __forceinline__ float pair32_max(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ __forceinline__ float pair32_sum(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}
// (value, index) maximum over each aligned group of 8 lanes, ties to the lowest index, in every lane of the group
__device__ __forceinline__ void group8_argmax(float& best, int& bi) {
    auto step = [&](float ov, int oi) {
        if (ov > best || (ov == best && oi < bi)) {
            best = ov;
            bi = oi;
        }
    };
    step(dpp_f<0xB1>(best), dpp_i<0xB1>(bi));
    step(dpp_f<0x4E>(best), dpp_i<0x4E>(bi));
    step(dpp_f<0x141>(best), dpp_i<0x141>(bi));
}
// the same over the whole wave (every lane active), in every lane
__device__ __forceinline__ void wave_argmax(float& best, int& bi) {
    group8_argmax(best, bi);
    const float ov = dpp_f<0x140>(best);
    const int oi = dpp_i<0x140>(bi);
    if (ov > best || (ov == best && oi < bi)) {
        best = ov;
        bi = oi;
    }
    const int fb = __builtin_bit_cast(int, best);
    float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(fb, 0));
    int i = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16) {
        const float rv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(fb, r));
        const int ri = __builtin_amdgcn_readlane(bi, r);
        if (rv > b || (rv == b && ri < i)) {
            b = rv;
            i = ri;
        }
    }
    best = b;
    bi = i;
}

// Exact (erf) GELU, as nn.GELU(): 0.5 v (1 + erf(v / sqrt 2)), with erf from Abramowitz & Stegun 7.1.26 (Hastings'
// rational approximation, |error| <= 1.5e-7 on erf). With u = |v| / sqrt 2, t = 1 / (1 + p u) and
// h = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-u^2) / 2 = (1 - erf(u)) / 2, GELU(v) = v (1 - h) for v >= 0 and
// v h for v < 0, so the negative side has no cancellation (the halving is folded into the coefficients, p / sqrt 2
// into one constant). Both sides are max(v, 0) - |v| h: one fused multiply-add (|v| is an operand modifier) in place
// of a compare, a select, 1 - h and a product, rounded once. Against the exact GELU, over every finite fp16 input:
// correctly rounded except for 257 values in the tail where 1 - erf(u) is below ~1e-4, at most 1.28 fp16 ulp (at
// v = -4.08); the reference's own fp32 formula reaches 1.7 ulp there from the cancellation in 1 + erf(u).
__device__ __forceinline__ float gelu_erf(float v) {
    const float t = __builtin_amdgcn_rcpf(fmaf(fabsf(v), 0.3275911f * 0.70710678118654752f, 1.f));
    const float hp = t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, 0.5307027145f, -0.7265760135f), 0.7107068705f), -0.142248368f),
                              0.127414796f);
    const float h = hp * __builtin_amdgcn_exp2f(v * (v * (-0.5f * 1.4426950408889634f)));
    return fmaf(-fabsf(v), h, fmaxf(v, 0.f));
}

// Exact (erf) GELU for fp16 outputs, with one transcendental: GELU(v) = v Phi(v) = max(v, 0) - |v| Phi(-|v|), and
// log2 Phi(-a) for a = |v| as one degree-7 polynomial in a (a minimax fit on [0, 6], |error| <= 5.3e-6 with these
// fp32 coefficients, so Phi(-a) within 3.7e-6 relative), then exp2: 7 fused multiply-adds, one exp2, a max and a
// fused multiply-add, where gelu_erf needs a reciprocal and an exp2 besides. Past a = 6 the polynomial keeps falling
// (below -29.9, checked out to 70000), so the output rounds to v or to zero in fp16 there, as the exact GELU does.
// Against the exact GELU over every finite fp16 input (fp32 arithmetic emulated, exp2 correctly rounded or one ulp
// off either way): at most 0.505 fp16 ulp, 157-171 values not correctly rounded. Rounded to fp16 only: for fp32
// outputs gelu_erf is ~50x closer.
__device__ __forceinline__ float gelu_erf_h(float v) {
    const float a = fabsf(v);
    float p = fmaf(a, -1.83480927e-06f, 6.15982644e-05f);
    p = fmaf(p, a, -0.00093052478f);
    p = fmaf(p, a, 0.00850789156f);
    p = fmaf(p, a, -0.05396007f);
    p = fmaf(p, a, -0.458464384f);
    p = fmaf(p, a, -1.15125108f);
    p = fmaf(p, a, -0.999995291f);
    return fmaf(-a, __builtin_amdgcn_exp2f(p), fmaxf(v, 0.f));
}

// A workgroup barrier for LDS traffic only: waits for this wave's LDS operations (lgkmcnt(0)) but not for its
// global loads and stores, which __syncthreads would drain (its vmcnt(0)), so loads issued ahead stay in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt and expcnt unconstrained
    asm volatile("s_barrier" ::: "memory");
}

// A raw buffer resource over `bytes` bytes at base (stride 0, dword data format): loads at offsets past the end
// return zeros and stores there are dropped; the range check covers the per-lane offset, not the scalar one.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ f16x8 ld8(const f16* p) { return *(const f16x8*)p; }
__device__ __forceinline__ void st4(f16* p, float a, float b, float c, float d) {
    f16x4 v = {(f16)a, (f16)b, (f16)c, (f16)d};
    *(f16x4*)p = v;
}
