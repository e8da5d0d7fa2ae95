// Token timestamps on the device: the alignment heads' cross-attention rows of every clip -> per-column z-scores ->
// median filter over time -> mean over heads -> dynamic time warping -> the time of each token's first frame.
// Follows src/align.rs:8-106 (transformers' _extract_token_timestamps) and computes exactly what the host routine
// mz_jump_times computes: the column statistics are accumulated in row order (in float with the fp16 roundings, as
// src/align.rs:18-23 does, or in double without them), every binary16 round trip is a round-to-nearest-even
// conversion, the DTW cost cells are (float)(-(double)s + (double)c), and contraction into fused multiply-adds is
// off, so both give identical bits.
//
// Three launches per batch of clips:
//   ts_stats_kernel  one thread per (clip, head, column) (ts_stats4_kernel: four adjacent columns per thread): mean
//                    and population standard deviation over the rows
//   ts_cost_kernel   one workgroup per 32 x 64 tile of (row, column): median of the width-w reflect-padded window
//                    of z-scores, summed over heads; the cells are stored in anti-diagonal-major order
//                    [d = i + j][i], so that the DTW reads each diagonal with consecutive addresses
//   ts_dtw_wave_kernel  tables of at most 256 rows: one wave per clip, four rows per lane, the previous two
//                    anti-diagonals in registers and the moves packed in LDS, where one lane walks the path back
//   ts_dtw_kernel    larger tables: one workgroup per clip; the DTW table is filled one anti-diagonal per step (every
//                    cell of a diagonal depends only on the two previous diagonals, kept in LDS), the move taken into
//                    each cell goes to a trace in the same diagonal-major order, and one lane walks the path back.
#include <math.h>

#include <algorithm>
#include <mutex>

#include "../../include/mimizuku.h"
#include "mz_common.h"
#include "mz_internal.h"
#include "mz_kernels.h"

#pragma clang fp contract(off)

namespace {

__device__ __forceinline__ float rh(float x) { return (float)(f16)x; }

__device__ __forceinline__ void cswap(float& a, float& b) {
    const float lo = a < b ? a : b, hi = a < b ? b : a;
    a = lo;
    b = hi;
}

// the middle of 7 values (the order statistic is the same whatever network computes it)
__device__ __forceinline__ float median7(float* a) {
    cswap(a[0], a[6]), cswap(a[2], a[3]), cswap(a[4], a[5]);
    cswap(a[0], a[2]), cswap(a[1], a[4]), cswap(a[3], a[6]);
    cswap(a[0], a[1]), cswap(a[2], a[5]), cswap(a[3], a[4]);
    cswap(a[1], a[2]), cswap(a[4], a[6]);
    cswap(a[2], a[3]), cswap(a[4], a[5]);
    cswap(a[1], a[2]), cswap(a[3], a[4]), cswap(a[5], a[6]);
    return a[3];
}

__global__ void __launch_bounds__(256) ts_stats_kernel(const MzTs p) {
    const int c = blockIdx.z, a = blockIdx.y, j = blockIdx.x * 256 + threadIdx.x;
    const int R = p.rc[c].x, C = p.rc[c].y;
    if (j >= C || R <= 0) return;
    const float* w = p.w + c * p.clip_stride + (long)a * p.cols_full + j;
    const long rs = (long)p.heads * p.cols_full;
    float mu, sd;
    if (p.half) {
        float sum = 0.f;
        for (int i = 0; i < R; i++) sum += w[i * rs];
        const float mean = sum / (float)R;
        float sq = 0.f;
        for (int i = 0; i < R; i++) {
            const float dv = w[i * rs] - mean;
            sq += dv * dv;
        }
        mu = rh(mean);
        sd = rh(__builtin_sqrtf(sq / (float)R));
    } else {
        double sum = 0.0;
        for (int i = 0; i < R; i++) sum += (double)w[i * rs];
        const float mean = (float)(sum / R);
        double sq = 0.0;
        for (int i = 0; i < R; i++) {
            const double dv = (double)(w[i * rs] - mean);
            sq += dv * dv;
        }
        mu = mean;
        sd = __builtin_sqrtf((float)(sq / R));
    }
    const long o = ((long)c * p.heads + a) * p.cols_full + j;
    p.mean[o] = mu;
    p.sd[o] = sd;
}

// The same statistics for four adjacent columns per thread through 16-byte loads (each column's sums in row order,
// exactly as above): for rows whose column count and clip stride are multiples of 4 at a 16-byte aligned base
// (every engine batch: 1500 columns). Columns past C are summed (their reads stay inside the row) but not stored.
__global__ void __launch_bounds__(256) ts_stats4_kernel(const MzTs p) {
    const int c = blockIdx.z, a = blockIdx.y, j = (blockIdx.x * 256 + threadIdx.x) * 4;
    const int R = p.rc[c].x, C = p.rc[c].y;
    if (j >= C || R <= 0) return;
    const float4* w = (const float4*)(p.w + c * p.clip_stride + (long)a * p.cols_full + j);
    const long rs = (long)p.heads * p.cols_full / 4;
    float mu[4], sd[4];
    if (p.half) {
        float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll 4
        for (int i = 0; i < R; i++) {
            const float4 v = w[i * rs];
            s0 += v.x;
            s1 += v.y;
            s2 += v.z;
            s3 += v.w;
        }
        const float m0 = s0 / (float)R, m1 = s1 / (float)R, m2 = s2 / (float)R, m3 = s3 / (float)R;
        float q0 = 0.f, q1 = 0.f, q2 = 0.f, q3 = 0.f;
#pragma unroll 4
        for (int i = 0; i < R; i++) {
            const float4 v = w[i * rs];
            const float d0 = v.x - m0, d1 = v.y - m1, d2 = v.z - m2, d3 = v.w - m3;
            q0 += d0 * d0;
            q1 += d1 * d1;
            q2 += d2 * d2;
            q3 += d3 * d3;
        }
        mu[0] = rh(m0), mu[1] = rh(m1), mu[2] = rh(m2), mu[3] = rh(m3);
        sd[0] = rh(__builtin_sqrtf(q0 / (float)R)), sd[1] = rh(__builtin_sqrtf(q1 / (float)R));
        sd[2] = rh(__builtin_sqrtf(q2 / (float)R)), sd[3] = rh(__builtin_sqrtf(q3 / (float)R));
    } else {
        double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
#pragma unroll 4
        for (int i = 0; i < R; i++) {
            const float4 v = w[i * rs];
            s0 += (double)v.x;
            s1 += (double)v.y;
            s2 += (double)v.z;
            s3 += (double)v.w;
        }
        const float m0 = (float)(s0 / R), m1 = (float)(s1 / R), m2 = (float)(s2 / R), m3 = (float)(s3 / R);
        double q0 = 0.0, q1 = 0.0, q2 = 0.0, q3 = 0.0;
#pragma unroll 4
        for (int i = 0; i < R; i++) {
            const float4 v = w[i * rs];
            const double d0 = (double)(v.x - m0), d1 = (double)(v.y - m1), d2 = (double)(v.z - m2),
                         d3 = (double)(v.w - m3);
            q0 += d0 * d0;
            q1 += d1 * d1;
            q2 += d2 * d2;
            q3 += d3 * d3;
        }
        mu[0] = m0, mu[1] = m1, mu[2] = m2, mu[3] = m3;
        sd[0] = __builtin_sqrtf((float)(q0 / R)), sd[1] = __builtin_sqrtf((float)(q1 / R));
        sd[2] = __builtin_sqrtf((float)(q2 / R)), sd[3] = __builtin_sqrtf((float)(q3 / R));
    }
    const long o = ((long)c * p.heads + a) * p.cols_full + j;
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (j + e < C) {
            p.mean[o + e] = mu[e];
            p.sd[o + e] = sd[e];
        }
}

// One workgroup per tile of COST_RT rows x COST_CT columns of a clip. Per head, the tile's z-scores (with the window's
// reflect-padded halo) are computed once into LDS; each cell takes the median of its window from there, summed over
// heads in head order. The tile's cells then leave diagonal by diagonal: the cells of one anti-diagonal within the
// tile are consecutive rows, so each diagonal's run is one contiguous store. W = 7: the window unrolled into registers
// (a sorting network); W = 0: any odd width up to MZ_TS_MAX_WIDTH (insertion sort).
constexpr int COST_RT = 32, COST_CT = 64, COST_HALO = MZ_TS_MAX_WIDTH - 1;

template <int W>
__global__ void __launch_bounds__(256) ts_cost_kernel(const MzTs p) {
    __shared__ float zt[COST_RT][COST_CT + COST_HALO + 1];
    __shared__ float val[COST_RT][COST_CT + 2];  // row stride 66: a diagonal's 32 rows fall in 32 different banks
    const int c = blockIdx.z, i0 = blockIdx.y * COST_RT, j0 = blockIdx.x * COST_CT, tid = threadIdx.x;
    const int R = p.rc[c].x, C = p.rc[c].y;
    if (i0 >= R || j0 >= C) return;
    const int width = W ? W : p.width, pad = width >> 1, span = COST_CT + 2 * pad;
    // the median phase: column jl = tid % 64 of rows il = tid / 64 + 4 k
    const int jl = tid & 63, ib = tid >> 6;
    float acc[COST_RT / 4];
#pragma unroll
    for (int k = 0; k < COST_RT / 4; k++) acc[k] = 0.f;
    for (int a = 0; a < p.heads; a++) {
        const float* mu = p.mean + ((long)c * p.heads + a) * p.cols_full;
        const float* sd = p.sd + ((long)c * p.heads + a) * p.cols_full;
        // z of tile column cl - pad (reflected into 0 .. C - 1 as the window reads it; columns of cells past C,
        // whose values are never stored, are clamped into range instead)
        for (int e = tid; e < COST_RT * span; e += 256) {
            const int il = e / span, cl = e - il * span, i = i0 + il;
            int t = j0 + cl - pad;
            if (t < 0) t = -t;
            if (t >= C) t = 2 * (C - 1) - t;
            t = t < 0 ? 0 : t > C - 1 ? C - 1 : t;
            float z = 0.f;
            if (i < R) {
                const float x = p.w[c * p.clip_stride + ((long)i * p.heads + a) * p.cols_full + t];
                const float sv = sd[t];
                if (sv > 0.f) z = p.half ? rh(rh(x - mu[t]) / sv) : (x - mu[t]) / sv;
            }
            zt[il][cl] = z;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < COST_RT / 4; k++) {
            const float* zr = &zt[ib + 4 * k][jl];
            if (C <= pad) {
                acc[k] += zr[pad];  // fewer columns than the half width: no filter
            } else if (W == 7) {
                float win[7];
#pragma unroll
                for (int q = 0; q < 7; q++) win[q] = zr[q];
                acc[k] += median7(win);
            } else {
                float win[MZ_TS_MAX_WIDTH];
                for (int q = 0; q < width; q++) {
                    const float v = zr[q];
                    int r = q - 1;
                    while (r >= 0 && win[r] > v) {
                        win[r + 1] = win[r];
                        r--;
                    }
                    win[r + 1] = v;
                }
                acc[k] += win[pad];
            }
        }
        __syncthreads();  // zt is rewritten for the next head
    }
#pragma unroll
    for (int k = 0; k < COST_RT / 4; k++) {
        float v = acc[k] / (float)p.heads;
        if (p.half) v = rh(v);
        val[ib + 4 * k][jl] = v;
    }
    __syncthreads();
    // DTW cell (i + 1, j + 1) lies on anti-diagonal i + j + 2: tile diagonal dl = il + jl holds rows il of one run
    float* dst = p.cost + c * p.diag_stride + (long)(i0 + j0 + 2) * p.ldd + (i0 + 1);
    const int il = tid & 31;
    for (int dl = tid >> 5; dl < COST_RT + COST_CT - 1; dl += 8) {
        const int cl = dl - il;
        if (cl >= 0 && cl < COST_CT && i0 + il < R && j0 + cl < C) dst[(long)dl * p.ldd + il] = val[il][cl];
    }
}

// One workgroup per clip. Row i of the table (0..R) is handled by threads i, i + blockDim, ... The costs are staged
// in LDS DTW_CH diagonals at a time (diagonal-major, so a chunk is one contiguous run, copied with direct-to-LDS
// loads) while the previous chunk is being used; within a chunk a diagonal waits only for the LDS traffic of the
// one before (lds_barrier), so the trace stores and the next chunk's loads stay in flight.
constexpr int DTW_CH = 12;

__global__ void __launch_bounds__(1024) ts_dtw_kernel(const MzTs p) {
#if defined(__HIP_DEVICE_COMPILE__)  // the buffer-resource type exists only in the device pass
    extern __shared__ float lds[];
    const int c = blockIdx.x, R = p.rc[c].x, C = p.rc[c].y, nt = blockDim.x, tid = threadIdx.x;
    float* out = p.out + (long)c * p.out_stride;
    if (R <= 0) return;
    if (C <= 0) {
        for (int k = tid; k < R; k += nt) out[k] = 0.f;
        return;
    }
    const int ld = p.ldd;
    float* diag = lds;                       // 3 x (R + 1): diagonals d, d - 1, d - 2 in rotation
    int* first = (int*)(lds + 3 * ld);       // per row: the column of the path's first cell in that row
    float* chunk = lds + 4 * ld;             // 2 x DTW_CH diagonals of costs
    const float* cost = p.cost + c * p.diag_stride;
    signed char* tr = p.trace + c * p.diag_stride;
    // reads past the clip's cost table return zeros (the descriptor's range check)
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(cost), (short)0,
                                                                         (int)(p.diag_stride * 4), 0x00020000);
    // a chunk buffer holds a whole number of 64-float wave copies (the last one may read past the chunk)
    const int lane = tid & 63, wave = tid >> 6, per = (DTW_CH * ld + 63) & ~63;
    auto stage = [&](int d0, float* dst) {
        // wave w's lanes copy floats w * 64 + lane, + nt, ... of diagonals d0 .. d0 + DTW_CH - 1
        for (int k = wave * 64; k < per; k += nt)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, (__attribute__((address_space(3))) void*)(dst + k), 4,
                                                     (unsigned)((d0 * ld + k + lane) * 4), 0, 0, 0);
    };
    stage(0, chunk);
    for (int d0 = 0; d0 <= R + C; d0 += DTW_CH) {
        float* cb = chunk + ((d0 / DTW_CH) & 1) * per;
        __builtin_amdgcn_s_waitcnt(0);  // this chunk's copies (and the trace stores so far) are done
        __syncthreads();                // ... in every wave, and the other buffer's last chunk is no longer read
        if (d0 + DTW_CH <= R + C) stage(d0 + DTW_CH, chunk + (((d0 / DTW_CH) + 1) & 1) * per);
        const int dend = min(d0 + DTW_CH, R + C + 1);
        for (int d = d0; d < dend; d++) {
            float* cur = diag + (d % 3) * ld;
            const float* p1 = diag + ((d + 2) % 3) * ld;
            const float* p2 = diag + ((d + 1) % 3) * ld;
            const float* cd = cb + (d - d0) * ld;
            const int lo = max(0, d - C), hi = min(R, d);
            for (int i = lo + tid; i <= hi; i += nt) {
                const int j = d - i;
                float v;
                signed char t;
                if (i == 0) {
                    v = d == 0 ? 0.f : INFINITY;
                    t = 2;
                } else if (j == 0) {
                    v = INFINITY;
                    t = 1;
                } else {
                    const float c0 = p2[i - 1], c1 = p1[i - 1], c2 = p1[i];
                    float m;
                    if (c0 < c1 && c0 < c2) {
                        m = c0;
                        t = 0;
                    } else if (c1 < c0 && c1 < c2) {
                        m = c1;
                        t = 1;
                    } else {
                        m = c2;
                        t = 2;
                    }
                    v = (float)(-(double)cd[i] + (double)m);
                }
                cur[i] = v;
                tr[(long)d * ld + i] = t;
            }
            lds_barrier();
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    // the trace stores went to global memory from every lane: make them visible to the walking lane
    __threadfence_block();
    __syncthreads();
    if (tid == 0) {
        int i = R, j = C;
        bool row0 = false;
        while (i > 0 || j > 0) {
            first[i] = j - 1;
            row0 |= i == 0;
            const signed char t = tr[(long)(i + j) * ld + i];
            if (t == 0) {
                i--;
                j--;
            } else if (t == 1) {
                i--;
            } else {
                j--;
            }
        }
        // the token rows start at text index -1 when the path ran along row 0, else at 0; one start per row
        const int r0 = row0 ? 0 : 1;
        for (int n = 0; n < R; n++) out[n] = (float)((double)first[r0 + n] * 0.02);
    }
#endif
}

// Tables of at most 256 rows (R <= 255): one wave per clip. Lane l holds table rows 4l .. 4l + 3 of the two
// previous anti-diagonals in registers and takes row 4l - 1 from lane l - 1 through cross-lane moves, so a diagonal
// needs no barrier and no LDS round trip; its costs arrive four per lane, one 16-byte load per lane for the whole
// diagonal, DTW_PF diagonals ahead. The move into each cell (2 bits) is packed into LDS ([diagonal][lane], a byte
// per lane), where the path is walked back. Same comparisons and results as ts_dtw_kernel, so the same bits.
constexpr int DTW_PF = 16;
constexpr int DTW_WAVE_ND = 256 + 1500;  // diagonals of a table: rows 0 .. 255, columns 0 .. 1500

// lane l gets lane l - 1's v (lane 0: 0): a row shift within each 16-lane row (DPP row_shr:1), and the first lane of
// rows 1 .. 3 takes the last lane of the row before through lane reads merged in with per-lane bit masks (made once
// by the caller). Bitwise merges, not selects: the compiler turns a select between lane reads into branches.
struct LaneMasks {
    int keep, m16, m32, m48;  // all ones where the lane keeps the row shift / is lane 16, 32, 48
};
__device__ __forceinline__ float lane_prev(float v, const LaneMasks& k) {
    const int x = __builtin_bit_cast(int, v);
    int y = __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false) & k.keep;
    y |= __builtin_amdgcn_readlane(x, 15) & k.m16;
    y |= __builtin_amdgcn_readlane(x, 31) & k.m32;
    y |= __builtin_amdgcn_readlane(x, 47) & k.m48;
    return __builtin_bit_cast(float, y);
}

__global__ void __launch_bounds__(64) ts_dtw_wave_kernel(const MzTs p) {
#if defined(__HIP_DEVICE_COMPILE__)
    __shared__ unsigned char moves[(DTW_WAVE_ND + DTW_PF) * 64];  // [diagonal][lane], whole rounds of DTW_PF
    __shared__ int first[257];                         // per row; [R + 1]: the first token row's offset
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const int c = blockIdx.x, R = p.rc[c].x, C = p.rc[c].y, lane = threadIdx.x;
    float* out = p.out + (long)c * p.out_stride;
    if (R <= 0) return;
    if (C <= 0) {
        for (int k = lane; k < R; k += 64) out[k] = 0.f;
        return;
    }
    const int ld = p.ldd, nd = R + C + 1;
    // reads past the clip's cost table return zeros (the descriptor's range check); rows past R are never used
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.cost + c * p.diag_stride), (short)0, (int)(p.diag_stride * 4), 0x00020000);
    auto load = [&](int d) {
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, (unsigned)((d * ld + 4 * lane) * 4),
                                                                                0, 0));
    };
    u32x4 ring[DTW_PF];
#pragma unroll
    for (int k = 0; k < DTW_PF; k++) ring[k] = load(k);
    float D1[4], D2[4];  // diagonals d - 1 and d - 2 of rows 4 lane + r
#pragma unroll
    for (int r = 0; r < 4; r++) D1[r] = D2[r] = INFINITY;
    // Every cell of a diagonal is computed, in or out of the table: a cell outside (row past R, column past C or
    // below 0) feeds only cells outside, and the walk back reads moves of cells inside only, forcing the edges' moves
    // itself, so no cell needs a range test and the choice is branch free. Row 0 is 0 at (0, 0) and +inf after;
    // column 0 (i == d) is +inf. The moves of rows 4 lane .. 4 lane + 3 pack into one byte.
    float up2 = INFINITY;  // lane_prev of diagonal d - 2's row 4 lane + 3, carried from the diagonal before
    const bool lane0 = lane == 0;
    const int m16 = -(lane == 16), m32 = -(lane == 32), m48 = -(lane == 48);
    const LaneMasks lm{~(m16 | m32 | m48), m16, m32, m48};
    // whole rounds of DTW_PF diagonals: the ones past the table are outside cells too
    const int ndr = (nd + DTW_PF - 1) / DTW_PF * DTW_PF;
    for (int d0 = 0; d0 < ndr; d0 += DTW_PF) {
#pragma unroll
        for (int k = 0; k < DTW_PF; k++) {
            const int d = d0 + k;
            const u32x4 cw = ring[k];
            ring[k] = load(d + DTW_PF);
            const float up1 = lane_prev(D1[3], lm);  // row 4 lane - 1 at d - 1 (lane 0: unused)
            float nv[4];
            unsigned bits = 0;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float c0 = r ? D2[r - 1] : up2, c1 = r ? D1[r - 1] : up1, c2 = D1[r];
                // the reference's comparisons as written (align.rs:77-83), so a NaN cost (a NaN or infinite
                // z-score in half mode) picks the same move as the host routine and ts_dtw_kernel: fminf would
                // drop the NaN operand
                const bool t0 = (c0 < c1) & (c0 < c2), t1 = (c1 < c0) & (c1 < c2);
                const float m = t0 ? c0 : t1 ? c1 : c2;
                // ts_dtw_kernel's fp64 -x + m rounded to fp32 equals the fp32 m - x: a sum rounded first to 53 bits
                // and then to 24 rounds as if once, since 53 >= 2 x 24 + 2 (Figueroa, 1995)
                float v = m - __uint_as_float(cw[r]);
                v = 4 * lane + r == d ? INFINITY : v;
                if (r == 0) v = lane0 ? (d == 0 ? 0.f : INFINITY) : v;
                nv[r] = v;
                bits |= (t0 ? 0u : t1 ? 1u : 2u) << (2 * r);
            }
            up2 = up1;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                D2[r] = D1[r];
                D1[r] = nv[r];
            }
            moves[d * 64 + lane] = (unsigned char)bits;
        }
    }
    __syncthreads();
    if (lane == 0) {
        // at most R + C moves from (R, C) to (0, 0); row 0 moves left and column 0 up, as the table's edges do
        int i = R, j = C;
        bool row0 = false;
        for (int n = 0; n < R + C && (i > 0 || j > 0); n++) {
            first[i] = j - 1;
            row0 |= i == 0;
            unsigned t = (moves[(i + j) * 64 + (i >> 2)] >> (2 * (i & 3))) & 3u;
            if (i == 0) t = 2;
            else if (j == 0) t = 1;
            if (t == 0) {
                i--;
                j--;
            } else if (t == 1) {
                i--;
            } else {
                j--;
            }
        }
        // the token rows start at text index -1 when the path ran along row 0, else at 0
        first[R + 1] = row0 ? 0 : 1;
    }
    __syncthreads();
    const int r0 = first[R + 1];  // one start per row
#pragma unroll 1
    for (int n = lane; n < R; n += 64) out[n] = (float)((double)first[r0 + n] * 0.02);
#endif
}

}  // namespace

// 3 diagonals, the first-column table and 2 chunks of DTW_CH diagonals of costs, ld = rmax + 1 floats each
size_t mz_ts_lds_bytes(int rmax) { return ((size_t)(rmax + 1) * 4 + 2 * (((size_t)DTW_CH * (rmax + 1) + 63) & ~(size_t)63)) * 4; }

hipError_t mz_ts_launch(hipStream_t s, const MzTs& p, int n) {
    if (n <= 0) return hipSuccess;
    if (p.width < 1 || p.width % 2 == 0 || p.width > MZ_TS_MAX_WIDTH || p.heads <= 0 || p.rmax < 0 ||
        p.ldd < p.rmax + 1 || p.cols_full <= 0)
        return hipErrorInvalidValue;
    if (p.cols_full % 4 == 0 && p.clip_stride % 4 == 0 && ((uintptr_t)p.w & 15) == 0) {
        const dim3 gs((p.cols_full / 4 + 255) / 256, p.heads, n);
        hipLaunchKernelGGL(ts_stats4_kernel, gs, dim3(256), 0, s, p);
    } else {
        const dim3 gs((p.cols_full + 255) / 256, p.heads, n);
        hipLaunchKernelGGL(ts_stats_kernel, gs, dim3(256), 0, s, p);
    }
    if (p.rmax > 0) {
        const dim3 gc((p.cols_full + COST_CT - 1) / COST_CT, (p.rmax + COST_RT - 1) / COST_RT, n);
        if (p.width == 7)
            hipLaunchKernelGGL(ts_cost_kernel<7>, gc, dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL(ts_cost_kernel<0>, gc, dim3(256), 0, s, p);
    }
    // the wave kernel loads rows 4 lane .. 4 lane + 3 of a diagonal as one aligned 16-byte group: ldd % 4 == 0
    if (p.rmax <= 255 && p.ldd % 4 == 0 && p.rmax + p.cols_full + 1 <= DTW_WAVE_ND && p.diag_stride * 4 < (1L << 31)) {
        hipLaunchKernelGGL(ts_dtw_wave_kernel, dim3(n), dim3(64), 0, s, p);
        return hipGetLastError();
    }
    int nt = ((p.rmax + 1 + 63) / 64) * 64;
    nt = nt < 256 ? 256 : nt > 1024 ? 1024 : nt;
    if (mz_ts_lds_bytes(p.ldd - 1) > 64 * 1024 || p.diag_stride * 4 >= (1L << 31)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(ts_dtw_kernel, dim3(n), dim3(nt), mz_ts_lds_bytes(p.ldd - 1), s, p);
    return hipGetLastError();
}

// ------------------------------------------------------------------ the entry point that allocates nothing

// Scratch of mz_jump_times_device_noalloc: a file-scope device array, one copy per GPU the library runs on, held until
// the process ends. In host code `scratch` names a host-side stand-in, never a device address: its address on each
// device comes from hipGetSymbolAddress (mz_ts_scratch_setup, called by mz_init with that device current) and only
// that address is passed to kernels and copies.
static __device__ __align__(256) unsigned char scratch[MZ_TS_SCRATCH_BYTES];

namespace {
constexpr int MZ_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch[MZ_MAX_DEVICES] = {};
// held by a call of mz_jump_times_device_noalloc for its whole use of that device's array
std::mutex g_scratch_use[MZ_MAX_DEVICES];
size_t up256(size_t n) { return (n + 255) & ~(size_t)255; }
}  // namespace

int mz_ts_scratch_setup(int device) {
    if (device < 0 || device >= MZ_MAX_DEVICES) return mz_fail(MZ_ERR_ARG, "device %d: at most %d devices", device, MZ_MAX_DEVICES);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[device]) return MZ_OK;
    int cur = -1;
    if (int r = mz_hip(hipGetDevice(&cur), "hipGetDevice")) return r;
    if (cur != device) return mz_fail(MZ_ERR_STATE, "timestamp scratch set-up: device %d is not current (%d)", device, cur);
    void* ptr = nullptr;
    if (int r = mz_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return r;
    if (!ptr) return mz_fail(MZ_ERR_HIP, "hipGetSymbolAddress(scratch) gave a null address");
    g_scratch[device] = ptr;
    return MZ_OK;
}

extern "C" int mz_jump_times_device_noalloc(mz_ctx* c, uint64_t w, int64_t clip_stride, int n, const int32_t* rows,
                                            const int32_t* cols, int heads, int cols_full, int width, int half,
                                            float* out, int64_t out_stride) {
    if (!c || !w || !rows || !cols || !out || n < 0 || heads <= 0 || cols_full <= 0 || clip_stride < 0)
        return mz_fail(MZ_ERR_ARG, "mz_jump_times_device_noalloc: bad argument");
    if (width < 1 || width % 2 == 0 || width > MZ_TS_MAX_WIDTH)
        return mz_fail(MZ_ERR_ARG, "mz_jump_times_device_noalloc: width %d (odd, at most %d)", width, MZ_TS_MAX_WIDTH);
    for (int i = 0; i < n; i++)
        if (rows[i] < 0 || cols[i] < 0 || cols[i] > cols_full || rows[i] > 4095 || rows[i] > out_stride)
            return mz_fail(MZ_ERR_ARG, "mz_jump_times_device_noalloc: clip %d has %d rows, %d columns", i, rows[i],
                           cols[i]);
    if (n == 0) return MZ_OK;
    if (int r = mz_hip(hipSetDevice(c->device), "hipSetDevice")) return r;
    if (int r = mz_ts_scratch_setup(c->device)) return r;
    unsigned char* base;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        base = (unsigned char*)g_scratch[c->device];
    }
    // the array is this device's only copy: calls from other threads (or contexts) on the same GPU wait until this
    // one's results are on the host (every chunk below ends with a synchronisation of the stream)
    std::lock_guard<std::mutex> use(g_scratch_use[c->device]);
    // scratch of k clips whose longest has rmax rows: (rows, columns), column statistics, DTW cost and trace, times
    auto need = [&](int k, int rmax) {
        return up256((size_t)k * sizeof(int2)) + 2 * up256((size_t)k * heads * cols_full * 4) +
               up256((size_t)k * mz_ts_diag_stride(rmax, cols_full) * 5) + up256((size_t)k * out_stride * 4);
    };
    // the clips go through the array in chunks of at most MZ_TS_NOALLOC_CHUNK that fit in it, one after the other
    int2 rc[MZ_TS_NOALLOC_CHUNK];
    for (int c0 = 0; c0 < n;) {
        int k = 0, rmax = 0;
        while (c0 + k < n && k < MZ_TS_NOALLOC_CHUNK && need(k + 1, std::max(rmax, (int)rows[c0 + k])) <= MZ_TS_SCRATCH_BYTES) {
            rmax = std::max(rmax, (int)rows[c0 + k]);
            k++;
        }
        if (k == 0)
            return mz_fail(MZ_ERR_ARG,
                           "mz_jump_times_device_noalloc: clip %d (%d rows, %d heads x %d columns) needs %zu bytes of "
                           "scratch; the static scratch holds %u",
                           c0, rows[c0], heads, cols_full, need(1, rows[c0]), (unsigned)MZ_TS_SCRATCH_BYTES);
        for (int i = 0; i < k; i++) rc[i] = int2{rows[c0 + i], cols[c0 + i]};
        const long ds = mz_ts_diag_stride(rmax, cols_full);
        unsigned char* q = base;
        auto carve = [&](size_t bytes) {
            unsigned char* r = q;
            q += up256(bytes);
            return r;
        };
        MzTs p{};
        p.w = (const float*)(uintptr_t)w + (size_t)c0 * clip_stride;
        p.clip_stride = clip_stride;
        p.heads = heads;
        p.cols_full = cols_full;
        p.width = width;
        p.half = half;
        p.rmax = rmax;
        p.rc = (const int2*)carve((size_t)k * sizeof(int2));
        p.mean = (float*)carve((size_t)k * heads * cols_full * 4);
        p.sd = (float*)carve((size_t)k * heads * cols_full * 4);
        p.cost = (float*)carve((size_t)k * ds * 5);
        p.trace = (signed char*)(p.cost + (size_t)k * ds);
        p.diag_stride = ds;
        p.ldd = mz_ts_ldd(rmax);
        p.out = (float*)carve((size_t)k * out_stride * 4);
        p.out_stride = out_stride;
        int r = mz_hip(hipMemcpyAsync((void*)p.rc, rc, (size_t)k * sizeof(int2), hipMemcpyHostToDevice, c->stream),
                       "upload");
        if (!r) r = mz_hip(mz_ts_launch(c->stream, p, k), "timestamp kernels");
        for (int i = 0; i < k && !r; i++)
            if (rows[c0 + i] > 0)
                r = mz_hip(hipMemcpyAsync(out + (size_t)(c0 + i) * out_stride, p.out + (size_t)i * out_stride,
                                          (size_t)rows[c0 + i] * 4, hipMemcpyDeviceToHost, c->stream),
                           "download");
        // the next chunk reuses the array (and rc): wait for this one
        if (!r) r = mz_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        if (r) return r;
        c0 += k;
    }
    return MZ_OK;
}
