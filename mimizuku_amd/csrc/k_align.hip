// Token timestamps on the device: the alignment heads' cross-attention rows of every clip -> per-column z-scores ->
// median filter over time -> mean over heads -> dynamic time warping -> the time of each token's first frame.
// Follows src/align.rs:8-106 (transformers' _extract_token_timestamps) and computes exactly what the host routine
// mz_jump_times computes: the column statistics are accumulated in row order (in float with the fp16 roundings, as
// src/align.rs:18-23 does, or in double without them), every binary16 round trip is a round-to-nearest-even
// conversion, the DTW cost cells are (float)(-(double)s + (double)c), and contraction into fused multiply-adds is
// off, so both give identical bits.
//
// Three launches per batch of clips:
//   ts_stats_kernel  one thread per (clip, head, column): mean and population standard deviation over the rows
//   ts_cost_kernel   one thread per (clip, row, column): median of the width-w reflect-padded window of z-scores,
//                    summed over heads; the cell is stored in anti-diagonal-major order [d = i + j][i], so that the
//                    DTW reads each diagonal with consecutive addresses
//   ts_dtw_kernel    one workgroup per clip: the DTW table is filled one anti-diagonal per step (every cell of a
//                    diagonal depends only on the two previous diagonals, kept in LDS), the move taken into each cell
//                    goes to a trace in the same diagonal-major order, and one lane walks the path back.
#include <math.h>

#include "mz_common.h"
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

// W = 7: the window unrolled into registers; W = 0: any odd width up to MZ_TS_MAX_WIDTH
template <int W>
__global__ void __launch_bounds__(256) ts_cost_kernel(const MzTs p) {
    const int c = blockIdx.z, i = blockIdx.y, j = blockIdx.x * 256 + threadIdx.x;
    const int R = p.rc[c].x, C = p.rc[c].y;
    if (i >= R || j >= C) return;
    const int width = W ? W : p.width, pad = width >> 1;
    float acc = 0.f;
    for (int a = 0; a < p.heads; a++) {
        const float* x = p.w + c * p.clip_stride + ((long)i * p.heads + a) * p.cols_full;
        const float* mu = p.mean + ((long)c * p.heads + a) * p.cols_full;
        const float* sd = p.sd + ((long)c * p.heads + a) * p.cols_full;
        auto z = [&](int t) {
            const float s = sd[t];
            if (!(s > 0.f)) return 0.f;
            return p.half ? rh(rh(x[t] - mu[t]) / s) : (x[t] - mu[t]) / s;
        };
        if (C <= pad) {
            acc += z(j);
            continue;
        }
        auto src = [&](int k) {
            int t = j + k - pad;
            if (t < 0) t = -t;
            if (t >= C) t = 2 * (C - 1) - t;
            return t;
        };
        if (W == 7) {
            float win[7];
#pragma unroll
            for (int k = 0; k < 7; k++) win[k] = z(src(k));
            acc += median7(win);
        } else {
            // insertion sort of the window, then its middle value
            float win[MZ_TS_MAX_WIDTH];
            for (int k = 0; k < width; k++) {
                const float v = z(src(k));
                int q = k - 1;
                while (q >= 0 && win[q] > v) {
                    win[q + 1] = win[q];
                    q--;
                }
                win[q + 1] = v;
            }
            acc += win[pad];
        }
    }
    float s = acc / (float)p.heads;
    if (p.half) s = rh(s);
    // DTW cell (i + 1, j + 1) lies on anti-diagonal i + j + 2
    p.cost[c * p.diag_stride + (long)(i + j + 2) * p.ldd + (i + 1)] = s;
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

}  // namespace

// 3 diagonals, the first-column table and 2 chunks of DTW_CH diagonals of costs, ld = rmax + 1 floats each
size_t mz_ts_lds_bytes(int rmax) { return ((size_t)(rmax + 1) * 4 + 2 * (((size_t)DTW_CH * (rmax + 1) + 63) & ~(size_t)63)) * 4; }

hipError_t mz_ts_launch(hipStream_t s, const MzTs& p, int n) {
    if (n <= 0) return hipSuccess;
    if (p.width < 1 || p.width % 2 == 0 || p.width > MZ_TS_MAX_WIDTH || p.heads <= 0 || p.rmax < 0 ||
        p.ldd < p.rmax + 1 || p.cols_full <= 0)
        return hipErrorInvalidValue;
    const dim3 gs((p.cols_full + 255) / 256, p.heads, n);
    hipLaunchKernelGGL(ts_stats_kernel, gs, dim3(256), 0, s, p);
    if (p.rmax > 0) {
        const dim3 gc((p.cols_full + 255) / 256, p.rmax, n);
        if (p.width == 7)
            hipLaunchKernelGGL(ts_cost_kernel<7>, gc, dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL(ts_cost_kernel<0>, gc, dim3(256), 0, s, p);
    }
    int nt = ((p.rmax + 1 + 63) / 64) * 64;
    nt = nt < 256 ? 256 : nt > 1024 ? 1024 : nt;
    if (mz_ts_lds_bytes(p.ldd - 1) > 64 * 1024 || p.diag_stride * 4 >= (1L << 31)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(ts_dtw_kernel, dim3(n), dim3(nt), mz_ts_lds_bytes(p.ldd - 1), s, p);
    return hipGetLastError();
}
