// Decoder-step kernels (one greedy step for B rows; the position p = ctr[0] is read from device memory, so one
// captured graph replays every step — kernels/whisper.cu:7-8, 301-567). The step is HBM-bound: every kernel
// streams its operand once with 16-byte loads and keeps the arithmetic in registers.
//
//   dec_gemm   skinny GEMM for M <= 32 rows per tile on the matrix cores (W rows are the 32x32x16 MFMA A operand,
//              the x rows the B operand), split-K across blocks and across the 4 waves of a block; epilogues:
//              fp32 partials, GELU -> fp16, fp32 logits, or the self-attention q/k/v scatter into the cache
//              (replaces gemv_{1,2,4,8} + cuBLAS + fill_bias + kv_write, whisper.cu:92-97, 309-317, 497-567).
//   dec_attn   attention of one query per (row, head) over a key range: self-attention over the cache
//              (whisper.cu:319-353) and cross-attention over the encoder keys/values split in chunks whose
//              partial (max, sum, P.V) the last block of a (row, head) combines, recording the alignment-head
//              probabilities on the way (whisper.cu:355-449, three kernels there).
//   dec_add_ln residual add of the split-K partials + bias, fused with the next LayerNorm (whisper.cu:71-82).
//   dec_embed_ln  token + position embedding fused with the first LayerNorm (whisper.cu:303-307).
//   dec_argmax greedy choice with suppression; the last block advances the position (whisper.cu:451-495).
#include "mz_common.h"
#include "mz_kernels.h"

namespace {

constexpr int MAXV = 16;  // float2 per lane in the row kernels: dim <= 2048
constexpr int CHMAX = 512;  // keys per attention block

__device__ __forceinline__ float block_reduce_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}
__device__ __forceinline__ float block_reduce_max(float v, float* red) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// ---------------------------------------------------------------- skinny GEMM

template <int EPI>
__global__ void __launch_bounds__(256) dec_gemm_kernel(const MzDec p) {
    __shared__ float red[4][32][33];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 31, lh = lane >> 5;
    const int n0 = blockIdx.x * 32, ks = blockIdx.y, m0 = blockIdx.z * 32;
    const int groups = (p.K >> 6) / p.ksplit, gbeg = ks * groups;

    const f16* wr = p.W + (long)min(n0 + lr, p.N - 1) * p.K + lh * 32;
    const f16* xr = p.x + (long)min(m0 + lr, p.M - 1) * p.ldx + lh * 32;
    f32x16 acc = {};
    int gi = wave;
    for (; gi + 4 < groups; gi += 8) {  // two groups in flight per wave
        const int ga = (gbeg + gi) * 64, gb = (gbeg + gi + 4) * 64;
        f16x8 wa[4], xa[4], wb[4], xb[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            wa[c] = ld8(wr + ga + 8 * c);
            wb[c] = ld8(wr + gb + 8 * c);
            xa[c] = ld8(xr + ga + 8 * c);
            xb[c] = ld8(xr + gb + 8 * c);
        }
#pragma unroll
        for (int c = 0; c < 4; c++) acc = mfma32(wa[c], xa[c], acc);
#pragma unroll
        for (int c = 0; c < 4; c++) acc = mfma32(wb[c], xb[c], acc);
    }
    if (gi < groups) {
        const int ga = (gbeg + gi) * 64;
        f16x8 wa[4], xa[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            wa[c] = ld8(wr + ga + 8 * c);
            xa[c] = ld8(xr + ga + 8 * c);
        }
#pragma unroll
        for (int c = 0; c < 4; c++) acc = mfma32(wa[c], xa[c], acc);
    }
    // accumulator r: n = n0 + 8 (r / 4) + 4 lh + r % 4, m = m0 + lr
#pragma unroll
    for (int r = 0; r < 16; r++) red[wave][8 * (r >> 2) + 4 * lh + (r & 3)][lr] = acc[r];
    __syncthreads();
    const int ml = tid >> 3, nl = (tid & 7) * 4;
    const int m = m0 + ml;
    if (m >= p.M) return;
    int pos = 0;
    if (EPI == DEPI_QKV) pos = p.ctr[0];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int n = n0 + nl + e;
        if (n >= p.N) continue;
        float v = red[0][nl + e][ml] + red[1][nl + e][ml] + red[2][nl + e][ml] + red[3][nl + e][ml];
        if (EPI == DEPI_PARTIAL) {
            ((float*)p.out)[((long)ks * p.M + m) * p.ldo + n] = v;
            continue;
        }
        if (p.bias) v += (float)p.bias[n];
        if (EPI == DEPI_GELU_F16) {
            ((f16*)p.out)[(long)m * p.ldo + n] = (f16)gelu_erf(v);
        } else if (EPI == DEPI_F16) {
            ((f16*)p.out)[(long)m * p.ldo + n] = (f16)v;
        } else if (EPI == DEPI_F32) {
            ((float*)p.out)[(long)m * p.ldo + n] = v;
        } else if (EPI == DEPI_QKV) {
            const int which = n / p.d, c = n - which * p.d, head = c >> 6, dim = c & 63, nh = p.d >> 6;
            if (which == 0) {
                ((float*)p.out)[(long)m * p.d + c] = v;
            } else if (which == 1) {
                p.kc[(((long)m * nh + head) * p.maxT + pos) * MZ_HD + dim] = (f16)v;
            } else {
                p.vct[(((long)m * nh + head) * MZ_HD + dim) * p.maxT + pos] = (f16)v;
            }
        }
    }
}

// ---------------------------------------------------------------- attention of one query per (row, head)

__global__ void __launch_bounds__(256) dec_attn_kernel(const MzDecAttn a) {
    __shared__ float qs[MZ_HD];
    __shared__ float sc[CHMAX];
    __shared__ __attribute__((aligned(16))) f16 pr[CHMAX + 8];
    __shared__ float red[4];
    __shared__ float ov[MZ_HD];
    __shared__ int last;

    const int bh = blockIdx.x, b = bh / a.nh, head = bh - b * a.nh, sp = blockIdx.y;
    if (a.done[b]) return;
    const int tid = threadIdx.x;
    const int L = a.L > 0 ? a.L : a.ctr[0] + 1;
    const int j0 = sp * a.chunk, j1 = min(j0 + a.chunk, L), n = max(j1 - j0, 0);

    if (tid < MZ_HD) {
        float q = a.qbias ? (float)a.qbias[head * MZ_HD + tid] : 0.f;
        for (int s = 0; s < a.nq; s++) q += a.q[s * a.qstride + (long)b * a.d + head * MZ_HD + tid];
        qs[tid] = q * 0.125f;
    }
    __syncthreads();

    // scores: 8 lanes per key (16 bytes each), 32 keys per pass, 4 keys in flight per lane
    const f16* kb = a.k + (long)b * a.kv_b + (long)head * a.kv_h;
    const int grp = tid >> 3, sub = tid & 7;
    float q8[8];
#pragma unroll
    for (int e = 0; e < 8; e++) q8[e] = qs[sub * 8 + e];
    float lmax = -INFINITY;
    for (int jb = grp; jb < n; jb += 128) {
        f16x8 kv[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            int jj = jb + 32 * u;
            kv[u] = jj < n ? ld8(kb + (long)(j0 + jj) * MZ_HD + sub * 8) : f16x8{};
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            float dt = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) dt = fmaf(q8[e], (float)kv[u][e], dt);
            dt += __shfl_xor(dt, 1);
            dt += __shfl_xor(dt, 2);
            dt += __shfl_xor(dt, 4);
            int jj = jb + 32 * u;
            if (jj < n) {
                if (sub == 0) sc[jj] = dt;
                lmax = fmaxf(lmax, dt);
            }
        }
    }
    const float mc = block_reduce_max(lmax, red);  // includes the barrier that publishes sc

    int slot = -1;
    if (a.aslot) slot = a.aslot[head];
    float ls = 0.f;
    for (int jj = tid; jj < n; jj += 256) {
        const float s = sc[jj];
        const f16 ph = (f16)__expf(s - mc);
        pr[jj] = ph;
        ls += (float)ph;
        if (slot >= 0) a.sal[((long)b * a.na + slot) * MZ_TPAD + j0 + jj] = s;
    }
    const int n8 = (n + 7) & ~7;
    if (tid < n8 - n) pr[n + tid] = (f16)0.f;
    const float lc = block_reduce_sum(ls, red);  // barrier: pr complete

    // P.V over V^T rows: 8 lanes per dim row (16 bytes = 8 keys each), dims grp and grp + 32
    const f16* vb = a.vt + (long)b * a.kv_b + (long)head * a.kv_h;
    const int ng = n8 >> 3;
#pragma unroll
    for (int hpass = 0; hpass < 2; hpass++) {
        const int dim = grp + 32 * hpass;
        const f16* vr = vb + (long)dim * a.vt_ld + j0;
        float acc = 0.f;
        for (int g0 = sub; g0 < ng; g0 += 32) {
            f16x8 vv[4], pp[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                int gg = g0 + 8 * u;
                vv[u] = gg < ng ? ld8(vr + gg * 8) : f16x8{};
                pp[u] = gg < ng ? *(const f16x8*)&pr[gg * 8] : f16x8{};
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    f16x2 x2 = {vv[u][2 * e], vv[u][2 * e + 1]}, p2 = {pp[u][2 * e], pp[u][2 * e + 1]};
                    acc = __builtin_amdgcn_fdot2(x2, p2, acc, false);
                }
        }
        acc += __shfl_xor(acc, 1);
        acc += __shfl_xor(acc, 2);
        acc += __shfl_xor(acc, 4);
        if (sub == 0) ov[dim] = acc;
    }
    __syncthreads();

    if (a.nsplit == 1) {
        if (tid < MZ_HD) a.out[(long)b * a.d + head * MZ_HD + tid] = (f16)(ov[tid] / lc);
        if (slot >= 0) {
            const int p = a.ctr[0];
            f16* al = a.align + (((long)b * a.maxT + p) * a.na + slot) * MZ_TENC;
            for (int jj = tid; jj < n; jj += 256) al[j0 + jj] = (f16)(__expf(sc[jj] - mc) / lc);
        }
        return;
    }

    // split: publish (max, sum, P.V) of this chunk; the last block of (row, head) combines
    float* mypart = a.part + ((long)bh * a.nsplit + sp) * 66;
    if (tid < MZ_HD) mypart[2 + tid] = ov[tid];
    if (tid == 0) {
        mypart[0] = mc;
        mypart[1] = lc;
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) last = atomicAdd(&a.counter[bh], 1u) == (unsigned)(a.nsplit - 1);
    __syncthreads();
    if (!last) return;
    __threadfence();
    const float* parts = a.part + (long)bh * a.nsplit * 66;
    float m = -INFINITY;
    for (int c = 0; c < a.nsplit; c++) m = fmaxf(m, parts[c * 66]);
    float l = 0.f, o = 0.f;
    for (int c = 0; c < a.nsplit; c++) {
        const float w = __expf(parts[c * 66] - m);
        l += parts[c * 66 + 1] * w;
        if (tid < MZ_HD) o += parts[c * 66 + 2 + tid] * w;
    }
    if (tid < MZ_HD) a.out[(long)b * a.d + head * MZ_HD + tid] = (f16)(o / l);
    if (slot >= 0) {
        const int p = a.ctr[0];
        const float* s = a.sal + ((long)b * a.na + slot) * MZ_TPAD;
        f16* al = a.align + (((long)b * a.maxT + p) * a.na + slot) * MZ_TENC;
        const float inv = 1.f / l;
        for (int j = tid; j < L; j += 256) al[j] = (f16)(__expf(s[j] - m) * inv);
    }
    if (tid == 0) a.counter[bh] = 0u;
}

// ---------------------------------------------------------------- row kernels (one wave per row)

__device__ __forceinline__ void ln_row_store(float2 (&v)[MAXV], int nv, int lane, const f16* w, const f16* b, f16* y,
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
            float c0 = v[i].x - mean, c1 = v[i].y - mean;
            q += c0 * c0 + c1 * c1;
        }
    const float rstd = rsqrtf(wave_sum(q) / dim + eps);
#pragma unroll
    for (int i = 0; i < MAXV; i++)
        if (i < nv) {
            int idx = (lane + 64 * i) * 2;
            f16x2 o = {(f16)((v[i].x - mean) * rstd * (float)w[idx] + (float)b[idx]),
                       (f16)((v[i].y - mean) * rstd * (float)w[idx + 1] + (float)b[idx + 1])};
            *(f16x2*)(y + idx) = o;
        }
}

__global__ void __launch_bounds__(256) dec_add_ln_kernel(float* x, const float* parts, int nparts, long part_stride,
                                                         const f16* bias, const f16* w, const f16* b, f16* y, int rows,
                                                         int dim, float eps) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int nv = dim / 128;
    float2 v[MAXV];
#pragma unroll
    for (int i = 0; i < MAXV; i++)
        if (i < nv) {
            const long idx = (long)row * dim + (lane + 64 * i) * 2;
            float2 a = *(const float2*)(x + idx);
            for (int s = 0; s < nparts; s++) {
                float2 pv = *(const float2*)(parts + s * part_stride + idx);
                a.x += pv.x;
                a.y += pv.y;
            }
            if (bias) {
                a.x += (float)bias[(lane + 64 * i) * 2];
                a.y += (float)bias[(lane + 64 * i) * 2 + 1];
            }
            *(float2*)(x + idx) = a;
            v[i] = a;
        }
    ln_row_store(v, nv, lane, w, b, y + (long)row * dim, dim, eps);
}

__global__ void __launch_bounds__(256) dec_embed_ln_kernel(const int* tok, const int* ctr, const f16* emb, const f16* pe,
                                                           float* x, const f16* w, const f16* b, f16* y, int rows,
                                                           int dim, int maxT, float eps) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int p = ctr[0], t = tok[(long)row * maxT + p], nv = dim / 128;
    float2 v[MAXV];
#pragma unroll
    for (int i = 0; i < MAXV; i++)
        if (i < nv) {
            const int idx = (lane + 64 * i) * 2;
            f16x2 e = *(const f16x2*)(emb + (long)t * dim + idx), q = *(const f16x2*)(pe + (long)p * dim + idx);
            float2 a = {(float)e[0] + (float)q[0], (float)e[1] + (float)q[1]};
            *(float2*)(x + (long)row * dim + idx) = a;
            v[i] = a;
        }
    ln_row_store(v, nv, lane, w, b, y + (long)row * dim, dim, eps);
}

// ---------------------------------------------------------------- greedy choice

__global__ void __launch_bounds__(256) dec_argmax_kernel(const float* logits, int V, const unsigned char* sup, int* tok,
                                                         int* done, int* ctr, unsigned* counter, int maxT,
                                                         int prompt_len, int eos, int bs1, int bs2, int advance) {
    __shared__ float sv[4];
    __shared__ int si[4];
    __shared__ int last;
    const int b = blockIdx.x, tid = threadIdx.x;
    const int p = ctr[0];
    if (!(p + 1 < prompt_len || p + 1 >= maxT)) {
        const bool first = p + 1 == prompt_len;
        const float* lg = logits + (long)b * V;
        float best = -INFINITY;
        int bi = 0x7fffffff;
        for (int i = tid; i < V; i += 256) {
            if (sup[i] || (first && (i == bs1 || i == bs2))) continue;
            const float v = lg[i];
            if (v > best || (v == best && i < bi)) {
                best = v;
                bi = i;
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(best, o);
            const int oi = __shfl_xor(bi, o);
            if (ov > best || (ov == best && oi < bi)) {
                best = ov;
                bi = oi;
            }
        }
        if ((tid & 63) == 0) {
            sv[tid >> 6] = best;
            si[tid >> 6] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < 4; w++)
                if (sv[w] > best || (sv[w] == best && si[w] < bi)) {
                    best = sv[w];
                    bi = si[w];
                }
            const int t = (done[b] || bi == 0x7fffffff) ? eos : bi;
            tok[(long)b * maxT + p + 1] = t;
            if (t == eos) done[b] = 1;
        }
    }
    if (!advance) return;
    __threadfence();
    __syncthreads();
    if (tid == 0) last = atomicAdd(counter, 1u) == gridDim.x - 1;
    __syncthreads();
    if (last && tid == 0) {
        __threadfence();
        ctr[0] = p + 1;
        counter[0] = 0u;
    }
}

}  // namespace

hipError_t mz_dec_gemm_launch(hipStream_t s, int epi, const MzDec& g) {
    if (g.K % 64 != 0 || g.M <= 0 || g.N <= 0 || g.ksplit <= 0 || (g.K / 64) % g.ksplit != 0) return hipErrorInvalidValue;
    if (epi == DEPI_QKV && (g.N != 3 * g.d || g.d % 64 != 0)) return hipErrorInvalidValue;
    if (epi != DEPI_PARTIAL && g.ksplit != 1) return hipErrorInvalidValue;
    dim3 grid((g.N + 31) / 32, g.ksplit, (g.M + 31) / 32);
    switch (epi) {
        case DEPI_PARTIAL: hipLaunchKernelGGL(dec_gemm_kernel<DEPI_PARTIAL>, grid, dim3(256), 0, s, g); break;
        case DEPI_GELU_F16: hipLaunchKernelGGL(dec_gemm_kernel<DEPI_GELU_F16>, grid, dim3(256), 0, s, g); break;
        case DEPI_F32: hipLaunchKernelGGL(dec_gemm_kernel<DEPI_F32>, grid, dim3(256), 0, s, g); break;
        case DEPI_QKV: hipLaunchKernelGGL(dec_gemm_kernel<DEPI_QKV>, grid, dim3(256), 0, s, g); break;
        case DEPI_F16: hipLaunchKernelGGL(dec_gemm_kernel<DEPI_F16>, grid, dim3(256), 0, s, g); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t mz_dec_attn_launch(hipStream_t s, const MzDecAttn& a) {
    if (a.chunk <= 0 || a.chunk > CHMAX || a.chunk % 8 != 0 || a.vt_ld % 8 != 0 || a.nsplit <= 0) return hipErrorInvalidValue;
    if (a.nsplit > 1 && (!a.part || !a.counter)) return hipErrorInvalidValue;
    if (a.L > 0 && a.nsplit * a.chunk < a.L) return hipErrorInvalidValue;
    dim3 grid(a.B * a.nh, a.nsplit);
    hipLaunchKernelGGL(dec_attn_kernel, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t mz_dec_add_ln_launch(hipStream_t s, float* x, const float* parts, int nparts, long part_stride,
                                const f16* bias, const f16* w, const f16* b, f16* y, int rows, int dim, float eps) {
    if (dim % 128 != 0 || dim > 128 * MAXV || rows <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dec_add_ln_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, parts, nparts, part_stride, bias, w,
                       b, y, rows, dim, eps);
    return hipGetLastError();
}

hipError_t mz_dec_embed_ln_launch(hipStream_t s, const int* tok, const int* ctr, const f16* emb, const f16* pe,
                                  float* x, const f16* w, const f16* b, f16* y, int rows, int dim, int maxT, float eps) {
    if (dim % 128 != 0 || dim > 128 * MAXV || rows <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dec_embed_ln_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, tok, ctr, emb, pe, x, w, b, y, rows,
                       dim, maxT, eps);
    return hipGetLastError();
}

hipError_t mz_dec_argmax_launch(hipStream_t s, const float* logits, int V, const unsigned char* sup, int* tok, int* done,
                                int* ctr, unsigned* counter, int B, int maxT, int prompt_len, int eos, int bs1, int bs2,
                                int advance) {
    if (B <= 0 || V <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dec_argmax_kernel, dim3(B), dim3(256), 0, s, logits, V, sup, tok, done, ctr, counter, maxT,
                       prompt_len, eos, bs1, bs2, advance);
    return hipGetLastError();
}
