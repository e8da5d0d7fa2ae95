// Whisper's log-mel features on the device (Mel::features, src/audio.rs:195-249; WhisperFeatureExtractor): the
// 30 s buffer zero padded, centred 400-point frames every 160 samples with reflect padding, the periodic-Hann-
// windowed DFT as power spectra, 201 x n_mels Slaney filters, log10 floored at 1e-10, clamped to (max - 8) per
// clip, then (x + 4) / 4. Frames past the audio are log10(1e-10) = -10 without computing them.
//
// The DFT follows the reference's arithmetic operation for operation: samples widened to double, each bin's real
// and imaginary sums accumulated in double in sample order (multiply, then add; contraction is off in this file),
// the power rounded to float. The filter sums are float, in bin order. So the power spectra equal the reference's
// bit for bit; log10 is the device library's (the reference's is the host libm's).
//
//   mel_dft_kernel    one workgroup per (16 frames, clip): the frames' 2,800 samples staged in LDS, thread k < 201
//                     owns bin k of the 16 frames (32 double accumulators), the basis read sample-major so a
//                     wave's loads are contiguous
//   mel_filter_kernel one workgroup per (frame, clip): the frame's power spectrum in LDS, one thread per mel
//   mel_norm_kernel   one workgroup per clip: the maximum, then the clamp and scale in place
#include <math.h>

#include "mz_common.h"
#include "mz_kernels.h"

#pragma clang fp contract(off)

namespace {

constexpr int FB = 16;                                     // frames per workgroup
constexpr int SPAN = (FB - 1) * MZ_MEL_HOP + MZ_MEL_NFFT;  // samples those frames read

__device__ __forceinline__ int live_frames(int n) {
    return min((n + MZ_MEL_NFFT / 2 + MZ_MEL_HOP - 1) / MZ_MEL_HOP, MZ_NFR_HOST);
}

__global__ void __launch_bounds__(256) mel_dft_kernel(const MzMel p) {
    __shared__ __attribute__((aligned(16))) float xs[SPAN];
    const int c = blockIdx.y, t0 = blockIdx.x * FB, n = p.ns[c];
    if (t0 >= live_frames(n)) return;
    const float* y = p.audio + (long)c * MZ_MEL_NSAMPLES;
    // sample i of the padded buffer: reflect at both ends of the 30 s window, zero past the audio
    for (int q = threadIdx.x; q < SPAN; q += blockDim.x) {
        int i = t0 * MZ_MEL_HOP + q - MZ_MEL_NFFT / 2;
        if (i < 0) i = -i;
        else if (i >= MZ_MEL_NSAMPLES) i = 2 * (MZ_MEL_NSAMPLES - 1) - i;
        xs[q] = i < n ? y[i] : 0.f;
    }
    __syncthreads();
    const int k = threadIdx.x;
    if (k >= MZ_MEL_BINS) return;
    double re[FB], im[FB];
#pragma unroll
    for (int f = 0; f < FB; f++) re[f] = im[f] = 0.0;
    // four samples per step: one 16-byte LDS read per frame, the sums still taken one sample at a time
    for (int j = 0; j < MZ_MEL_NFFT; j += 4) {
        double cj[4], sj[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            cj[q] = p.cosb[(j + q) * MZ_MEL_BINS + k];
            sj[q] = p.sinb[(j + q) * MZ_MEL_BINS + k];
        }
#pragma unroll
        for (int f = 0; f < FB; f++) {
            const float4 x4 = *(const float4*)&xs[f * MZ_MEL_HOP + j];
            const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const double x = (double)xv[q];
                re[f] = re[f] + x * cj[q];
                im[f] = im[f] + x * sj[q];
            }
        }
    }
    const int live = live_frames(n);
#pragma unroll
    for (int f = 0; f < FB; f++) {
        const int t = t0 + f;
        if (t < live) p.pow[((long)c * MZ_NFR_HOST + t) * MZ_MEL_BINS + k] = (float)(re[f] * re[f] + im[f] * im[f]);
    }
}

__global__ void __launch_bounds__(256) mel_filter_kernel(const MzMel p) {
    __shared__ float pw[MZ_MEL_BINS];
    const int c = blockIdx.y, t = blockIdx.x;
    const bool live = t < live_frames(p.ns[c]);
    if (live)
        for (int k = threadIdx.x; k < MZ_MEL_BINS; k += blockDim.x)
            pw[k] = p.pow[((long)c * MZ_NFR_HOST + t) * MZ_MEL_BINS + k];
    __syncthreads();
    for (int m = threadIdx.x; m < p.n_mels; m += blockDim.x) {
        float v = -10.f;
        if (live) {
            float acc = 0.f;
            for (int k = 0; k < MZ_MEL_BINS; k++) acc = acc + p.filt[k * p.n_mels + m] * pw[k];
            v = log10f(fmaxf(acc, 1e-10f));
        }
        p.mel[((long)c * p.n_mels + m) * MZ_NFR_HOST + t] = v;
    }
}

__global__ void __launch_bounds__(1024) mel_norm_kernel(const MzMel p) {
    __shared__ float red[16];
    const int c = blockIdx.x;
    float* m = p.mel + (long)c * p.n_mels * MZ_NFR_HOST;
    const int total = p.n_mels * MZ_NFR_HOST;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < total; i += blockDim.x) mx = fmaxf(mx, m[i]);
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) mx = fmaxf(mx, red[w]);
    const float lo = mx - 8.0f;
    for (int i = threadIdx.x; i < total; i += blockDim.x) m[i] = (fmaxf(m[i], lo) + 4.0f) / 4.0f;
    if (threadIdx.x == 0) p.mx[c] = mx;
}

}  // namespace

hipError_t mz_log_mel_launch(hipStream_t s, const MzMel& p) {
    if (p.n <= 0 || p.n_mels <= 0 || p.n_mels > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mel_dft_kernel, dim3((MZ_NFR_HOST + FB - 1) / FB, p.n), dim3(256), 0, s, p);
    hipLaunchKernelGGL(mel_filter_kernel, dim3(MZ_NFR_HOST, p.n), dim3(p.n_mels <= 128 ? 128 : 256), 0, s, p);
    hipLaunchKernelGGL(mel_norm_kernel, dim3(p.n), dim3(1024), 0, s, p);
    return hipGetLastError();
}
