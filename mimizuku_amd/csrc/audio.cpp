// Audio front end, host side: WAV reading (read_wav, src/audio.rs:14-75), resampling to 16 kHz (to_16k,
// src/audio.rs:77-145) and the tables of the log-mel features (Mel::new, src/audio.rs:146-193). The features
// themselves run on the device (k_mel.hip, mz_log_mel).
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/mimizuku.h"
#include "mz_internal.h"
#include "mz_kernels.h"

#pragma clang fp contract(off)

namespace {

bool read_all(const char* path, std::vector<unsigned char>* b) {
    FILE* f = fopen(path, "rb");
    if (!f) return false;
    unsigned char buf[1 << 16];
    size_t r;
    while ((r = fread(buf, 1, sizeof buf, f)) > 0) b->insert(b->end(), buf, buf + r);
    fclose(f);
    return true;
}

double bessel_i0(double x) {
    double s = 1.0, t = 1.0, k = 1.0;
    while (t > 1e-12 * s) {
        const double q = x / (2.0 * k);
        t *= q * q;
        s += t;
        k += 1.0;
    }
    return s;
}

size_t gcd(size_t a, size_t b) { return b == 0 ? a : gcd(b, a % b); }

double hz_to_mel(double f) {
    const double logstep = 27.0 / log(6.4);
    return f >= 1000.0 ? 15.0 + log(f / 1000.0) * logstep : 3.0 * f / 200.0;
}

double mel_to_hz(double m) {
    const double logstep = log(6.4) / 27.0;
    return m >= 15.0 ? 1000.0 * exp(logstep * (m - 15.0)) : 200.0 * m / 3.0;
}

}  // namespace

extern "C" int mz_wav_read(const char* path, float* y, size_t cap, size_t* n, int* sr) {
    if (!path || !n || !sr) return mz_fail(MZ_ERR_ARG, "mz_wav_read: null argument");
    std::vector<unsigned char> b;
    if (!read_all(path, &b)) return mz_fail(MZ_ERR_ARG, "%s: cannot read", path);
    if (b.size() < 12 || memcmp(b.data(), "RIFF", 4) || memcmp(b.data() + 8, "WAVE", 4))
        return mz_fail(MZ_ERR_ARG, "%s: not a RIFF/WAVE file", path);
    auto u16le = [&](size_t i) { return (unsigned)(b[i] | (b[i + 1] << 8)); };
    auto u32le = [&](size_t i) { return (uint32_t)b[i] | ((uint32_t)b[i + 1] << 8) | ((uint32_t)b[i + 2] << 16) | ((uint32_t)b[i + 3] << 24); };
    unsigned fmt = 0, bits = 0;
    size_t ch = 0, rate = 0, i = 12;
    while (i + 8 <= b.size()) {
        const unsigned char* id = &b[i];
        const size_t len = u32le(i + 4), body = i + 8;
        const bool is_data = !memcmp(id, "data", 4);
        if (body + len > b.size() && !is_data)
            return mz_fail(MZ_ERR_ARG, "%s: truncated %.4s chunk", path, (const char*)id);
        if (!memcmp(id, "fmt ", 4)) {
            if (len < 16 || (u16le(body) == 0xfffe && len < 26)) return mz_fail(MZ_ERR_ARG, "%s: short fmt chunk", path);
            fmt = u16le(body);
            ch = u16le(body + 2);
            rate = u32le(body + 4);
            bits = u16le(body + 14);
            if (fmt == 0xfffe) fmt = u16le(body + 24);  // WAVE_FORMAT_EXTENSIBLE: the sub-format GUID starts with it
        } else if (is_data) {
            if (ch == 0 || bits == 0) return mz_fail(MZ_ERR_ARG, "%s: data before fmt", path);
            if (!((fmt == 1 && (bits == 16 || bits == 24 || bits == 32)) || (fmt == 3 && bits == 32)))
                return mz_fail(MZ_ERR_ARG, "%s: unsupported WAV format %u/%u bit (16/24/32-bit PCM or 32-bit float)",
                               path, fmt, bits);
            const size_t frame = ch * bits / 8;
            // a streaming writer leaves the size at 0xFFFFFFFF: then the data runs to the end of the file
            const bool streamed = len == 0xffffffffu;
            if (!streamed && (body + len > b.size() || len % frame != 0))
                return mz_fail(MZ_ERR_ARG, "%s: data chunk is truncated or not whole frames", path);
            const size_t dlen = streamed ? b.size() - body : len, nf = dlen / frame;
            const unsigned char* d = &b[body];
            *n = nf;
            *sr = (int)rate;
            if (!y || cap < nf) return MZ_OK;  // size query
            for (size_t t = 0; t < nf; t++) {
                float acc = 0.f;
                for (size_t c = 0; c < ch; c++) {
                    const size_t o = (t * ch + c) * (bits / 8);
                    float v;
                    if (fmt == 1 && bits == 16) {
                        v = (float)(int16_t)(d[o] | (d[o + 1] << 8)) / 32768.0f;
                    } else if (fmt == 1 && bits == 24) {
                        const int32_t w = (int32_t)(((uint32_t)d[o] << 8) | ((uint32_t)d[o + 1] << 16) | ((uint32_t)d[o + 2] << 24));
                        v = (float)(w >> 8) / 8388608.0f;
                    } else if (fmt == 1) {
                        const int32_t w = (int32_t)((uint32_t)d[o] | ((uint32_t)d[o + 1] << 8) | ((uint32_t)d[o + 2] << 16) | ((uint32_t)d[o + 3] << 24));
                        v = (float)w / 2147483648.0f;
                    } else {
                        uint32_t w = (uint32_t)d[o] | ((uint32_t)d[o + 1] << 8) | ((uint32_t)d[o + 2] << 16) | ((uint32_t)d[o + 3] << 24);
                        memcpy(&v, &w, 4);
                    }
                    acc += v;  // channels summed in order, then averaged (librosa's mono=True)
                }
                y[t] = acc / (float)ch;
                if (!isfinite(y[t])) return mz_fail(MZ_ERR_ARG, "%s: samples that are not finite numbers", path);
            }
            return MZ_OK;
        }
        i = body + len + (len & 1);
    }
    return mz_fail(MZ_ERR_ARG, "%s: no data chunk", path);
}

// Kaiser-windowed sinc low-pass (passband to 95% of the lower Nyquist frequency, 32 zero crossings per side,
// beta 9), one filter per output phase; evaluated in double in the order src/audio.rs:97-145 uses.
extern "C" int mz_resample_16k(const float* y, size_t n, int sr, float* out, size_t cap, size_t* n_out) {
    if ((!y && n) || !n_out) return mz_fail(MZ_ERR_ARG, "mz_resample_16k: null argument");
    const size_t SR = 16000;
    if (sr == (int)SR) {
        *n_out = n;
        if (out && cap >= n) std::copy(y, y + n, out);
        return MZ_OK;
    }
    if (sr < 1000 || sr > 768000) return mz_fail(MZ_ERR_ARG, "unsupported sample rate %d", sr);
    const size_t g = gcd((size_t)sr, SR), up = SR / g, down = (size_t)sr / g;
    const double scale = std::min((double)SR / (double)sr, 1.0), fc = 0.95 * scale / 2.0;
    const long half = (long)ceil(32.0 / scale);
    const double beta = 9.0, i0b = bessel_i0(beta);
    const size_t ntaps = (size_t)(2 * half + 2);
    auto taps = [&](size_t ph, std::vector<double>& w) {
        const double frac = (double)ph / (double)up;
        w.resize(ntaps);
        for (long k = -half; k <= half + 1; k++) {
            const double t = (double)k - frac;
            const double sinc = t == 0.0 ? 2.0 * fc : sin(2.0 * M_PI * fc * t) / (M_PI * t);
            const double r = t / (double)half;
            w[(size_t)(k + half)] = fabs(r) > 1.0 ? 0.0 : sinc * bessel_i0(beta * sqrt(1.0 - r * r)) / i0b;
        }
        double norm = 0.0;
        for (double v : w) norm += v;
        for (double& v : w) v = v / norm;
    };
    const size_t nout = (n * up + down - 1) / down;
    *n_out = nout;
    if (!out || cap < nout) return MZ_OK;  // size query
    // the filters of every phase are tabulated unless the ratio makes that table large
    const bool tab = up * ntaps <= ((size_t)1 << 22);
    std::vector<std::vector<double>> table;
    if (tab) {
        table.resize(up);
        for (size_t p = 0; p < up; p++) taps(p, table[p]);
    }
    std::vector<double> tmp;
    for (size_t k = 0; k < nout; k++) {
        const size_t pos = k * down;
        const long c = (long)(pos / up);
        const size_t ph = pos % up;
        const std::vector<double>* w = &tmp;
        if (tab) w = &table[ph];
        else taps(ph, tmp);
        double acc = 0.0;
        for (size_t q = 0; q < ntaps; q++) {
            const long idx = c + (long)q - half;
            if (idx >= 0 && (size_t)idx < n) acc += (*w)[q] * (double)y[idx];
        }
        out[k] = (float)acc;
    }
    return MZ_OK;
}

// Slaney mel filters [201][n_mels] up to 8 kHz and the periodic-Hann-windowed DFT basis [400][201] (cos, sin),
// as Mel::new (src/audio.rs:161-189) builds them, the basis stored sample-major for the device.
extern "C" int mz_mel_tables(int n_mels, float* filters, double* cosb, double* sinb) {
    if (n_mels <= 0 || n_mels > 256) return mz_fail(MZ_ERR_ARG, "mz_mel_tables: n_mels %d out of range", n_mels);
    const int NB = MZ_MEL_BINS, NF = MZ_MEL_NFFT;
    if (filters) {
        const double m0 = hz_to_mel(0.0), m1 = hz_to_mel(8000.0);
        std::vector<double> ff(n_mels + 2);
        for (int i = 0; i < n_mels + 2; i++) ff[i] = mel_to_hz(m0 + (m1 - m0) * (double)i / (double)(n_mels + 1));
        for (int k = 0; k < NB; k++) {
            const double fq = (double)k * (16000.0 / 2.0) / (double)(NB - 1);
            for (int m = 0; m < n_mels; m++) {
                const double dn = (fq - ff[m]) / (ff[m + 1] - ff[m]);
                const double upv = (ff[m + 2] - fq) / (ff[m + 2] - ff[m + 1]);
                const double enorm = 2.0 / (ff[m + 2] - ff[m]);
                filters[(size_t)k * n_mels + m] = (float)(std::max(std::min(dn, upv), 0.0) * enorm);
            }
        }
    }
    if (cosb || sinb) {
        for (int j = 0; j < NF; j++) {
            const double win = 0.5 - 0.5 * cos(2.0 * M_PI * (double)j / (double)NF);
            for (int k = 0; k < NB; k++) {
                const double a = 2.0 * M_PI * (double)((k * j) % NF) / (double)NF;
                if (cosb) cosb[(size_t)j * NB + k] = win * cos(a);
                if (sinb) sinb[(size_t)j * NB + k] = win * sin(a);
            }
        }
    }
    return MZ_OK;
}

extern "C" int mz_log_mel(mz_ctx* c, uint64_t audio, const int32_t* n_samples, int n, int n_mels, uint64_t mel,
                          int32_t* frames) {
    if (!c || !audio || !n_samples || !mel) return mz_fail(MZ_ERR_ARG, "mz_log_mel: null argument");
    if (n <= 0 || n_mels <= 0 || n_mels > 256) return mz_fail(MZ_ERR_ARG, "mz_log_mel: bad sizes");
    const int NB = MZ_MEL_BINS, NF = MZ_MEL_NFFT, T = MZ_NFR_HOST;
    std::vector<int32_t> ns(n);
    for (int i = 0; i < n; i++) {
        if (n_samples[i] < 0) return mz_fail(MZ_ERR_ARG, "mz_log_mel: negative sample count");
        ns[i] = std::min(n_samples[i], (int32_t)MZ_MEL_NSAMPLES);
        if (frames) frames[i] = std::min((ns[i] + MZ_MEL_HOP - 1) / MZ_MEL_HOP, T);
    }
    std::vector<float> filt((size_t)NB * n_mels);
    std::vector<double> cb((size_t)NF * NB), sb((size_t)NF * NB);
    mz_mel_tables(n_mels, filt.data(), cb.data(), sb.data());
    // scratch: tables, per-clip sample counts, power spectra [n][3000][201], per-clip maxima
    const size_t bytes_f = filt.size() * 4, bytes_b = cb.size() * 8, bytes_p = (size_t)n * T * NB * 4;
    char* base = nullptr;
    const size_t total = bytes_f + 2 * bytes_b + (size_t)n * 4 + bytes_p + (size_t)n * 4 + 1024;
    if (int r = mz_hip(hipMalloc((void**)&base, total), "hipMalloc")) return r;
    auto align = [](size_t v) { return (v + 255) & ~(size_t)255; };
    size_t off = 0;
    float* d_filt = (float*)(base + off);
    off = align(off + bytes_f);
    double* d_cos = (double*)(base + off);
    off = align(off + bytes_b);
    double* d_sin = (double*)(base + off);
    off = align(off + bytes_b);
    int* d_ns = (int*)(base + off);
    off = align(off + (size_t)n * 4);
    float* d_pow = (float*)(base + off);
    off = align(off + bytes_p);
    float* d_max = (float*)(base + off);
    int r = MZ_OK;
    if (off + (size_t)n * 4 > total) r = mz_fail(MZ_ERR_STATE, "mz_log_mel: scratch layout");
    if (!r) r = mz_hip(hipMemcpyAsync(d_filt, filt.data(), bytes_f, hipMemcpyHostToDevice, c->stream), "hipMemcpy");
    if (!r) r = mz_hip(hipMemcpyAsync(d_cos, cb.data(), bytes_b, hipMemcpyHostToDevice, c->stream), "hipMemcpy");
    if (!r) r = mz_hip(hipMemcpyAsync(d_sin, sb.data(), bytes_b, hipMemcpyHostToDevice, c->stream), "hipMemcpy");
    if (!r) r = mz_hip(hipMemcpyAsync(d_ns, ns.data(), (size_t)n * 4, hipMemcpyHostToDevice, c->stream), "hipMemcpy");
    if (!r) {
        MzMel p{(const float*)(uintptr_t)audio, d_ns, d_cos, d_sin, d_filt, d_pow, d_max, (float*)(uintptr_t)mel, n, n_mels};
        r = mz_hip(mz_log_mel_launch(c->stream, p), "log-mel");
    }
    const int rs = mz_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    hipFree(base);
    return r ? r : rs;
}
