// Host-side helpers: IEEE binary16 conversions and the token-timestamp alignment (median filter + DTW over the
// alignment heads' cross-attention), following src/align.rs:8-106 and transformers' _extract_token_timestamps.
#include <immintrin.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "../../include/mimizuku.h"
#include "mz_internal.h"

// binary16 from binary32, round to nearest even; NaN stays NaN (quiet), overflow goes to infinity.
uint16_t mz_f2h_host(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u);
    if (a >= 0x477ff000u) return sign | 0x7c00u;  // >= 65520: rounds past the largest finite half
    if (a < 0x38800000u) {
        // below 2^-14: a multiple of 2^-24 (subnormal half); the scaling is exact, nearbyint rounds to even
        float f;
        std::memcpy(&f, &a, 4);
        return sign | (uint16_t)std::nearbyint(f * 16777216.0f);
    }
    // normal: drop 13 mantissa bits with round-half-to-even (a carry into the exponent is the right result)
    const uint32_t r = a + 0x0fffu + ((a >> 13) & 1u);
    return sign | (uint16_t)((r >> 13) - (112u << 10));
}

float mz_h2f_host(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t u;
    if (e == 0) {
        float v = std::ldexp((float)m, -24);
        return sign ? -v : v;
    } else if (e == 31) {
        u = sign | 0x7f800000u | (m << 13);
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

extern "C" uint16_t mz_f2h(float x) { return mz_f2h_host(x); }
extern "C" float mz_h2f(uint16_t h) { return mz_h2f_host(h); }

// DTW over cost m [rows][cols] with a float32 cost table; ties go to the horizontal move (j - 1). Cells are filled
// row by row: each depends only on its left, upper and upper-left neighbours, so the table equals the column-order
// fill of the numpy reference while walking memory contiguously.
static void dtw_path(const double* m, int rows, int cols, std::vector<int>& text, std::vector<int>& time) {
    const int w = cols + 1;
    std::vector<float> cost((size_t)(rows + 1) * w, INFINITY);
    std::vector<int8_t> trace((size_t)(rows + 1) * w, -1);
    cost[0] = 0.f;
    for (int i = 1; i <= rows; i++) {
        const float* up = &cost[(size_t)(i - 1) * w];
        float* cur = &cost[(size_t)i * w];
        int8_t* tr = &trace[(size_t)i * w];
        const double* mr = m + (size_t)(i - 1) * cols;
        for (int j = 1; j <= cols; j++) {
            const float c0 = up[j - 1], c1 = up[j], c2 = cur[j - 1];
            float c;
            int8_t t;
            if (c0 < c1 && c0 < c2) {
                c = c0;
                t = 0;
            } else if (c1 < c0 && c1 < c2) {
                c = c1;
                t = 1;
            } else {
                c = c2;
                t = 2;
            }
            cur[j] = (float)(mr[j - 1] + (double)c);
            tr[j] = t;
        }
    }
    for (int j = 0; j <= cols; j++) trace[j] = 2;
    for (int i = 0; i <= rows; i++) trace[(size_t)i * w] = 1;
    text.clear();
    time.clear();
    int i = rows, j = cols;
    while (i > 0 || j > 0) {
        text.push_back(i - 1);
        time.push_back(j - 1);
        const int8_t t = trace[(size_t)i * w + j];
        if (t == 0) {
            i--;
            j--;
        } else if (t == 1) {
            i--;
        } else {
            j--;
        }
    }
    std::reverse(text.begin(), text.end());
    std::reverse(time.begin(), time.end());
}

extern "C" int mz_dtw(const double* m, int rows, int cols, int32_t* text, int32_t* time, int32_t* len) {
    if (!m || !text || !time || !len || rows < 0 || cols < 0) return mz_fail(MZ_ERR_ARG, "mz_dtw: bad argument");
    std::vector<int> a, b;
    dtw_path(m, rows, cols, a, b);
    for (size_t k = 0; k < a.size(); k++) {
        text[k] = a[k];
        time[k] = b[k];
    }
    *len = (int32_t)a.size();
    return MZ_OK;
}

namespace {

// This file is built with F16C and AVX2 (checked at run time by host_ok): the fp16 round trips of the timestamp
// arithmetic use the hardware conversion (round to nearest even, as the software mz_f2h_host), and the median
// network vectorises over frames.
inline float rhw(float x) { return _cvtsh_ss(_cvtss_sh(x, 0)); }
inline float load_w(const float* w, size_t i) { return w[i]; }

inline void cswap(float& a, float& b) {
    const float lo = a < b ? a : b, hi = a < b ? b : a;
    a = lo;
    b = hi;
}

// median of 7 finite values: a 16-comparator sorting network, middle element
inline float median7(const float* p) {
    float a[7] = {p[0], p[1], p[2], p[3], p[4], p[5], p[6]};
    cswap(a[0], a[6]), cswap(a[2], a[3]), cswap(a[4], a[5]);
    cswap(a[0], a[2]), cswap(a[1], a[4]), cswap(a[3], a[6]);
    cswap(a[0], a[1]), cswap(a[2], a[5]), cswap(a[3], a[4]);
    cswap(a[1], a[2]), cswap(a[4], a[6]);
    cswap(a[2], a[3]), cswap(a[4], a[5]);
    cswap(a[1], a[2]), cswap(a[3], a[4]), cswap(a[5], a[6]);
    return a[3];
}

// The DTW cost of jump_times (src/align.rs:8-52): m [rows][cols] = minus the head average of the median-filtered
// per-column z-scores of w [rows][heads][cols_full] cropped to cols columns (rows, cols >= 1).
template <class T>
void align_cost_impl(const T* w, int rows, int heads, int cols_full, int cols, int width, int half, double* m) {
    const int pad = width / 2;
    std::vector<float> avg((size_t)rows * cols, 0.f), z((size_t)rows * cols), win(width), padded(cols + 2 * pad);
    std::vector<double> sum(cols), sq(cols);
    std::vector<float> sumf(cols), sqf(cols), mean(cols), sd(cols);
    for (int a = 0; a < heads; a++) {
        // normalise each column over the rows (population std); a constant column scores 0. half: the column sum and
        // the sum of squared deviations from the unrounded mean accumulate in float in row order, then the mean and
        // deviation are rounded through fp16 (src/align.rs:18-20); otherwise both sums are taken in double
        std::fill(sum.begin(), sum.end(), 0.0);
        std::fill(sq.begin(), sq.end(), 0.0);
        std::fill(sumf.begin(), sumf.end(), 0.f);
        std::fill(sqf.begin(), sqf.end(), 0.f);
        for (int i = 0; i < rows; i++) {
            const size_t o = ((size_t)i * heads + a) * cols_full;
            if (half)
                for (int j = 0; j < cols; j++) sumf[j] += load_w(w, o + j);
            else
                for (int j = 0; j < cols; j++) sum[j] += load_w(w, o + j);
        }
        for (int j = 0; j < cols; j++) mean[j] = half ? sumf[j] / (float)rows : (float)(sum[j] / rows);
        for (int i = 0; i < rows; i++) {
            const size_t o = ((size_t)i * heads + a) * cols_full;
            for (int j = 0; j < cols; j++) {
                if (half) {
                    const float dv = load_w(w, o + j) - mean[j];
                    sqf[j] += dv * dv;
                } else {
                    const double dv = (double)(load_w(w, o + j) - mean[j]);
                    sq[j] += dv * dv;
                }
            }
        }
        for (int j = 0; j < cols; j++) {
            if (half) {
                sd[j] = rhw(std::sqrt(sqf[j] / (float)rows));
                mean[j] = rhw(mean[j]);
            } else {
                sd[j] = std::sqrt((float)(sq[j] / rows));
            }
        }
        for (int i = 0; i < rows; i++) {
            const size_t o = ((size_t)i * heads + a) * cols_full;
            float* zr = &z[(size_t)i * cols];
            for (int j = 0; j < cols; j++) {
                const float x = load_w(w, o + j);
                float v = 0.f;
                if (sd[j] > 0.f) v = half ? rhw(rhw(x - mean[j]) / sd[j]) : (x - mean[j]) / sd[j];
                zr[j] = v;
            }
        }
        // median over a width-`width` window with reflect padding, then accumulate over heads
        for (int i = 0; i < rows; i++) {
            const float* row = &z[(size_t)i * cols];
            float* ar = &avg[(size_t)i * cols];
            if (cols <= pad) {
                for (int j = 0; j < cols; j++) ar[j] += row[j];
                continue;
            }
            for (int k = 0; k < cols + 2 * pad; k++) {
                int t = k - pad;
                if (t < 0) t = -t;
                if (t >= cols) t = 2 * (cols - 1) - t;
                padded[k] = row[t];
            }
            if (width == 7) {
                for (int j = 0; j < cols; j++) ar[j] += median7(&padded[j]);
            } else {
                for (int j = 0; j < cols; j++) {
                    std::copy(&padded[j], &padded[j] + width, win.begin());
                    std::nth_element(win.begin(), win.begin() + pad, win.end());
                    ar[j] += win[pad];
                }
            }
        }
    }
    for (size_t k = 0; k < (size_t)rows * cols; k++) {
        float s = avg[k] / (float)heads;
        if (half) s = rhw(s);
        m[k] = -(double)s;
    }
}

// Token start times (src/align.rs:8-63) from w [rows][heads][cols_full].
template <class T>
void jump_times_impl(const T* w, int rows, int heads, int cols_full, int cols, int width, int half, float* out) {
    if (rows == 0) return;
    if (cols == 0) {
        std::fill(out, out + rows, 0.f);
        return;
    }
    std::vector<double> m((size_t)rows * cols);
    align_cost_impl(w, rows, heads, cols_full, cols, width, half, m.data());
    std::vector<int> text, time;
    dtw_path(m.data(), rows, cols, text, time);
    int n = 0;
    for (size_t k = 0; k < text.size() && n < rows; k++)
        if (k == 0 || text[k] != text[k - 1]) out[n++] = (float)((double)time[k] * 0.02);
    const float lastv = n ? out[n - 1] : 0.f;
    for (; n < rows; n++) out[n] = lastv;  // degenerate scores can bend the path (src/align.rs:60-61)
}

}  // namespace

static bool jump_args_ok(int rows, int heads, int cols_full, int cols, int width) {
    return rows >= 0 && heads > 0 && cols >= 0 && cols <= cols_full && width > 0 && width % 2 == 1;
}

static int host_ok() {
    static const bool ok = __builtin_cpu_supports("f16c") && __builtin_cpu_supports("avx2");
    return ok ? MZ_OK : mz_fail(MZ_ERR_STATE, "token timestamps need a host CPU with F16C and AVX2");
}

extern "C" int mz_align_cost(const float* w, int rows, int heads, int cols_full, int cols, int width, int half,
                             double* m) {
    if (!w || !m || rows <= 0 || cols <= 0 || !jump_args_ok(rows, heads, cols_full, cols, width))
        return mz_fail(MZ_ERR_ARG, "mz_align_cost: bad argument");
    if (int r = host_ok()) return r;
    align_cost_impl(w, rows, heads, cols_full, cols, width, half, m);
    return MZ_OK;
}

extern "C" int mz_jump_times(const float* w, int rows, int heads, int cols_full, int cols, int width, int half,
                             float* out) {
    if (!w || !out || !jump_args_ok(rows, heads, cols_full, cols, width))
        return mz_fail(MZ_ERR_ARG, "mz_jump_times: bad argument");
    if (int r = host_ok()) return r;
    jump_times_impl(w, rows, heads, cols_full, cols, width, half, out);
    return MZ_OK;
}
