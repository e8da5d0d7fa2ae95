// Host-side helpers: IEEE binary16 conversions and the token-timestamp alignment (median filter + DTW over the
// alignment heads' cross-attention), following src/align.rs:8-106 and transformers' _extract_token_timestamps.
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

static inline float rh(float x) { return mz_h2f_host(mz_f2h_host(x)); }

// DTW over cost m [rows][cols] with a float32 cost table; ties go to the horizontal move (j - 1).
static void dtw_path(const double* m, int rows, int cols, std::vector<int>& text, std::vector<int>& time) {
    const int w = cols + 1;
    std::vector<float> cost((size_t)(rows + 1) * w, INFINITY);
    std::vector<int8_t> trace((size_t)(rows + 1) * w, -1);
    cost[0] = 0.f;
    for (int j = 1; j <= cols; j++)
        for (int i = 1; i <= rows; i++) {
            const float c0 = cost[(size_t)(i - 1) * w + j - 1], c1 = cost[(size_t)(i - 1) * w + j],
                        c2 = cost[(size_t)i * w + j - 1];
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
            cost[(size_t)i * w + j] = (float)(m[(size_t)(i - 1) * cols + j - 1] + (double)c);
            trace[(size_t)i * w + j] = t;
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

extern "C" int mz_jump_times(const float* w, int rows, int heads, int cols_full, int cols, int width, int half,
                             float* out) {
    if (!w || !out || rows < 0 || heads <= 0 || cols < 0 || cols > cols_full || width <= 0 || width % 2 == 0)
        return mz_fail(MZ_ERR_ARG, "mz_jump_times: bad argument");
    if (rows == 0) return MZ_OK;
    if (cols == 0) {
        std::fill(out, out + rows, 0.f);
        return MZ_OK;
    }
    auto at = [&](int i, int a, int j) { return w[((size_t)i * heads + a) * cols_full + j]; };
    const int pad = width / 2;
    std::vector<float> avg((size_t)rows * cols, 0.f), z((size_t)rows * cols), win(width);
    for (int a = 0; a < heads; a++) {
        // normalise each column over the rows (population std); a constant column scores 0
        for (int j = 0; j < cols; j++) {
            double s = 0;
            for (int i = 0; i < rows; i++) s += at(i, a, j);
            float mean = (float)(s / rows);
            double q = 0;
            for (int i = 0; i < rows; i++) {
                const double dv = (double)(at(i, a, j) - mean);
                q += dv * dv;
            }
            float sd = std::sqrt((float)(q / rows));
            if (half) {
                mean = rh(mean);
                sd = rh(sd);
            }
            for (int i = 0; i < rows; i++) {
                float v = 0.f;
                if (sd > 0.f) v = half ? rh(rh(at(i, a, j) - mean) / sd) : (at(i, a, j) - mean) / sd;
                z[(size_t)i * cols + j] = v;
            }
        }
        // median over a width-`width` window with reflect padding, then accumulate over heads
        for (int i = 0; i < rows; i++) {
            const float* row = &z[(size_t)i * cols];
            for (int j = 0; j < cols; j++) {
                float v;
                if (cols <= pad) {
                    v = row[j];
                } else {
                    for (int k = 0; k < width; k++) {
                        int t = j + k - pad;
                        if (t < 0) t = -t;
                        if (t >= cols) t = 2 * (cols - 1) - t;
                        win[k] = row[t];
                    }
                    std::nth_element(win.begin(), win.begin() + pad, win.end());
                    v = win[pad];
                }
                avg[(size_t)i * cols + j] += v;
            }
        }
    }
    std::vector<double> m((size_t)rows * cols);
    for (size_t k = 0; k < m.size(); k++) {
        float s = avg[k] / (float)heads;
        if (half) s = rh(s);
        m[k] = -(double)s;
    }
    std::vector<int> text, time;
    dtw_path(m.data(), rows, cols, text, time);
    int n = 0;
    for (size_t k = 0; k < text.size() && n < rows; k++)
        if (k == 0 || text[k] != text[k - 1]) out[n++] = (float)((double)time[k] * 0.02);
    const float lastv = n ? out[n - 1] : 0.f;
    for (; n < rows; n++) out[n] = lastv;  // degenerate scores can bend the path (src/align.rs:60-61)
    return MZ_OK;
}
