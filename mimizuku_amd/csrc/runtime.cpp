// C ABI: device runtime (context, memory, copies, events, graphs) and the per-kernel entry points.
// Replaces the reference's cudarc layer (src/gpu.rs:69-287). Errors are returned as codes with a thread-local
// message, never thrown across the ABI.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <set>
#include <string>
#include <vector>
#include <algorithm>

#include "../../include/mimizuku.h"
#include "mz_internal.h"
#include "mz_kernels.h"

static thread_local std::string g_err;

int mz_fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int mz_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return MZ_OK;
    return mz_fail(MZ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

extern "C" const char* mz_last_error(void) { return g_err.c_str(); }
extern "C" const char* mz_version(void) { return "mimizuku_amd 0.1.0 (gfx950)"; }

// ------------------------------------------------------------------ context

extern "C" int mz_init(int device, mz_ctx** out) {
    if (!out) return mz_fail(MZ_ERR_ARG, "mz_init: null out");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) return mz_fail(MZ_ERR_HIP, "mz_init: no HIP device available (%s)", hipGetErrorString(e));
    if (device < 0 || device >= n) return mz_fail(MZ_ERR_ARG, "mz_init: device %d of %d", device, n);
    if (int r = mz_hip(hipSetDevice(device), "hipSetDevice")) return r;
    // the no-allocation timestamp entry point's static scratch: its address on this device, looked up once
    if (int r = mz_ts_scratch_setup(device)) return r;
    auto* c = new mz_ctx();
    c->device = device;
    // graph capture is not allowed on the legacy default stream (src/gpu.rs:125); default priority
    if (int r = mz_hip(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate")) {
        delete c;
        return r;
    }
    *out = c;
    return MZ_OK;
}

extern "C" int mz_ctx_free(mz_ctx* c) {
    if (!c) return MZ_OK;
    hipSetDevice(c->device);
    hipStreamSynchronize(c->stream);
    for (void* p : c->allocs) hipFree(p);
    hipStreamDestroy(c->stream);
    delete c;
    return MZ_OK;
}

int mz_ctx_alloc(mz_ctx* c, size_t bytes, void** p) {
    bytes = bytes < 16 ? 16 : bytes;
    *p = nullptr;
    if (int r = mz_hip(hipMalloc(p, bytes), "hipMalloc")) return mz_fail(r, "hipMalloc of %zu bytes failed", bytes);
    if (int r = mz_hip(hipMemsetAsync(*p, 0, bytes, c->stream), "hipMemsetAsync")) return r;
    if (int r = mz_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize")) return r;
    c->allocs.insert(*p);
    return MZ_OK;
}

extern "C" int mz_alloc(mz_ctx* c, size_t bytes, uint64_t* dptr) {
    if (!c || !dptr) return mz_fail(MZ_ERR_ARG, "mz_alloc: null argument");
    void* p;
    if (int r = mz_ctx_alloc(c, bytes, &p)) return r;
    *dptr = (uint64_t)(uintptr_t)p;
    return MZ_OK;
}

extern "C" int mz_free(mz_ctx* c, uint64_t dptr) {
    if (!c) return mz_fail(MZ_ERR_ARG, "mz_free: null ctx");
    void* p = (void*)(uintptr_t)dptr;
    if (!c->allocs.count(p)) return mz_fail(MZ_ERR_ARG, "mz_free: not a buffer of this context");
    hipStreamSynchronize(c->stream);
    c->allocs.erase(p);
    return mz_hip(hipFree(p), "hipFree");
}

extern "C" int mz_mem_info(mz_ctx* c, size_t* free_bytes, size_t* total_bytes) {
    if (!c || !free_bytes || !total_bytes) return mz_fail(MZ_ERR_ARG, "mz_mem_info: null argument");
    return mz_hip(hipMemGetInfo(free_bytes, total_bytes), "hipMemGetInfo");
}

extern "C" int mz_upload(mz_ctx* c, uint64_t dst, const void* src, size_t bytes) {
    if (!c || (!src && bytes)) return mz_fail(MZ_ERR_ARG, "mz_upload: null argument");
    if (!bytes) return MZ_OK;
    if (int r = mz_hip(hipMemcpyAsync((void*)(uintptr_t)dst, src, bytes, hipMemcpyHostToDevice, c->stream), "upload"))
        return r;
    return mz_hip(hipStreamSynchronize(c->stream), "upload sync");
}

extern "C" int mz_download(mz_ctx* c, void* dst, uint64_t src, size_t bytes) {
    if (!c || (!dst && bytes)) return mz_fail(MZ_ERR_ARG, "mz_download: null argument");
    if (!bytes) return mz_hip(hipStreamSynchronize(c->stream), "download sync");
    if (int r = mz_hip(hipMemcpyAsync(dst, (const void*)(uintptr_t)src, bytes, hipMemcpyDeviceToHost, c->stream),
                       "download"))
        return r;
    return mz_hip(hipStreamSynchronize(c->stream), "download sync");
}

extern "C" int mz_copy(mz_ctx* c, uint64_t dst, uint64_t src, size_t bytes) {
    if (!c) return mz_fail(MZ_ERR_ARG, "mz_copy: null ctx");
    if (!bytes) return MZ_OK;
    return mz_hip(hipMemcpyAsync((void*)(uintptr_t)dst, (const void*)(uintptr_t)src, bytes, hipMemcpyDeviceToDevice,
                                 c->stream),
                  "copy");
}

extern "C" int mz_sync(mz_ctx* c) {
    if (!c) return mz_fail(MZ_ERR_ARG, "mz_sync: null ctx");
    return mz_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

extern "C" int mz_event_create(mz_ctx* c, uint64_t* ev) {
    if (!c || !ev) return mz_fail(MZ_ERR_ARG, "mz_event_create: null argument");
    hipEvent_t e;
    if (int r = mz_hip(hipEventCreate(&e), "hipEventCreate")) return r;
    *ev = (uint64_t)(uintptr_t)e;
    return MZ_OK;
}
extern "C" int mz_event_record(mz_ctx* c, uint64_t ev) {
    if (!c) return mz_fail(MZ_ERR_ARG, "mz_event_record: null ctx");
    return mz_hip(hipEventRecord((hipEvent_t)(uintptr_t)ev, c->stream), "hipEventRecord");
}
extern "C" int mz_event_elapsed_ms(uint64_t a, uint64_t b, float* ms) {
    if (!ms) return mz_fail(MZ_ERR_ARG, "mz_event_elapsed_ms: null out");
    if (int r = mz_hip(hipEventSynchronize((hipEvent_t)(uintptr_t)b), "hipEventSynchronize")) return r;
    return mz_hip(hipEventElapsedTime(ms, (hipEvent_t)(uintptr_t)a, (hipEvent_t)(uintptr_t)b), "hipEventElapsedTime");
}
extern "C" int mz_event_destroy(uint64_t ev) { return mz_hip(hipEventDestroy((hipEvent_t)(uintptr_t)ev), "hipEventDestroy"); }

// ------------------------------------------------------------------ graphs

extern "C" int mz_graph_begin(mz_ctx* c) {
    if (!c) return mz_fail(MZ_ERR_ARG, "mz_graph_begin: null ctx");
    return mz_hip(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
}

extern "C" int mz_graph_end(mz_ctx* c, mz_graph** out) {
    if (!c || !out) return mz_fail(MZ_ERR_ARG, "mz_graph_end: null argument");
    *out = nullptr;
    hipGraph_t g = nullptr;
    if (int r = mz_hip(hipStreamEndCapture(c->stream, &g), "hipStreamEndCapture")) return r;
    if (!g) return mz_fail(MZ_ERR_STATE, "empty graph");
    hipGraphExec_t x = nullptr;
    hipError_t e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        hipGraphDestroy(g);
        return mz_hip(e, "hipGraphInstantiate");
    }
    if (int r = mz_hip(hipGraphUpload(x, c->stream), "hipGraphUpload")) {
        hipGraphExecDestroy(x);
        hipGraphDestroy(g);
        return r;
    }
    *out = new mz_graph{g, x};
    return MZ_OK;
}

extern "C" int mz_graph_launch(mz_ctx* c, mz_graph* g) {
    if (!c || !g) return mz_fail(MZ_ERR_ARG, "mz_graph_launch: null argument");
    return mz_hip(hipGraphLaunch(g->exec, c->stream), "hipGraphLaunch");
}

extern "C" int mz_graph_free(mz_graph* g) {
    if (!g) return MZ_OK;
    hipGraphExecDestroy(g->exec);
    hipGraphDestroy(g->graph);
    delete g;
    return MZ_OK;
}

// ------------------------------------------------------------------ per-kernel entry points

#define DP(x) ((void*)(uintptr_t)(x))
#define CDP(T, x) ((const T*)(uintptr_t)(x))

extern "C" int mz_gemm(mz_ctx* c, uint64_t x, int ldx, uint64_t w, uint64_t y, int ldy, int m, int n, int k,
                       uint64_t bias) {
    if (!c) return mz_fail(MZ_ERR_ARG, "mz_gemm: null ctx");
    if (m <= 0 || n <= 0 || k <= 0 || k % 64 || n % 4 || ldx < k || ldy < n)
        return mz_fail(MZ_ERR_ARG, "mz_gemm: unsupported shape m=%d n=%d k=%d ldx=%d ldy=%d (k %% 64, n %% 4)", m, n, k,
                       ldx, ldy);
    if (m <= 32) {
        MzDec g{};
        g.x = CDP(f16, x);
        g.ldx = ldx;
        g.W = CDP(f16, w);
        g.bias = CDP(f16, bias);
        g.M = m;
        g.N = n;
        g.K = k;
        g.ksplit = 1;
        g.out = DP(y);
        g.ldo = ldy;
        return mz_hip(mz_dec_gemm_launch(c->stream, DEPI_F16, g), "mz_gemm");
    }
    MzGemm g{};
    g.A = CDP(f16, x);
    g.lda = ldx;
    g.W = CDP(f16, w);
    g.bias = CDP(f16, bias);
    g.M = m;
    g.N = n;
    g.K = k;
    g.out = DP(y);
    g.ldo = ldy;
    return mz_hip(mz_gemm_launch(c->stream, ALOAD_PLAIN, EPI_F16, g), "mz_gemm");
}

extern "C" int mz_linear(mz_ctx* c, const mz_linear_args* a) {
    if (!c || !a) return mz_fail(MZ_ERR_ARG, "mz_linear: null argument");
    if (a->m <= 0 || a->n <= 0 || a->k <= 0 || a->k % 64 || a->n % 4)
        return mz_fail(MZ_ERR_ARG, "mz_linear: unsupported shape m=%d n=%d k=%d", a->m, a->n, a->k);
    if (a->epilogue < MZ_EPI_F16 || a->epilogue > MZ_EPI_HEADS) return mz_fail(MZ_ERR_ARG, "mz_linear: bad epilogue");
    if (a->epilogue == MZ_EPI_HEADS && (a->n % 64 || (a->kind != 2 && a->kind != 3) || a->nh <= 0 ||
                                        a->blocks_per_clip < a->n / 64 || a->m % 1500))
        return mz_fail(MZ_ERR_ARG, "mz_linear: bad head scatter (n %% 64, kind 2|3, m multiple of 1500)");
    if (a->conv_cin > 0 && (a->conv_cin % 8 || a->k < 3 * a->conv_cin || a->conv_tout <= 0 || a->m % a->conv_tout ||
                            (a->conv_stride != 1 && a->conv_stride != 2)))
        return mz_fail(MZ_ERR_ARG, "mz_linear: bad conv geometry");
    MzGemm g{};
    g.A = CDP(f16, a->a);
    g.lda = a->lda;
    g.W = CDP(f16, a->w);
    g.bias = CDP(f16, a->bias);
    g.M = a->m;
    g.N = a->n;
    g.K = a->k;
    g.conv_cin = a->conv_cin;
    g.conv_tin = a->conv_tin;
    g.conv_tout = a->conv_tout;
    g.conv_stride = a->conv_stride;
    g.out = DP(a->out);
    g.ldo = a->ldo;
    g.pos = CDP(f16, a->pos);
    g.heads = (f16*)DP(a->heads);
    g.blocks_per_clip = a->blocks_per_clip;
    g.nh = a->nh;
    g.kind = a->kind;
    g.slot0 = a->slot0;
    return mz_hip(mz_gemm_launch(c->stream, a->conv_cin > 0 ? ALOAD_CONV : ALOAD_PLAIN, a->epilogue, g), "mz_linear");
}

extern "C" int mz_layernorm(mz_ctx* c, uint64_t x, long ldx, uint64_t w, uint64_t b, uint64_t y, long ldy, int rows,
                            int dim, float eps) {
    if (!c) return mz_fail(MZ_ERR_ARG, "mz_layernorm: null ctx");
    if (dim % 128 || dim > 2048 || rows <= 0) return mz_fail(MZ_ERR_ARG, "mz_layernorm: dim %d (multiple of 128, <= 2048)", dim);
    return mz_hip(mz_layernorm_launch(c->stream, CDP(float, x), ldx, CDP(f16, w), CDP(f16, b), (f16*)DP(y), ldy, rows,
                                      dim, eps),
                  "mz_layernorm");
}

extern "C" int mz_add_layernorm(mz_ctx* c, uint64_t x, uint64_t d, uint64_t w, uint64_t b, uint64_t y, int rows,
                                int dim, float eps) {
    if (!c) return mz_fail(MZ_ERR_ARG, "mz_add_layernorm: null ctx");
    if (dim % 128 || dim > 2048 || rows <= 0) return mz_fail(MZ_ERR_ARG, "mz_add_layernorm: dim %d", dim);
    return mz_hip(mz_add_layernorm_launch(c->stream, (float*)DP(x), CDP(f16, d), CDP(f16, w), CDP(f16, b), (f16*)DP(y),
                                          rows, dim, eps),
                  "mz_add_layernorm");
}

extern "C" int mz_enc_attention(mz_ctx* c, uint64_t qkvh, uint64_t out, int clips, int nh) {
    if (!c) return mz_fail(MZ_ERR_ARG, "mz_enc_attention: null ctx");
    if (clips <= 0 || nh <= 0) return mz_fail(MZ_ERR_ARG, "mz_enc_attention: clips %d heads %d", clips, nh);
    return mz_hip(mz_enc_attention_launch(c->stream, CDP(f16, qkvh), (f16*)DP(out), clips, nh), "mz_enc_attention");
}

extern "C" int mz_mel_transpose(mz_ctx* c, uint64_t mel, uint64_t melT, int clips, int n_mels) {
    if (!c) return mz_fail(MZ_ERR_ARG, "mz_mel_transpose: null ctx");
    return mz_hip(mz_mel_transpose_launch(c->stream, CDP(float, mel), (f16*)DP(melT), clips, n_mels), "mz_mel_transpose");
}

// ------------------------------------------------------------------ token timestamps on the device

extern "C" int mz_jump_times_device(mz_ctx* c, uint64_t w, int64_t clip_stride, int n, const int32_t* rows,
                                    const int32_t* cols, int heads, int cols_full, int width, int half, float* out,
                                    int64_t out_stride) {
    if (!c || !w || !rows || !cols || !out || n < 0 || heads <= 0 || cols_full <= 0 || clip_stride < 0)
        return mz_fail(MZ_ERR_ARG, "mz_jump_times_device: bad argument");
    if (width < 1 || width % 2 == 0 || width > MZ_TS_MAX_WIDTH)
        return mz_fail(MZ_ERR_ARG, "mz_jump_times_device: width %d (odd, at most %d)", width, MZ_TS_MAX_WIDTH);
    if (n == 0) return MZ_OK;
    int rmax = 0;
    std::vector<int2> rc(n);
    for (int i = 0; i < n; i++) {
        if (rows[i] < 0 || cols[i] < 0 || cols[i] > cols_full || rows[i] > 4095 || rows[i] > out_stride)
            return mz_fail(MZ_ERR_ARG, "mz_jump_times_device: clip %d has %d rows, %d columns", i, rows[i], cols[i]);
        rc[i] = int2{rows[i], cols[i]};
        rmax = std::max(rmax, rows[i]);
    }
    if (int r = mz_hip(hipSetDevice(c->device), "hipSetDevice")) return r;
    const long ds = mz_ts_diag_stride(rmax, cols_full);
    const size_t stat = (size_t)n * heads * cols_full;
    const size_t bytes[5] = {(size_t)n * sizeof(int2), stat * 4, stat * 4, (size_t)n * ds * 5,
                             (size_t)n * out_stride * 4};
    void* buf[5] = {};
    auto release = [&]() {
        for (void* b : buf)
            if (b) hipFree(b);
    };
    for (int i = 0; i < 5; i++)
        if (int r = mz_hip(hipMalloc(&buf[i], std::max<size_t>(bytes[i], 4)), "hipMalloc")) {
            release();
            return r;
        }
    MzTs p{};
    p.w = (const float*)(uintptr_t)w;
    p.clip_stride = clip_stride;
    p.heads = heads;
    p.cols_full = cols_full;
    p.width = width;
    p.half = half;
    p.rmax = rmax;
    p.rc = (const int2*)buf[0];
    p.mean = (float*)buf[1];
    p.sd = (float*)buf[2];
    p.cost = (float*)buf[3];
    p.trace = (signed char*)((float*)buf[3] + (size_t)n * ds);
    p.diag_stride = ds;
    p.ldd = mz_ts_ldd(rmax);
    p.out = (float*)buf[4];
    p.out_stride = out_stride;
    int r = mz_hip(hipMemcpyAsync(buf[0], rc.data(), bytes[0], hipMemcpyHostToDevice, c->stream), "upload");
    if (!r) r = mz_hip(mz_ts_launch(c->stream, p, n), "timestamp kernels");
    for (int i = 0; i < n && !r; i++)
        if (rows[i] > 0)
            r = mz_hip(hipMemcpyAsync(out + i * out_stride, (float*)buf[4] + i * out_stride, (size_t)rows[i] * 4,
                                      hipMemcpyDeviceToHost, c->stream),
                       "download");
    if (!r) r = mz_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    release();
    return r;
}
