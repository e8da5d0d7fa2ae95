// Internal host-side definitions shared by the C ABI translation units.
#pragma once
#include <hip/hip_runtime.h>

#include <set>

struct mz_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::set<void*> allocs;  // device buffers owned by the context, freed at mz_ctx_free
};

struct mz_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

// set the thread-local error message and return `code`
int mz_fail(int code, const char* fmt, ...);
// MZ_OK, or MZ_ERR_HIP with the runtime's message
int mz_hip(hipError_t e, const char* what);
// zero-filled device allocation owned by the context
int mz_ctx_alloc(mz_ctx* c, size_t bytes, void** p);

// IEEE binary16 conversions (round to nearest even), host side
uint16_t mz_f2h_host(float x);
float mz_h2f_host(uint16_t h);
