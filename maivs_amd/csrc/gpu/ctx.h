// The context behind the C ABI of libmaivs_gpu.so and the host helpers every translation unit
// of the library shares: error reporting, HIP call checking and tracked device allocations.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "../../../include/maivs_gpu.h"
#include "types.h"

using namespace maivs_dev;

struct maivs_gpu_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::mutex mu;
    std::string err;
    bool uploaded = false;
    DevArena A{};
    std::vector<void*> arena_allocs;
    // host copies needed by the host checks
    std::vector<float> h_r_bound;
    // work buffers
    Work Wk{};
    std::vector<void*> work_allocs;   // per-query / per-cell buffers, sized by (nq, nprobe, k)
    std::vector<void*> cand_allocs;   // candidate buffers, sized by (nq, cand_cap); grow on overflow
    uint32_t cap_nq = 0, cap_nprobe = 0, cap_k = 0, cap_cand = 0, cap_seed = 0, cap_fin = 0, cap_key = 0, cap_bucket = 0;
    uint32_t cand_nq = 0;
    uint32_t max_sort_cap_route = 0;  // largest shortlist sort the route kernel's LDS can hold
    uint32_t seed_cap = 0;            // sum of the SEED_CELLS largest cells: bound of one seed set
    size_t lds_prep = 0, lds_seed = 0, lds_finish = 0;
    hipEvent_t ev[8] = {};
    // last call, for maivs_gpu_last_candidates / maivs_gpu_last_counters
    uint32_t last_nq = 0, last_fin_cap = 0;
    KParams last_K{};
    uint32_t initial_cand_cap = 4096;
    // the main pass captured as one HIP graph, replayed while its key matches
    struct GraphKey {
        KParams K;
        const float* q;
        uint32_t* slots;
        float* scores;
        uint64_t gen;
    };
    bool use_graph = true;
    uint64_t buf_gen = 0;  // bumped whenever a buffer the graph references is reallocated
    hipGraphExec_t gexec = nullptr;
    GraphKey gkey{};
};

namespace maivs_host {

inline int fail(maivs_gpu_ctx* ctx, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx) ctx->err = buf;
    return code;
}

#define HIP_TRY(ctx, call)                                                                      \
    do {                                                                                        \
        hipError_t e_ = (call);                                                                 \
        if (e_ != hipSuccess)                                                                   \
            return fail(ctx, e_ == hipErrorOutOfMemory ? MAIVS_ERR_OOM : MAIVS_ERR_HIP, "%s: %s", \
                        #call, hipGetErrorString(e_));                                          \
    } while (0)

template <class T>
inline int dalloc(maivs_gpu_ctx* ctx, std::vector<void*>& owner, T** p, size_t count) {
    *p = nullptr;
    if (count == 0) count = 1;
    void* v = nullptr;
    HIP_TRY(ctx, hipMalloc(&v, count * sizeof(T)));
    owner.push_back(v);
    *p = static_cast<T*>(v);
    return 0;
}

template <class T>
inline int dupload(maivs_gpu_ctx* ctx, const T* src, size_t count, T** out) {
    int rc = dalloc(ctx, ctx->arena_allocs, out, count);
    if (rc) return rc;
    if (src && count) HIP_TRY(ctx, hipMemcpyAsync(*out, src, count * sizeof(T), hipMemcpyHostToDevice, ctx->stream));
    return 0;
}

inline void free_all(std::vector<void*>& v) {
    for (void* p : v) (void)hipFree(p);
    v.clear();
}

}  // namespace maivs_host
