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
#include "wave_tree.h"

using namespace maivs_dev;

// The index's per-slot rows in HBM through the build (maivs_gpu_store_*): f32 rows, i8 / SQ8
// rows and sign codes in slot order, the arrays the layout flags name. `token` changes with every
// write, so an arena description can name the exact state it was made from.
struct RowStore {
    uint32_t dim = 0, W = 0, flags = 0;
    uint32_t n = 0, cap = 0;
    float* f32 = nullptr;
    int8_t* codes = nullptr;
    uint64_t* bits = nullptr;
    uint64_t token = 0;  // 0: never reset
    std::vector<void*> allocs;
};

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
    uint32_t pq_tree_block_max_q = 1000000;  // the block-wide tree descent up to this many queries
    uint32_t pq_rounds_max_q = 64;           // the per-query scan in rounds of cells up to this many queries
    uint32_t pq_split_max_q = 64;            // the split per-query scan up to this many queries
    uint32_t finish_wide_max_q = 64;         // the finish with kFinishWideThreads threads up to this many queries
    uint32_t pq_front_max_q = 64;            // the per-query path's fused prep + tree + route up to this many queries
    uint32_t pq_finish_split_max_q = 64;     // the per-query path's rerank spread over workgroups up to this many queries
    Ctl* h_ctl = nullptr;  // pinned host copy of the control block (read after each pass)
    // pinned staging of the host-buffer entry points (queries in, slots and scores out), grown on
    // demand and kept for the context's life
    void* h_stage = nullptr;
    size_t h_stage_bytes = 0;
    hipEvent_t ev[8] = {};
    // last call, for maivs_gpu_last_candidates / maivs_gpu_last_counters
    uint32_t last_nq = 0, last_fin_cap = 0;
    bool last_pq = false;  // the last search ran the per-query path (no seed / rest-cut state kept)
    KParams last_K{};
    uint32_t initial_cand_cap = 4096;
    int front_rest_mode = -1;  // rest ranks the seed stage scans itself: -1 by cell sharing, else 0 or 8
    int mma_min_mode = -1;     // matrix-core scan items: -1 by cell sharing, 0 off, else their least query count
    bool xcd_order = true;     // matrix-core scan items in cell order, a contiguous chunk per XCD
    bool ham_mma = false;      // the query-tiled Hamming rows on the matrix cores (else by popcounts)
    bool rows_pass = false;    // the batched pass by Hamming rows at any cell count
    // the main pass captured as one HIP graph, replayed while its key matches
    struct GraphKey {
        KParams K;
        const float* q;
        uint32_t* slots;
        float* scores;
        uint64_t gen;
    };
    bool use_graph = false;  // MAIVS_GPU_GRAPH=1: replay the main pass as one captured graph
    bool counters_clean = false;  // ctl / cell_cnt / cand_cnt / done are zero (a pass needs no clear first)
    uint64_t buf_gen = 0;  // bumped whenever a buffer the graph references is reallocated
    hipGraphExec_t gexec = nullptr;
    GraphKey gkey{};
    // the per-query path's buffers (tree lists, scan candidates, beams), sized by (nq, tcap, pq_cap)
    std::vector<void*> pq_allocs;
    uint32_t cap_pq_nq = 0, cap_tcap = 0, cap_pq = 0, pq_cap_min = 0;
    std::vector<void*> split_allocs;  // the split per-query scan's per-cell entries, histograms and counts
    uint64_t cap_split_e = 0, cap_split_h = 0, cap_split_n = 0;
    uint32_t* d_beams = nullptr;
    std::vector<uint32_t> beams_on_device;  // what d_beams holds (empty: unknown)
    // the centroid tree (per-query path); n_levels 0 when the arena has none
    TreeDev tree{};
    std::vector<uint32_t> tree_level_n;
    float tree_beam_frac = 0.5f;
    uint32_t tree_min_beam = 32;
    // this device's fixed scratch array (ScratchSlot, maivs_gpu.hip), set at create
    void* scratch = nullptr;
    RowStore store;
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

// Check a centroid tree (every child range inside the next level, leaves naming cells < M) and
// copy it to HBM; allocations go to `owner`. An absent tree (null or no levels) gives n_levels 0.
inline int upload_tree(maivs_gpu_ctx* ctx, std::vector<void*>& owner, const maivs_tree_desc* T, uint32_t W, uint32_t M,
                       TreeDev* out, std::vector<uint32_t>* level_n_host) {
    *out = TreeDev{};
    if (level_n_host) level_n_host->clear();
    if (!T || T->n_levels == 0) return 0;
    if (!T->level_n || !T->level_codes || !T->child_start || !T->child_len || !T->leaf_codes || !T->leaf_cells ||
        T->n_leaf == 0 || !(T->beam_frac > 0.0f))
        return fail(ctx, MAIVS_ERR_ARG, "centroid tree: incomplete description");
    std::vector<uint32_t> off(T->n_levels + 1, 0);
    for (uint32_t l = 0; l < T->n_levels; ++l) {
        if (T->level_n[l] == 0) return fail(ctx, MAIVS_ERR_ARG, "centroid tree: empty level %u", l);
        off[l + 1] = off[l] + T->level_n[l];
    }
    for (uint32_t l = 0; l < T->n_levels; ++l) {
        const uint32_t next = l + 1 < T->n_levels ? T->level_n[l + 1] : T->n_leaf;
        for (uint32_t j = off[l]; j < off[l + 1]; ++j)
            if (static_cast<uint64_t>(T->child_start[j]) + T->child_len[j] > next)
                return fail(ctx, MAIVS_ERR_ARG, "centroid tree: child range past level %u", l + 1);
    }
    for (uint32_t j = 0; j < T->n_leaf; ++j)
        if (T->leaf_cells[j] >= M) return fail(ctx, MAIVS_ERR_ARG, "centroid tree: leaf cell out of range");
    const uint32_t nodes = off[T->n_levels];
    uint32_t *d_off, *d_cs, *d_cl, *d_leaf;
    uint64_t *d_codes, *d_leaf_codes;
    int rc;
    if ((rc = dalloc(ctx, owner, &d_off, off.size())) || (rc = dalloc(ctx, owner, &d_codes, static_cast<size_t>(nodes) * W)) ||
        (rc = dalloc(ctx, owner, &d_cs, nodes)) || (rc = dalloc(ctx, owner, &d_cl, nodes)) ||
        (rc = dalloc(ctx, owner, &d_leaf_codes, static_cast<size_t>(T->n_leaf) * W)) ||
        (rc = dalloc(ctx, owner, &d_leaf, T->n_leaf)))
        return rc;
    HIP_TRY(ctx, hipMemcpyAsync(d_off, off.data(), off.size() * 4, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(d_codes, T->level_codes, static_cast<size_t>(nodes) * W * 8, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(d_cs, T->child_start, static_cast<size_t>(nodes) * 4, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(d_cl, T->child_len, static_cast<size_t>(nodes) * 4, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(d_leaf_codes, T->leaf_codes, static_cast<size_t>(T->n_leaf) * W * 8, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(d_leaf, T->leaf_cells, static_cast<size_t>(T->n_leaf) * 4, hipMemcpyHostToDevice, ctx->stream));
    out->lv_off = d_off;
    out->lv_codes = d_codes;
    out->lv_cs = d_cs;
    out->lv_cl = d_cl;
    out->leaf_codes = d_leaf_codes;
    out->leaf_ids = d_leaf;
    out->n_levels = T->n_levels;
    out->n_leaf = T->n_leaf;
    if (level_n_host) level_n_host->assign(T->level_n, T->level_n + T->n_levels);
    return 0;
}

}  // namespace maivs_host
