// libmaivs_gpu.so: MI355X (gfx950) batched cell-major search behind the C ABI of
// include/maivs_gpu.h. Restates MAIVS's FlatCellIndex::search_batch_cellmajor
// (src/index.rs:1999-2311) with route_batch (:1873-1980) and rerank_exact (:1309-1378).
//
// Pipeline of one batch (one HIP stream; the host syncs once, at the end, on a small control block):
//   reset        zero the per-call counters
//   prep_route   one workgroup per query: rotation (2 x sign flip + FWHT), 1-bit code,
//                FastScan table, Hamming against every centroid code, tie-inclusive
//                shortlist, exact SQ8 rescore, probe list sorted (score desc, cell asc)
//   seed         one workgroup per query: every member of the first 8 probed cells scored at
//                once, seed cut-off tau (only d <= tau kept), adaptive probe cut, probe counts
//   invert       scan / fill: cell -> probing queries
//   cell_scan    one workgroup per probed cell: each lane holds one member's code; groups of 4
//                probing queries' tables are interleaved in LDS so one ds_read_b32 looks up a
//                nibble for 4 queries; survivors d <= tau appended per query
//   finish       one workgroup per query: exact tie-inclusive cut at k*rerank_factor, exact
//                f32 / SQ8 rerank over chain-major rows, top-k (score desc, slot asc)
// Rare events (candidate buffer overflow, libm-sensitive decisions near their threshold) re-run
// the affected stages after the host has read the control block.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <utility>
#include <string>
#include <type_traits>
#include <vector>

#include "ctx.h"
#include "kernels.h"

namespace {
// Host re-evaluation bands around libm-sensitive thresholds (see host_nucleus / host_rest_end).
constexpr float kPruneBand = 4e-6f;
constexpr float kNucleusBand = 2e-3f;
constexpr size_t kLdsBudget = 160 * 1024;
// The matrix-core scan takes every bucket work item (of up to kBucketQ queries) when the
// cell-major scan averages at least kMmaShare queries per live cell; below that the lookups win
// (measured on the 500k mixture: lookups ahead at 12 queries per cell, matrix cores at 20 and up).
constexpr uint32_t kMmaMinQ = 1;
constexpr double kMmaShare = 16.0;
constexpr uint32_t kScanGridMax = 16384;  // workgroups of the bucket-mode scan (they stride over the items)
}  // namespace

// ================================================================ host side

using namespace maivs_host;

namespace {

void drop_graph(maivs_gpu_ctx* ctx) {
    if (ctx->gexec) (void)hipGraphExecDestroy(ctx->gexec);
    ctx->gexec = nullptr;
    ctx->buf_gen++;
}

bool supported_nw(uint32_t w) { return w == 1 || w == 2 || w == 4 || w == 8 || w == 16; }

#define DISPATCH_EPL(E, ...)                              \
    switch (E) {                                          \
        case 1: { constexpr int EPL = 1; __VA_ARGS__; break; } \
        case 2: { constexpr int EPL = 2; __VA_ARGS__; break; } \
        case 4: { constexpr int EPL = 4; __VA_ARGS__; break; } \
        case 8: { constexpr int EPL = 8; __VA_ARGS__; break; } \
        case 16: { constexpr int EPL = 16; __VA_ARGS__; break; } \
        case 32: { constexpr int EPL = 32; __VA_ARGS__; break; } \
        default: { constexpr int EPL = 64; __VA_ARGS__; break; } \
    }

#define DISPATCH_NW(W, ...)                              \
    switch (W) {                                         \
        case 1: { constexpr int NW = 1; __VA_ARGS__; break; } \
        case 2: { constexpr int NW = 2; __VA_ARGS__; break; } \
        case 4: { constexpr int NW = 4; __VA_ARGS__; break; } \
        case 8: { constexpr int NW = 8; __VA_ARGS__; break; } \
        default: { constexpr int NW = 16; __VA_ARGS__; break; } \
    }

// LDS of prep: codes[kPrepWaves * 16] u64 | per wave x[P] | mins[npos4] | cqp[d4] | rqp[d4]
size_t prep_lds(const DevArena& A) {
    return kPrepWaves * 16 * 8 +
           static_cast<size_t>(kPrepWaves) * (A.P + ((A.npos + 3) & ~3u) + 2 * ((A.d + 3) & ~3u)) * 4;
}

// LDS of route (route_lds_bytes; ex holds the nucleus weights of the capped list, at most
// min(nprobe, sort_cap) of them)
size_t route_lds(const DevArena& A, uint32_t sort_cap, uint32_t nprobe) {
    return route_lds_bytes(A.d, A.W, A.Mp, sort_cap, nprobe);
}

// LDS of one query's prep in the fused front kernel: codes[16] u64 | x[P] | mins[npos4] | cqp[d4] | rqp[d4]
size_t prep1_lds(const DevArena& A) {
    return 16 * 8 + static_cast<size_t>(A.P + ((A.npos + 3) & ~3u) + 2 * ((A.d + 3) & ~3u)) * 4;
}

// The fused front kernel runs when the code covers the whole padded dimension.
bool fused_front(const DevArena& A) { return static_cast<uint64_t>(A.W) * 64 == A.P; }

// Dynamic LDS of seed: probed[MW4] | coarse[256] | fine[256] | misc[64] | sbuf[seed_cap8] u16
// (plus its static table of W*256 bytes)
size_t seed_lds(const DevArena& A, uint32_t seed_cap) {
    return ((A.MW + 3) & ~3u) * 4 + 512 * 4 + 64 * 4 + static_cast<size_t>((seed_cap + 7) & ~7u) * 2;
}

// LDS of finish: hist[256] | scratch[32] | qs[d4] | ent[kFinishLdsCap] (d, slot) | keys[kFinishLdsCap] u64
size_t finish_lds(const DevArena& A) {
    return kHistBins * 4 + 32 * 4 + ((A.d + 3) & ~3u) * 4 + static_cast<size_t>(kFinishLdsCap) * 16;
}

Chain make_chain(uint32_t d, uint32_t vec) {
    Chain c{};
    c.T = d / 8;
    c.Tp = (c.T + vec - 1) / vec * vec;
    c.tail = d - 8 * c.T;
    c.stride = 8 * c.Tp + (c.tail + vec - 1) / vec * vec;
    return c;
}

// Per-cell query buckets: room for 4x the mean number of queries per live cell in the rest scan,
// a power of two in [32, 4096]; a fuller cell sends the pass to the counting-sort inversion.
uint32_t bucket_cap_for(const DevArena& A, uint32_t nq, uint32_t nprobe) {
    const uint64_t pairs = static_cast<uint64_t>(nq) * (nprobe > kSeedCells ? nprobe - kSeedCells : 0u);
    const uint64_t mean = pairs / std::max<uint32_t>(A.n_live, 1u);
    uint32_t cap = 32;
    while (cap < 4 * mean + 32 && cap < 4096) cap <<= 1;
    return cap;
}

// Lays buffers out back to back from a base address, each on a 256-byte boundary. With a null
// base it only counts: the same walk sizes an allocation, then carves it (or a fixed array).
struct Carver {
    uint8_t* base;
    size_t used = 0;
    template <class T>
    void take(T** p, uint64_t count) {
        used = (used + 255) & ~size_t{255};
        *p = base ? reinterpret_cast<T*>(base + used) : nullptr;
        used += static_cast<size_t>(std::max<uint64_t>(count, 1)) * sizeof(T);
    }
};

// The per-query and per-cell work buffers of a batched call of nq queries (everything but the
// candidate lists). host_io: the staged queries and outputs of the host-buffer entry points.
void carve_work(const DevArena& A, uint32_t nq, uint32_t nprobe, uint32_t k, uint32_t seed_cap, uint32_t bcap,
                bool host_io, Carver& c, Work& W, bool rows = false) {
    const uint64_t nql = nq;
    if (host_io) {
        c.take(&W.q, nql * A.d);
        c.take(&W.out_slots, nql * k);
        c.take(&W.out_scores, nql * k);
    } else {
        W.q = nullptr;
        W.out_slots = nullptr;
        W.out_scores = nullptr;
    }
    c.take(&W.qbits, nql * A.W);
    c.take(&W.lut, nql * A.npos * 16);
    c.take(&W.delta, nql);
    c.take(&W.bias, nql);
    c.take(&W.cqs, nql * A.d);
    c.take(&W.cqbase, nql);
    c.take(&W.rbase, nql);
    W.hs = nullptr;
    if (rows || A.Mp > kHdLdsCells) c.take(&W.hs, nql * A.Mp);
    c.take(&W.bnd, nql * nprobe);
    c.take(&W.chosen, nql * nprobe);
    c.take(&W.cscore, nql * nprobe);
    c.take(&W.nchosen, nql);
    c.take(&W.probed, nql * A.MW);
    c.take(&W.seed, nql * seed_cap);
    c.take(&W.seed_cnt, nql);
    c.take(&W.tau, nql);
    c.take(&W.rest_end, nql);
    c.take(&W.cand_cnt, nql);
    c.take(&W.cut, nql);
    c.take(&W.ncand, nql);
    c.take(&W.cell_cnt, static_cast<uint64_t>(A.M) + 1);
    c.take(&W.cell_off, static_cast<uint64_t>(A.M) + 1);
    c.take(&W.cell_cur, static_cast<uint64_t>(A.M) + 1);
    c.take(&W.qof, nql * nprobe);
    c.take(&W.qbuck, static_cast<uint64_t>(A.M) * bcap);
    // scan work items: at most one per kBucketQ (kItemQ) bucket entries plus one per cell
    c.take(&W.active, static_cast<uint64_t>(A.M) + nql * nprobe / kBucketQ + 1);
    c.take(&W.active8, static_cast<uint64_t>(A.M) + nql * nprobe / kItemQ + 1);
    c.take(&W.active_cs, static_cast<uint64_t>(A.M) + nql * nprobe / kBucketQ + 1);
    c.take(&W.flag_route, nql);
    c.take(&W.flag_prune, nql);
    c.take(&W.thr, nql);
    c.take(&W.dhist, nql * kThrBins);
    c.take(&W.thr_at, nql);
    c.take(&W.ctl, 1);
    c.take(&W.cand_n, nql);
    c.take(&W.done, 1);
}

// Room of the final list of one query (seed survivors + candidates) and of its sort keys.
void cand_caps(uint32_t seed_cap, uint32_t cand_cap, uint32_t* fin_cap, uint32_t* key_cap) {
    *fin_cap = seed_cap + cand_cap;
    uint32_t kc = 1;
    while (kc < *fin_cap) kc <<= 1;
    *key_cap = kc;
}

// The candidate, final-list and sort-key buffers of nq queries.
void carve_cand(uint32_t nq, uint32_t seed_cap, uint32_t cand_cap, Carver& c, Work& W) {
    uint32_t fin_cap, key_cap;
    cand_caps(seed_cap, cand_cap, &fin_cap, &key_cap);
    const uint64_t nql = nq;
    c.take(&W.cand, nql * cand_cap);
    c.take(&W.fin, nql * fin_cap);
    c.take(&W.keys, nql * key_cap);
}

// Per-query and per-cell work buffers for (nq, nprobe, k), one allocation; grows only. Candidate
// buffers are a separate allocation (ensure_cand) so that growing them never moves the staged
// queries or outputs.
int ensure_work(maivs_gpu_ctx* ctx, uint32_t nq, uint32_t nprobe, uint32_t k) {
    const DevArena& A = ctx->A;
    const uint32_t seed_cap = ctx->seed_cap;
    const uint32_t bcap = bucket_cap_for(A, nq, nprobe);
    if (nq <= ctx->cap_nq && nprobe <= ctx->cap_nprobe && k <= ctx->cap_k && seed_cap <= ctx->cap_seed &&
        bcap <= ctx->cap_bucket)
        return 0;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    drop_graph(ctx);
    free_all(ctx->work_allocs);
    free_all(ctx->cand_allocs);
    ctx->cand_nq = 0;
    nq = std::max(nq, ctx->cap_nq);
    nprobe = std::max(nprobe, ctx->cap_nprobe);
    k = std::max(k, ctx->cap_k);
    const uint32_t bcap_all = std::max(bcap, ctx->cap_bucket);
    Carver count{nullptr};
    Work& W = ctx->Wk;
    carve_work(A, nq, nprobe, k, seed_cap, bcap_all, true, count, W, ctx->rows_pass);
    uint8_t* base = nullptr;
    int rc = dalloc(ctx, ctx->work_allocs, &base, count.used);
    ctx->counters_clean = false;  // fresh buffers: the next pass clears them first
    if (rc) {
        free_all(ctx->work_allocs);
        ctx->cap_nq = ctx->cap_nprobe = ctx->cap_k = ctx->cap_seed = ctx->cap_bucket = 0;
        return rc;
    }
    Carver cv{base};
    carve_work(A, nq, nprobe, k, seed_cap, bcap_all, true, cv, W, ctx->rows_pass);
    ctx->cap_nq = nq;
    ctx->cap_nprobe = nprobe;
    ctx->cap_k = k;
    ctx->cap_seed = seed_cap;
    ctx->cap_bucket = bcap_all;
    return 0;
}

// Candidate, final-list and sort-key buffers for (cap_nq, cand_cap); grows only.
int ensure_cand(maivs_gpu_ctx* ctx, uint32_t cand_cap) {
    if (ctx->cand_nq >= ctx->cap_nq && cand_cap <= ctx->cap_cand && ctx->cand_nq) return 0;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    drop_graph(ctx);
    free_all(ctx->cand_allocs);
    cand_cap = std::max(cand_cap, ctx->cap_cand);
    Carver count{nullptr};
    carve_cand(ctx->cap_nq, ctx->cap_seed, cand_cap, count, ctx->Wk);
    uint8_t* base = nullptr;
    int rc = dalloc(ctx, ctx->cand_allocs, &base, count.used);
    if (rc) {
        free_all(ctx->cand_allocs);
        ctx->cand_nq = 0;
        ctx->cap_cand = 0;
        return rc;
    }
    Carver cv{base};
    carve_cand(ctx->cap_nq, ctx->cap_seed, cand_cap, cv, ctx->Wk);
    ctx->cand_nq = ctx->cap_nq;
    ctx->cap_cand = cand_cap;
    cand_caps(ctx->cap_seed, cand_cap, &ctx->cap_fin, &ctx->cap_key);
    return 0;
}

int ensure_all(maivs_gpu_ctx* ctx, uint32_t nq, uint32_t nprobe, uint32_t k) {
    int rc = ensure_work(ctx, nq, std::max<uint32_t>(nprobe, 1), std::max<uint32_t>(k, 1));
    if (rc) return rc;
    return ensure_cand(ctx, std::max(ctx->cap_cand, ctx->initial_cand_cap));
}

// ---------------------------------------------------------------- the centroid tree's buffers and descent

constexpr uint32_t kPqPairMaxQ = 256;   // batches up to this many queries use the pair tables in the per-query scan
constexpr uint32_t kPqMaxProbe = 8192;  // probe-list bound of the per-query scan's on-chip suffix array
constexpr uint32_t kSplitMaxProbe = 256;                // the split per-query scan: probe lists up to this long
constexpr uint64_t kSplitMaxBytes = 512ull << 20;       // and per-cell entry buffers up to this size
constexpr uint32_t kPqMaxLevels = 64;

// Tree lists (nq x tcap), scan candidate buffers (nq x pq_cap) and the beams; grow only.
int ensure_pq(maivs_gpu_ctx* ctx, uint32_t nq, uint32_t tcap, uint32_t pq_cap) {
    if (nq <= ctx->cap_pq_nq && tcap <= ctx->cap_tcap && pq_cap <= ctx->cap_pq && ctx->d_beams) return 0;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    drop_graph(ctx);
    free_all(ctx->pq_allocs);
    const uint32_t n = std::max(nq, ctx->cap_pq_nq), t = std::max(tcap, ctx->cap_tcap), c = std::max(pq_cap, ctx->cap_pq);
    Work& W = ctx->Wk;
    int rc = 0;
    rc |= dalloc(ctx, ctx->pq_allocs, &W.tlist, static_cast<size_t>(n) * t);
    rc |= dalloc(ctx, ctx->pq_allocs, &W.tcount, n);
    rc |= dalloc(ctx, ctx->pq_allocs, &W.pqc, static_cast<size_t>(n) * c);
    rc |= dalloc(ctx, ctx->pq_allocs, &ctx->d_beams, kPqMaxLevels);
    ctx->beams_on_device.clear();
    if (rc) {
        free_all(ctx->pq_allocs);
        ctx->cap_pq_nq = ctx->cap_tcap = ctx->cap_pq = 0;
        ctx->d_beams = nullptr;
        return rc;
    }
    ctx->cap_pq_nq = n;
    ctx->cap_tcap = t;
    ctx->cap_pq = c;
    return 0;
}

// The split per-query scan's buffers (Work::pqe, pqh, pqn) for nq queries of nprobe cells of up to
// room entries and nb4 histogram bins each; grow only.
int ensure_split(maivs_gpu_ctx* ctx, uint32_t nq, uint32_t nprobe, uint32_t room, uint32_t nb4) {
    const uint64_t cells = static_cast<uint64_t>(nq) * nprobe;
    const uint64_t ne = cells * room, nh = cells * nb4;
    if (ne <= ctx->cap_split_e && nh <= ctx->cap_split_h && cells <= ctx->cap_split_n) return 0;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    drop_graph(ctx);
    free_all(ctx->split_allocs);
    const uint64_t e = std::max(ne, ctx->cap_split_e), h = std::max(nh, ctx->cap_split_h),
                   n = std::max(cells, ctx->cap_split_n);
    Work& W = ctx->Wk;
    int rc = 0;
    rc |= dalloc(ctx, ctx->split_allocs, &W.pqe, e);
    rc |= dalloc(ctx, ctx->split_allocs, &W.pqh, h);
    rc |= dalloc(ctx, ctx->split_allocs, &W.pqn, n);
    if (rc) {
        free_all(ctx->split_allocs);
        ctx->cap_split_e = ctx->cap_split_h = ctx->cap_split_n = 0;
        return rc;
    }
    ctx->cap_split_e = e;
    ctx->cap_split_h = h;
    ctx->cap_split_n = n;
    return 0;
}

// A kernel's dynamic-LDS limit, raised only when a launch needs more than it was last raised to on
// this device (the limit only grows): the attribute call costs a few µs of host time, which a
// one-query search would otherwise spend while the GPU waits for its next launch.
int raise_lds_limit(maivs_gpu_ctx* ctx, const void* fn, size_t lds) {
    static std::mutex mu;
    static std::map<std::pair<const void*, int>, size_t> raised;
    std::lock_guard<std::mutex> lock(mu);
    size_t& have = raised[{fn, ctx->device}];
    if (lds <= have) return 0;
    HIP_TRY(ctx, hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    have = lds;
    return 0;
}

int launch_pq_tree(maivs_gpu_ctx* ctx, const KParams& K, uint32_t cap) {
    if (K.nq <= ctx->pq_tree_block_max_q) {
        // a workgroup per query, the top level's codes staged in LDS when they fit
        const uint32_t top_n = ctx->tree_level_n.empty() ? 0u : ctx->tree_level_n[0];
        const uint32_t top = top_n * ctx->A.W * 2 <= kTreeTopWords ? top_n * ctx->A.W * 2 : 0u;
        const size_t lds = static_cast<size_t>(pq_tree_block_lds_words(ctx->A.W, cap, top)) * 4;
        if (lds > kLdsBudget) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "tree descent needs %zu bytes of LDS", lds);
        int rc;
        if (lds > 64 * 1024 && (rc = raise_lds_limit(ctx, reinterpret_cast<const void*>(pq_tree_block_kernel), lds)))
            return rc;
        hipLaunchKernelGGL(pq_tree_block_kernel, dim3(K.nq), dim3(kPqTreeBlock), lds, ctx->stream, ctx->A, ctx->Wk, K,
                           ctx->tree, ctx->d_beams, cap, top);
        HIP_TRY(ctx, hipGetLastError());
        return 0;
    }
    const uint32_t words = pq_tree_lds_words(ctx->A.W, cap);
    const uint32_t per_wave = (words * 4 + 15) & ~15u;
    const size_t lds = static_cast<size_t>(per_wave) * kPqTreeWaves;
    if (lds > kLdsBudget) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "tree descent needs %zu bytes of LDS", lds);
    int rc;
    if (lds > 64 * 1024 && (rc = raise_lds_limit(ctx, reinterpret_cast<const void*>(pq_tree_kernel), lds))) return rc;
    hipLaunchKernelGGL(pq_tree_kernel, dim3((K.nq + kPqTreeWaves - 1) / kPqTreeWaves), dim3(kPqTreeWaves * kWave), lds,
                       ctx->stream, ctx->A, ctx->Wk, K, ctx->tree, ctx->d_beams, cap, per_wave);
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

// The per-query path's prep, tree descent and route in one launch (pq_front_kernel), two
// workgroups per query; the counters must be clear.
int launch_pq_front(maivs_gpu_ctx* ctx, const KParams& K, const float* d_q, uint32_t cap) {
    const DevArena& A = ctx->A;
    uint32_t top = 0;
    if (K.tree_list) {
        const uint32_t top_n = ctx->tree_level_n.empty() ? 0u : ctx->tree_level_n[0];
        top = top_n * A.W * 2 <= kTreeTopWords ? top_n * A.W * 2 : 0u;
    }
    // the region kept across the phases (cqs, leaves, bounds) when it fits beside the rest
    const size_t base = pq_front_keep_off(A.P, A.npos, A.d, A.W, A.Mp, K.sort_cap, K.nprobe, cap, top);
    const uint32_t keep = base + pq_front_keep_bytes(A.d, K.tcap) <= kLdsBudget ? 1u : 0u;
    const size_t lds = keep ? base + pq_front_keep_bytes(A.d, K.tcap) : base;
    if (lds > kLdsBudget) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "the fused route needs %zu bytes of LDS", lds);
    int rc = 0;
    auto go = [&](const void* fn, auto kernel) -> int {
        int r;
        if (lds > 64 * 1024 && (r = raise_lds_limit(ctx, fn, lds))) return r;
        hipLaunchKernelGGL(kernel, dim3(2 * K.nq), dim3(kPqTreeBlock), lds, ctx->stream, A, ctx->Wk, K, d_q, ctx->tree,
                           ctx->d_beams, cap, top, keep);
        return 0;
    };
    DISPATCH_NW(A.W, rc = go(reinterpret_cast<const void*>(pq_front_kernel<NW>), pq_front_kernel<NW>));
    if (rc) return rc;
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

KParams make_params(maivs_gpu_ctx* ctx, uint32_t nq, const maivs_search_params* p) {
    const DevArena& A = ctx->A;
    KParams K{};
    K.nq = nq;
    K.k = p->k;
    K.nprobe = p->nprobe;
    K.want_c = std::min<uint32_t>(p->nprobe * std::max<uint32_t>(p->shortlist_mult, 2u), A.n_live);
    K.target = std::max<uint32_t>(p->k * std::max<uint32_t>(p->rerank_factor, 1u), 1u);
    K.adaptive = p->adaptive;
    // shortlist sort on chip: room for 4x want_c (ties included), at least 1024 entries
    uint32_t sc = 1024;
    while (sc < 4u * K.want_c && sc < ctx->max_sort_cap_route) sc <<= 1;
    K.sort_cap = std::min(sc, ctx->max_sort_cap_route);
    K.use_nucleus = p->target_confidence < 1.0f;
    K.seed_cap = ctx->cap_seed;
    K.bucket_cap = ctx->cap_bucket;
    // The seed stage scans every rest cell itself, query-major, when there are at most 8 per query
    // (nprobe <= 16) and the batch shares them little (under kFrontRestShare probes per live cell):
    // the cell-major scan is then not launched at all. Past that its 4-query tables pay off.
    {
        const double rest = p->nprobe > kSeedCells ? static_cast<double>(p->nprobe - kSeedCells) : 0.0;
        const double per_cell = static_cast<double>(nq) * rest / std::max<uint32_t>(A.n_live, 1u);
        const bool front = p->nprobe <= kSeedCells + kFrontRestMax && per_cell < kFrontRestShare;
        K.front_rest = ctx->front_rest_mode >= 0 ? static_cast<uint32_t>(std::min<int>(ctx->front_rest_mode, kFrontRestMax))
                                                 : (front ? kFrontRestMax : 0u);
        // work items of at least mma_min queries run on the matrix cores, when cells gather
        // enough queries of the batch for such items to be common
        const double scan_rest = p->nprobe > kSeedCells + K.front_rest ? static_cast<double>(p->nprobe - kSeedCells - K.front_rest) : 0.0;
        const double scan_per_cell = static_cast<double>(nq) * scan_rest / std::max<uint32_t>(A.n_live, 1u);
        K.mma_min = ctx->mma_min_mode >= 0 ? static_cast<uint32_t>(std::min<int>(ctx->mma_min_mode, kBucketQ))
                                           : (scan_per_cell >= kMmaShare ? kMmaMinQ : 0u);
    }
    K.cand_cap = ctx->cap_cand;
    K.fin_cap = ctx->cap_fin;
    K.key_cap = ctx->cap_key;
    K.xcd_order = ctx->xcd_order ? 1u : 0u;
    // the running cut only where a cell-major scan runs after the seed stage
    K.run_thr = p->nprobe > kSeedCells + K.front_rest ? 1u : 0u;
    K.tc = p->target_confidence;
    K.beta = p->beta;
    K.at_margin = p->at_margin;
    K.filter = (p->filter && A.entry_tag) ? 1u : 0u;
    K.tag_lo = p->tag_lo;
    K.tag_hi = p->tag_hi;
    // norm = sqrt(2 * dim_pad / pi) in f32 (src/index.rs:2169)
    K.norm = std::sqrt(2.0f * static_cast<float>(A.P) / static_cast<float>(M_PI));
    K.prune_band = kPruneBand;
    K.nucleus_band = kNucleusBand;
    K.bnd_from = kSeedCells;
    K.tcap = 1;
    return K;
}

// The routing of a call (src/index.rs:1168-1305, 1873-1877), into K's routing fields. Batched
// (search_batch_cellmajor): the two-stage shortlist when p->route_mode is 0 (route_batch), else
// route_query's routing, the tree when the arena has one, else every live cell. Per query
// (search_one, route_query): the tree first, then the two-stage shortlist (route_mode 0), then every
// live cell. With the tree, *beams receives the descent's beam per level.
int route_setup(maivs_gpu_ctx* ctx, const maivs_search_params* p, bool batched, KParams& K,
                std::vector<uint32_t>* beams) {
    const DevArena& A = ctx->A;
    const bool tree = ctx->tree.n_levels > 0 && (!batched || p->route_mode != 0);
    const bool two = !tree && p->route_mode == 0;
    if (beams) beams->clear();
    K.tree_list = 0;
    K.flat_route = 0;
    K.tcap = 1;
    auto sort_room = [&](uint32_t need) {
        uint32_t sc = 1024;
        while (sc < need && sc < ctx->max_sort_cap_route) sc <<= 1;
        K.sort_cap = std::min(sc, ctx->max_sort_cap_route);
    };
    if (two) {
        if (!A.cent_bits)
            return fail(ctx, MAIVS_ERR_ARG, "route_mode 0 (two-stage routing) needs the arena's centroid codes");
        // route_batch keeps nprobe * max(mult, 2) cells, route_query's branch nprobe * mult (:1886, 1245)
        K.want_c = std::min<uint32_t>(p->nprobe * (batched ? std::max<uint32_t>(p->shortlist_mult, 2u) : p->shortlist_mult),
                                      A.n_live);
        sort_room(4u * K.want_c);
        return 0;
    }
    if (tree) {
        // the tree keeps nprobe * max(mult, 2) leaves (:1194)
        K.want_c = std::min<uint32_t>(p->nprobe * std::max<uint32_t>(p->shortlist_mult, 2u), ctx->tree.n_leaf);
        sort_room(4u * K.want_c);
        K.tree_list = 1;
        K.tcap = std::max(K.want_c, 1u);
        if (ctx->tree_level_n.size() > kPqMaxLevels) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "tree deeper than %u", kPqMaxLevels);
        if (beams) {
            beams->resize(ctx->tree_level_n.size());
            tree_beams(ctx->tree_level_n.data(), static_cast<uint32_t>(beams->size()), ctx->tree_beam_frac,
                       ctx->tree_min_beam, K.want_c, beams->data());
        }
        return 0;
    }
    // every live cell is rescored and sorted on chip
    if (A.n_live > ctx->max_sort_cap_route)
        return fail(ctx, MAIVS_ERR_UNSUPPORTED,
                    "routing over every live cell sorts at most %u cells on chip, this arena has %u (use two-stage "
                    "routing or a centroid tree)",
                    ctx->max_sort_cap_route, A.n_live);
    K.want_c = A.n_live;
    K.flat_route = 1;
    sort_room(A.n_live);
    return 0;
}

// Copies the tree descent's beams to d_beams when they differ from what it holds.
int upload_beams(maivs_gpu_ctx* ctx, const std::vector<uint32_t>& beams) {
    if (beams.empty() || beams == ctx->beams_on_device) return 0;
    HIP_TRY(ctx, hipMemcpyAsync(ctx->d_beams, beams.data(), beams.size() * 4, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));  // the host vector is about to go
    ctx->beams_on_device = beams;
    return 0;
}

// ---- host re-evaluation of libm-sensitive decisions (the reference's libm, same host) ----

// Nucleus count of src/index.rs:1960-1973 over a sorted score list.
uint32_t host_nucleus(const float* cs, uint32_t cap, float tc, float beta) {
    if (cap == 0) return 0;
    float max_s = cs[0];
    float z = -0.0f;
    for (uint32_t i = 0; i < cap; ++i) z += std::exp((cs[i] - max_s) * beta);
    float cum = 0.0f;
    for (uint32_t i = 0; i < cap; ++i) {
        cum += std::exp((cs[i] - max_s) * beta) / (z + 1e-9f);
        if (cum >= tc) return i + 1;
    }
    return cap;
}

// Adaptive probe cut of src/index.rs:2166-2188 for one query.
uint32_t host_rest_end(const float* cscore, const uint32_t* chosen, uint32_t nch, uint32_t ns, const float* r_bound,
                       float T) {
    std::vector<float> suffix(nch + 1, -INFINITY);
    for (uint32_t i = nch; i-- > ns;) {
        float cs = std::fmin(std::fmax(cscore[i], -1.0f), 1.0f);
        float ang = std::acos(cs);
        float b = std::cos(std::fmax(ang - r_bound[chosen[i]], 0.0f));
        suffix[i] = std::fmax(b, suffix[i + 1]);
    }
    for (uint32_t i = ns; i < nch; ++i)
        if (suffix[i] < T) return i;
    return nch;
}

// ---- pipeline stages ----

int launch_reset(maivs_gpu_ctx* ctx, uint32_t nq) {
    const uint32_t n = std::max(ctx->A.M + 1, nq);
    const uint32_t blocks = std::min<uint32_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(reset_kernel, dim3(std::max(blocks, 1u)), dim3(256), 0, ctx->stream, ctx->Wk, ctx->A.M, nq);
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

int launch_prep(maivs_gpu_ctx* ctx, const KParams& K, const float* d_q, uint32_t flags) {
    const DevArena& A = ctx->A;
    const uint32_t blocks = (K.nq + kPrepWaves - 1) / kPrepWaves;
    DISPATCH_EPL(A.P / 64, hipLaunchKernelGGL(prep_kernel<EPL>, dim3(blocks), dim3(kPrepWaves * kWave), ctx->lds_prep,
                                              ctx->stream, A, ctx->Wk, K, d_q, flags));
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

// The per-query route alone (needs the Hamming rows of prep).
int launch_route(maivs_gpu_ctx* ctx, const KParams& K) {
    const DevArena& A = ctx->A;
    const size_t lds = route_lds(A, K.sort_cap, K.nprobe);
    DISPATCH_NW(A.W, hipLaunchKernelGGL(route_kernel<NW>, dim3(K.nq), dim3(kRouteThreads), lds, ctx->stream, A,
                                        ctx->Wk, K));
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

// Prep, route and seed fused, one workgroup per query (the counters are reset beforehand).
int launch_front(maivs_gpu_ctx* ctx, const KParams& K, const float* d_q) {
    const DevArena& A = ctx->A;
    const size_t lds = std::max(route_lds(A, K.sort_cap, K.nprobe) + prep1_lds(A), ctx->lds_seed);
    DISPATCH_NW(A.W, hipLaunchKernelGGL(front_kernel<NW>, dim3(K.nq), dim3(kSeedThreads), lds, ctx->stream, A,
                                        ctx->Wk, K, d_q));
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

// Route and seed fused, one workgroup per query. rows_ready: hamming_kernel wrote the Hamming rows.
int launch_route_seed(maivs_gpu_ctx* ctx, const KParams& K, bool rows_ready = false) {
    const DevArena& A = ctx->A;
    const size_t lds = std::max(route_lds(A, K.sort_cap, K.nprobe), ctx->lds_seed);
    if (rows_ready) {
        DISPATCH_NW(A.W, hipLaunchKernelGGL((route_seed_kernel<NW, true>), dim3(K.nq), dim3(kSeedThreads), lds,
                                            ctx->stream, A, ctx->Wk, K));
    } else {
        DISPATCH_NW(A.W, hipLaunchKernelGGL((route_seed_kernel<NW, false>), dim3(K.nq), dim3(kSeedThreads), lds,
                                            ctx->stream, A, ctx->Wk, K));
    }
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

// The Hamming rows of every query (indexes with more cells than a route keeps in LDS).
int launch_hamming(maivs_gpu_ctx* ctx, uint32_t nq) {
    const DevArena& A = ctx->A;
    if (ctx->ham_mma) {
        // on the matrix cores: 128 queries x 256 cells per workgroup
        const dim3 grid((nq + kHamMmaQ - 1) / kHamMmaQ, (A.Mp + kHamMmaC - 1) / kHamMmaC);
        DISPATCH_NW(A.W, hipLaunchKernelGGL(hamming_mma_kernel<NW>, grid, dim3(256), 0, ctx->stream, A, ctx->Wk, nq));
        HIP_TRY(ctx, hipGetLastError());
        return 0;
    }
    const dim3 grid((nq + kHamQ - 1) / kHamQ, (A.Mp + kHamC - 1) / kHamC);
    DISPATCH_NW(A.W, hipLaunchKernelGGL(hamming_kernel<NW>, grid, dim3(kHamC), 0, ctx->stream, A, ctx->Wk, nq));
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

int launch_seed(maivs_gpu_ctx* ctx, const KParams& K) {
    const DevArena& A = ctx->A;
    DISPATCH_NW(A.W, hipLaunchKernelGGL(seed_kernel<NW>, dim3(K.nq), dim3(kSeedThreads), ctx->lds_seed,
                                        ctx->stream, A, ctx->Wk, K));
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

// The cell-major scan. In bucket mode (K.bucket_cap > 0) the seed stage already filed every
// query into its cells' buckets. Otherwise the counting-sort inversion runs first, from the seed
// stage's probe counts, or from invert_count when the cuts changed afterwards (recount = true,
// counters reset first).
int launch_scan(maivs_gpu_ctx* ctx, const KParams& K, bool recount, bool events = false) {
    const DevArena& A = ctx->A;
    Work& W = ctx->Wk;
    if (!K.bucket_cap) {
        if (recount) {
            int rc = launch_reset(ctx, K.nq);
            if (rc) return rc;
            hipLaunchKernelGGL(invert_count_kernel, dim3(K.nq), dim3(64), 0, ctx->stream, W, K);
        }
        hipLaunchKernelGGL(invert_scan_kernel, dim3(1), dim3(1024), 0, ctx->stream, W, A.M);
        hipLaunchKernelGGL(invert_fill_kernel, dim3(K.nq), dim3(64), 0, ctx->stream, W, K);
        HIP_TRY(ctx, hipGetLastError());
    }
    if (events) HIP_TRY(ctx, hipEventRecord(ctx->ev[4], ctx->stream));
    // bucket mode: a grid that strides over the work items (their count is on the device)
    const uint64_t items = static_cast<uint64_t>(A.M) + static_cast<uint64_t>(K.nq) * K.nprobe / kBucketQ + 1;
    const uint32_t grid = K.bucket_cap ? static_cast<uint32_t>(std::min<uint64_t>(items, kScanGridMax)) : A.M;
    const uint64_t items8 = static_cast<uint64_t>(A.M) + static_cast<uint64_t>(K.nq) * K.nprobe / kItemQ + 1;
    const uint32_t sgrid = K.bucket_cap ? static_cast<uint32_t>(std::min<uint64_t>(items8, kScanGridMax)) : A.M;
    // the lookup scan, unless the matrix-core scan takes every bucket work item
    if (!(K.bucket_cap && K.mma_min == 1)) {
        DISPATCH_NW(A.W, hipLaunchKernelGGL(cell_scan_kernel<NW>, dim3(std::max(sgrid, 1u)), dim3(kScanThreads), 0,
                                            ctx->stream, A, W, K));
        HIP_TRY(ctx, hipGetLastError());
    }
    // the items with many queries, on the matrix cores (in cell order, by XCD)
    if (K.bucket_cap && K.mma_min) {
        if (K.xcd_order) {
            hipLaunchKernelGGL(order_items_kernel, dim3(1), dim3(1024), 0, ctx->stream, W, K, A.M);
            HIP_TRY(ctx, hipGetLastError());
        }
        DISPATCH_NW(A.W, hipLaunchKernelGGL(cell_mma_kernel<NW>, dim3(std::max(grid, 1u)), dim3(kScanThreads), 0,
                                            ctx->stream, A, W, K));
        HIP_TRY(ctx, hipGetLastError());
    }
    return 0;
}

// The same parameters with the counting-sort inversion instead of the buckets, and every rest
// cell left to the cell-major scan (every re-run).
KParams csr(KParams K) {
    K.bucket_cap = 0;
    K.front_rest = 0;
    K.mma_min = 0;
    return K;
}

int launch_pad(maivs_gpu_ctx* ctx, uint32_t* d_slots, float* d_scores, uint64_t n) {
    const uint32_t blocks = static_cast<uint32_t>(std::min<uint64_t>((n + 255) / 256, 1024));
    hipLaunchKernelGGL(pad_kernel, dim3(std::max(blocks, 1u)), dim3(256), 0, ctx->stream, d_slots, d_scores, n);
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

int launch_finish(maivs_gpu_ctx* ctx, const KParams& K, const float* d_q, uint32_t* d_slots, float* d_scores) {
    if (K.nq <= ctx->finish_wide_max_q)
        hipLaunchKernelGGL(finish_kernel<kFinishWideThreads>, dim3(K.nq), dim3(kFinishWideThreads), ctx->lds_finish,
                           ctx->stream, ctx->A, ctx->Wk, K, d_q, d_slots, d_scores);
    else
        hipLaunchKernelGGL(finish_kernel<kFinishThreads>, dim3(K.nq), dim3(kFinishThreads), ctx->lds_finish,
                           ctx->stream, ctx->A, ctx->Wk, K, d_q, d_slots, d_scores);
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

// The per-query path's finish: for small batches whose candidate lists the scan cut to the target
// (the FastScan branch), the rerank over workgroups of kRerankRows rows and then the top k
// (pq_rerank_kernel, pq_topk_kernel); else finish_kernel.
int launch_pq_finish(maivs_gpu_ctx* ctx, const KParams& K, const float* d_q, uint32_t* d_slots, float* d_scores) {
    if (K.nq > ctx->pq_finish_split_max_q || K.pq_ham) return launch_finish(ctx, K, d_q, d_slots, d_scores);
    const uint32_t groups = (K.target + kRerankRows - 1) / kRerankRows;
    hipLaunchKernelGGL(pq_rerank_kernel, dim3(groups, K.nq), dim3(kRerankRows * 8), ((ctx->A.d + 3) & ~3u) * 4,
                       ctx->stream, ctx->A, ctx->Wk, K, d_q);
    hipLaunchKernelGGL(pq_topk_kernel, dim3(K.nq), dim3(kFinishThreads), kFinishLdsCap * 8 + 32 * 4, ctx->stream,
                       ctx->A, ctx->Wk, K, d_slots, d_scores);
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

// Fetch one query's probe list and scores (host check helpers).
int fetch_probe_list(maivs_gpu_ctx* ctx, uint32_t qi, uint32_t nprobe, std::vector<float>& cs,
                     std::vector<uint32_t>& ch) {
    cs.resize(nprobe);
    ch.resize(nprobe);
    HIP_TRY(ctx, hipMemcpy(cs.data(), ctx->Wk.cscore + static_cast<uint64_t>(qi) * nprobe, nprobe * 4,
                           hipMemcpyDeviceToHost));
    HIP_TRY(ctx, hipMemcpy(ch.data(), ctx->Wk.chosen + static_cast<uint64_t>(qi) * nprobe, nprobe * 4,
                           hipMemcpyDeviceToHost));
    return 0;
}

// The control block of a pass that ended with finish_kernel: its epilogue mirrored the block to
// pinned host memory and cleared the counters, so this only waits for the stream.
int read_ctl(maivs_gpu_ctx* ctx, Ctl* ctl) {
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    *ctl = *ctx->h_ctl;
    ctx->counters_clean = true;
    return 0;
}

// The live control block (after kernels other than finish_kernel; the counters stay set).
int read_ctl_live(maivs_gpu_ctx* ctx, Ctl* ctl) {
    ctx->counters_clean = false;
    HIP_TRY(ctx, hipMemcpyAsync(ctx->h_ctl, ctx->Wk.ctl, sizeof(Ctl), hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    *ctl = *ctx->h_ctl;
    return 0;
}

// A fixed device region the work buffers are carved from instead of the context's allocations
// (the no-allocation entry point): the candidate buffers start at cand_off.
struct Scratch {
    uint8_t* base;
    size_t bytes;
    size_t cand_off;
};

// Re-carve the candidate buffers of a scratch-backed call for cand_cap candidates per query.
int recarve_cand(maivs_gpu_ctx* ctx, const Scratch& sc, uint32_t cand_cap) {
    Carver c{nullptr};
    c.used = sc.cand_off;
    Work W = ctx->Wk;
    carve_cand(ctx->cap_nq, ctx->cap_seed, cand_cap, c, W);
    if (c.used > sc.bytes)
        return fail(ctx, MAIVS_ERR_UNSUPPORTED,
                    "%u candidates per query for %u queries need %zu bytes of scratch, more than its %zu", cand_cap,
                    ctx->cap_nq, c.used, sc.bytes);
    Carver cv{sc.base};
    cv.used = sc.cand_off;
    carve_cand(ctx->cap_nq, ctx->cap_seed, cand_cap, cv, ctx->Wk);
    ctx->cap_cand = cand_cap;
    cand_caps(ctx->cap_seed, cand_cap, &ctx->cap_fin, &ctx->cap_key);
    return 0;
}

// The whole batch. Stages after the first pass only re-run when the control block asks:
// (1) a nucleus decision within kNucleusBand of tc, (2) an adaptive cut within kPruneBand of its
// threshold (both re-evaluated with the host libm the reference uses), (3) a candidate buffer
// overflow (grown to the exact count), (4) a shortlist larger than the on-chip sort.
// With a scratch region (sc), the work buffers were carved from it beforehand: nothing is
// allocated, the stages run eagerly (no graph), and a candidate overflow re-carves within it.
int run_search(maivs_gpu_ctx* ctx, const float* d_q, uint32_t nq, const maivs_search_params* p, uint32_t* d_slots,
               float* d_scores, maivs_gpu_stats* st, const Scratch* sc = nullptr) {
    if (!ctx->uploaded) return fail(ctx, MAIVS_ERR_NOT_UPLOADED, "no arena uploaded");
    if (p->k == 0) return fail(ctx, MAIVS_ERR_ARG, "k must be > 0");
    const DevArena& A = ctx->A;
    if (!A.fs)
        return fail(ctx, MAIVS_ERR_UNSUPPORTED,
                    "the batched path scans FastScan blocks; this arena has per-slot codes only (not compacted)");
    int rc = sc ? 0 : ensure_all(ctx, nq, p->nprobe, p->k);
    if (rc) return rc;
    Work& W = ctx->Wk;
    maivs_gpu_stats local{};
    maivs_gpu_stats& S = st ? *st : local;
    S = maivs_gpu_stats{};
    ctx->last_nq = 0;
    if (nq == 0) return 0;
    KParams K = make_params(ctx, nq, p);
    std::vector<uint32_t> beams;
    if ((rc = route_setup(ctx, p, true, K, &beams))) return rc;
    const bool two_stage = !K.tree_list && !K.flat_route;
    uint32_t tree_cap = 1;
    for (uint32_t b : beams) tree_cap = std::max(tree_cap, b);
    if (p->nprobe == 0 || K.want_c == 0) {
        // route_batch returns empty probe lists (src/index.rs:1887-1889): padded results
        if ((rc = launch_pad(ctx, d_slots, d_scores, static_cast<uint64_t>(nq) * p->k))) return rc;
        HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        return 0;
    }
    if (K.tree_list) {
        // the descent's leaf lists (a scratch-backed call has them carved already) and beams
        if (!sc && (rc = ensure_pq(ctx, nq, K.tcap, 0))) return rc;
        if ((rc = upload_beams(ctx, beams))) return rc;
    }
    Ctl ctl{};
    // the main pass; run eagerly it has an event between stages (the per-stage device times)
    auto enqueue_main = [&](bool events) -> int {
        int r;
        auto mark = [&](int i) -> int {
            if (events) HIP_TRY(ctx, hipEventRecord(ctx->ev[i], ctx->stream));
            return 0;
        };
        if (!two_stage) {
            // route_query's routing (src/index.rs:2105-2124): prep, the tree's descent, then route
            // (the tree's leaves or every live cell, rescored) and seed
            if ((r = mark(0)) || (r = launch_prep(ctx, K, d_q, kPrepReset))) return r;
            if (K.tree_list && (r = launch_pq_tree(ctx, K, tree_cap))) return r;
            if ((r = mark(3)) || (r = launch_route_seed(ctx, K)) || (r = mark(2))) return r;
        } else if (ctx->A.Mp > kHdLdsCells || ctx->rows_pass) {
            // many cells: Hamming rows by query tiles, then route and seed from them
            if ((r = mark(0)) || (r = launch_prep(ctx, K, d_q, 0)) || (r = launch_hamming(ctx, K.nq)) || (r = mark(3)))
                return r;
            if ((r = launch_route_seed(ctx, K, true)) || (r = mark(2))) return r;
        } else if (fused_front(ctx->A)) {
            // the counters are clear: the previous pass's epilogue (or a clearing launch) did it
            if ((r = mark(0)) || (r = mark(3))) return r;
            if ((r = launch_front(ctx, K, d_q)) || (r = mark(2))) return r;
        } else {
            if ((r = mark(0)) || (r = launch_prep(ctx, K, d_q, kPrepReset)) || (r = mark(3))) return r;
            if ((r = launch_route_seed(ctx, K)) || (r = mark(2))) return r;
        }
        // with at most SEED_CELLS + front_rest probes the seed stage scanned every rest cell itself
        if (K.nprobe > kSeedCells + K.front_rest) {
            if ((r = launch_scan(ctx, K, false, events)) || (r = mark(5))) return r;
        } else if ((r = mark(4)) || (r = mark(5))) {
            return r;
        }
        if ((r = launch_finish(ctx, K, d_q, d_slots, d_scores)) || (r = mark(6))) return r;
        return 0;
    };
    bool staged = true;  // per-stage events recorded (eager pass)
    // replayed as one captured graph when possible (one launch instead of a dozen); the capture
    // is keyed by the parameters and every buffer address it bakes in
    auto run_main = [&]() -> int {
        if (ctx->use_graph && !sc) {
            maivs_gpu_ctx::GraphKey key{};
            key.K = K;
            key.q = d_q;
            key.slots = d_slots;
            key.scores = d_scores;
            key.gen = ctx->buf_gen;
            const auto& g0 = ctx->gkey;
            const bool same = ctx->gexec && std::memcmp(&key.K, &g0.K, sizeof(KParams)) == 0 && key.q == g0.q &&
                              key.slots == g0.slots && key.scores == g0.scores && key.gen == g0.gen;
            if (!same) {
                if (ctx->gexec) (void)hipGraphExecDestroy(ctx->gexec);
                ctx->gexec = nullptr;
                hipGraph_t g = nullptr;
                bool ok = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed) == hipSuccess;
                int r = ok ? enqueue_main(false) : 0;
                if (ok) ok = hipStreamEndCapture(ctx->stream, &g) == hipSuccess && r == 0 && g;
                if (ok) ok = hipGraphInstantiate(&ctx->gexec, g, nullptr, nullptr, 0) == hipSuccess;
                if (g) (void)hipGraphDestroy(g);
                (void)hipGetLastError();
                if (!ok) {  // capture is unavailable: run the stages eagerly from now on
                    if (ctx->gexec) (void)hipGraphExecDestroy(ctx->gexec);
                    ctx->gexec = nullptr;
                    ctx->use_graph = false;
                    staged = st != nullptr;
                    return enqueue_main(staged);
                }
                ctx->gkey = key;
            }
            // whole-pass time only (events recorded inside a graph do not time stages), and only
            // when the caller asks for measurements
            staged = false;
            if (st) HIP_TRY(ctx, hipEventRecord(ctx->ev[0], ctx->stream));
            HIP_TRY(ctx, hipGraphLaunch(ctx->gexec, ctx->stream));
            if (st) HIP_TRY(ctx, hipEventRecord(ctx->ev[6], ctx->stream));
            return 0;
        }
        // eager launches; the per-stage events only when the caller asks for measurements
        staged = st != nullptr;
        return enqueue_main(staged);
    };
    for (;;) {
        if (!ctx->counters_clean && (rc = launch_reset(ctx, nq))) return rc;
        ctx->counters_clean = false;
        if ((rc = run_main())) return rc;
        if ((rc = read_ctl(ctx, &ctl))) return rc;
        if (ctl.err_shortlist && K.sort_cap < ctx->max_sort_cap_route) {
            K.sort_cap = ctx->max_sort_cap_route;  // ties at the Hamming cut: retry with the largest sort
            S.reruns++;
            continue;
        }
        break;
    }
    if (ctl.err_shortlist)
        return fail(ctx, MAIVS_ERR_UNSUPPORTED,
                    "a routing shortlist of %u cells exceeds the on-chip sort capacity %u (lower nprobe)",
                    ctl.max_shortlist, ctx->max_sort_cap_route);
    if (ctl.err_seed) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "a seed set exceeds its on-chip capacity");
    float ms;
    if ((st || staged) && hipEventElapsedTime(&ms, ctx->ev[0], ctx->ev[6]) == hipSuccess) S.ms_total = ms;
    if (staged) {
        if (hipEventElapsedTime(&ms, ctx->ev[0], ctx->ev[3]) == hipSuccess) S.ms_prep = ms;
        if (hipEventElapsedTime(&ms, ctx->ev[3], ctx->ev[2]) == hipSuccess) S.ms_route = ms;
        if (hipEventElapsedTime(&ms, ctx->ev[2], ctx->ev[4]) == hipSuccess) S.ms_invert = ms;
        if (hipEventElapsedTime(&ms, ctx->ev[4], ctx->ev[5]) == hipSuccess) S.ms_scan = ms;
        if (hipEventElapsedTime(&ms, ctx->ev[5], ctx->ev[6]) == hipSuccess) S.ms_rerank = ms;
    }
    (void)hipGetLastError();  // a failed timing query must not surface as a later call's error

    std::vector<float> cs;
    std::vector<uint32_t> ch;
    // (1) nucleus decisions near tc
    if (ctl.nflag_route) {
        std::vector<uint32_t> fl(ctl.nflag_route);
        HIP_TRY(ctx, hipMemcpy(fl.data(), W.flag_route, fl.size() * 4, hipMemcpyDeviceToHost));
        bool fixed = false;
        for (uint32_t qi : fl) {
            uint32_t nch;
            HIP_TRY(ctx, hipMemcpy(&nch, W.nchosen + qi, 4, hipMemcpyDeviceToHost));
            if ((rc = fetch_probe_list(ctx, qi, p->nprobe, cs, ch))) return rc;
            uint32_t cap = 0;
            while (cap < p->nprobe && ch[cap] != kNone) ++cap;
            uint32_t exact = host_nucleus(cs.data(), cap, p->target_confidence, p->beta);
            S.host_checks++;
            if (exact != nch) {
                S.host_fixes++;
                HIP_TRY(ctx, hipMemcpy(W.nchosen + qi, &exact, 4, hipMemcpyHostToDevice));
                fixed = true;
            }
        }
        if (fixed) {
            S.reruns++;
            if ((rc = launch_reset(ctx, nq))) return rc;
            if ((rc = launch_seed(ctx, csr(K)))) return rc;
            if ((rc = launch_scan(ctx, csr(K), false))) return rc;
            if ((rc = launch_finish(ctx, csr(K), d_q, d_slots, d_scores))) return rc;
            if ((rc = read_ctl(ctx, &ctl))) return rc;
            if (ctl.err_seed) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "a seed set exceeds its on-chip capacity");
        }
    }
    // (2) adaptive cuts near their threshold; a full query bucket re-runs the scan from the
    // counting-sort inversion
    bool rerun_scan = ctl.bucket_overflow != 0;
    bool cells_changed = false;  // a re-run scans other cells than the running cuts were counted on
    if (ctl.nflag_prune) {
        std::vector<uint32_t> fl(ctl.nflag_prune);
        HIP_TRY(ctx, hipMemcpy(fl.data(), W.flag_prune, fl.size() * 4, hipMemcpyDeviceToHost));
        for (uint32_t qi : fl) {
            uint32_t nch, tau, re;
            float delta, bias;
            HIP_TRY(ctx, hipMemcpy(&nch, W.nchosen + qi, 4, hipMemcpyDeviceToHost));
            HIP_TRY(ctx, hipMemcpy(&tau, W.tau + qi, 4, hipMemcpyDeviceToHost));
            HIP_TRY(ctx, hipMemcpy(&re, W.rest_end + qi, 4, hipMemcpyDeviceToHost));
            HIP_TRY(ctx, hipMemcpy(&delta, W.delta + qi, 4, hipMemcpyDeviceToHost));
            HIP_TRY(ctx, hipMemcpy(&bias, W.bias + qi, 4, hipMemcpyDeviceToHost));
            if ((rc = fetch_probe_list(ctx, qi, p->nprobe, cs, ch))) return rc;
            float est = delta * static_cast<float>(A.maxk - tau) + bias;
            float thr = std::fmin(std::fmax(est / K.norm, -1.0f), 1.0f);
            uint32_t ns = std::min(kSeedCells, nch);
            uint32_t exact = host_rest_end(cs.data(), ch.data(), nch, ns, ctx->h_r_bound.data(), thr - p->at_margin);
            S.host_checks++;
            if (exact != re) {
                S.host_fixes++;
                HIP_TRY(ctx, hipMemcpy(W.rest_end + qi, &exact, 4, hipMemcpyHostToDevice));
                rerun_scan = true;
                cells_changed = true;
            }
        }
    }
    // (3) candidate overflow: grow to the exact count (cand_cnt counts past the capacity)
    if (ctl.max_cand > ctx->cap_cand) {
        uint32_t need = ctl.max_cand + ctl.max_cand / 4 + 64;
        ctx->initial_cand_cap = std::max(ctx->initial_cand_cap, need);
        if ((rc = sc ? recarve_cand(ctx, *sc, need) : ensure_cand(ctx, need))) return rc;
        K.cand_cap = ctx->cap_cand;
        K.fin_cap = ctx->cap_fin;
        K.key_cap = ctx->cap_key;
        rerun_scan = true;
    }
    if (rerun_scan) {
        // the same cells: the running cuts as they stand (their entries were counted); other cells:
        // tau. A re-run under a higher cut may append more than the buffer took: it grows once more.
        K.run_thr = K.run_thr && !cells_changed ? 2u : 0u;
        for (int attempt = 0;; ++attempt) {
            S.reruns++;
            if ((rc = launch_scan(ctx, csr(K), true))) return rc;
            if ((rc = launch_finish(ctx, csr(K), d_q, d_slots, d_scores))) return rc;
            if ((rc = read_ctl(ctx, &ctl))) return rc;
            if (ctl.max_cand <= ctx->cap_cand) break;
            if (attempt > 0) return fail(ctx, MAIVS_ERR_HIP, "candidate count changed between passes");
            const uint32_t need = ctl.max_cand + ctl.max_cand / 4 + 64;
            ctx->initial_cand_cap = std::max(ctx->initial_cand_cap, need);
            if ((rc = sc ? recarve_cand(ctx, *sc, need) : ensure_cand(ctx, need))) return rc;
            K.cand_cap = ctx->cap_cand;
            K.fin_cap = ctx->cap_fin;
            K.key_cap = ctx->cap_key;
        }
    }
    ctx->last_nq = nq;
    ctx->last_K = K;
    ctx->last_pq = false;
    return 0;
}

// ---------------------------------------------------------------- the per-query path

int launch_pq_scan(maivs_gpu_ctx* ctx, const KParams& K) {
    const DevArena& A = ctx->A;
    const uint32_t mode = K.pq_split ? 2u : K.pq_rounds ? 1u : 0u;
    const size_t lds =
        static_cast<size_t>(pq_scan_lds_words(A.MW, A.maxk, K.nprobe, A.W, K.pq_pair != 0, K.pq_ham != 0, mode)) * 4;
    const uint32_t threads = mode ? kScanRoundThreads : kScanThreads;
    if (lds + A.W * 256 + threads * 4 > kLdsBudget)
        return fail(ctx, MAIVS_ERR_UNSUPPORTED, "per-query scan needs %zu bytes of LDS", lds);
    auto go = [&](const void* fn, auto kernel) -> int {
        int rc;
        if (lds > 48 * 1024 && (rc = raise_lds_limit(ctx, fn, lds))) return rc;
        hipLaunchKernelGGL(kernel, dim3(K.nq), dim3(threads), lds, ctx->stream, A, ctx->Wk, K);
        return 0;
    };
    int rc = 0;
    if (K.pq_split) {
        // every probed cell by its own workgroup, then the bucket queue replayed per query
        const size_t lds1 = static_cast<size_t>(pq_cells_lds_words(A.MW, A.maxk, A.W, K.pq_ham != 0)) * 4;
        auto cells = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3(K.nprobe, K.nq), dim3(kScanThreads), lds1, ctx->stream, A, ctx->Wk, K);
        };
        if (K.pq_ham) {
            DISPATCH_NW(A.W, cells(pq_cells_kernel<NW, true>));
            DISPATCH_NW(A.W, rc = go(reinterpret_cast<const void*>(pq_scan_kernel<NW, true, 2>), pq_scan_kernel<NW, true, 2>));
        } else {
            DISPATCH_NW(A.W, cells(pq_cells_kernel<NW, false>));
            DISPATCH_NW(A.W, rc = go(reinterpret_cast<const void*>(pq_scan_kernel<NW, false, 2>), pq_scan_kernel<NW, false, 2>));
        }
    } else if (K.pq_ham && K.pq_rounds) {
        DISPATCH_NW(A.W, rc = go(reinterpret_cast<const void*>(pq_scan_kernel<NW, true, true>), pq_scan_kernel<NW, true, true>));
    } else if (K.pq_ham) {
        DISPATCH_NW(A.W, rc = go(reinterpret_cast<const void*>(pq_scan_kernel<NW, true>), pq_scan_kernel<NW, true>));
    } else if (K.pq_rounds) {
        DISPATCH_NW(A.W, rc = go(reinterpret_cast<const void*>(pq_scan_kernel<NW, false, true>), pq_scan_kernel<NW, false, true>));
    } else {
        DISPATCH_NW(A.W, rc = go(reinterpret_cast<const void*>(pq_scan_kernel<NW, false>), pq_scan_kernel<NW, false>));
    }
    if (rc) return rc;
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

// The per-query search of nq queries in device memory (search_one, src/index.rs:1381-1864).
int run_search_pq(maivs_gpu_ctx* ctx, const float* d_q, uint32_t nq, const maivs_search_params* p, uint32_t* d_slots,
                  float* d_scores, maivs_gpu_stats* st) {
    if (!ctx->uploaded) return fail(ctx, MAIVS_ERR_NOT_UPLOADED, "no arena uploaded");
    if (p->k == 0) return fail(ctx, MAIVS_ERR_ARG, "k must be > 0");
    if (p->nprobe > kPqMaxProbe)
        return fail(ctx, MAIVS_ERR_UNSUPPORTED, "the per-query path probes at most %u cells", kPqMaxProbe);
    const DevArena& A = ctx->A;
    maivs_gpu_stats local{};
    maivs_gpu_stats& S = st ? *st : local;
    S = maivs_gpu_stats{};
    ctx->last_nq = 0;
    if (nq == 0) return 0;
    int rc = ensure_all(ctx, nq, p->nprobe, p->k);
    if (rc) return rc;
    KParams K = make_params(ctx, nq, p);
    if (K.target > ctx->cap_cand) {
        if ((rc = ensure_cand(ctx, K.target))) return rc;
        K = make_params(ctx, nq, p);
    }
    // route_query: the tree, else the two-stage shortlist, else every live cell
    std::vector<uint32_t> beams;
    if ((rc = route_setup(ctx, p, false, K, &beams))) return rc;
    const bool tree = K.tree_list != 0;
    K.bnd_from = 0;
    K.pq_room = std::max(A.max_cell_len, 1u);
    // small batches scan their probed cells in rounds (a round appends up to kRoundBudget entries,
    // or one larger cell)
    // (codes of up to 512 bits: the widest codes would spill registers at 1024 threads)
    K.pq_rounds = nq <= ctx->pq_rounds_max_q && A.W <= 8 ? 1u : 0u;
    const uint32_t pq_need = std::max({4u * K.target + 1024u, 2u * K.pq_room + K.target, ctx->pq_cap_min,
                                       K.pq_rounds ? 2u * kRoundBudget + K.target : 0u});
    if ((rc = ensure_pq(ctx, nq, K.tcap, pq_need))) return rc;
    K.pq_cap = ctx->cap_pq;
    K.pq_noflag = 0;
    // without FastScan blocks: search_one's Hamming branch (src/index.rs:1694-1760)
    K.pq_ham = A.fs ? 0u : 1u;
    if (K.pq_rounds && pq_scan_lds_words(A.MW, A.maxk, K.nprobe, A.W, false, K.pq_ham != 0, 1) * 4 + A.W * 256 +
                               kScanRoundThreads * 4 >
                           kLdsBudget)
        K.pq_rounds = 0;
    // the split scan: small batches of at most kSplitMaxProbe probes whose per-cell buffers stay modest
    K.pq_split = 0;
    if (nq <= ctx->pq_split_max_q && A.W <= 8 && p->nprobe <= kSplitMaxProbe &&
        static_cast<uint64_t>(nq) * p->nprobe * K.pq_room * 8 <= kSplitMaxBytes &&
        pq_scan_lds_words(A.MW, A.maxk, K.nprobe, A.W, false, K.pq_ham != 0, 2) * 4 + A.W * 256 + kScanRoundThreads * 4 <=
            kLdsBudget) {
        K.pq_split = 1;
        if ((rc = ensure_split(ctx, nq, K.nprobe, K.pq_room, (pq_bins(A.maxk, A.W, K.pq_ham != 0) + 3) & ~3u))) return rc;
    }
    // small batches (at most one workgroup per CU) look up position pairs: half the LDS lookups
    K.pq_pair = !K.pq_ham && nq <= kPqPairMaxQ &&
                        pq_scan_lds_words(A.MW, A.maxk, K.nprobe, A.W, true, false, K.pq_rounds ? 1u : 0u) * 4 + A.W * 256 +
                                (K.pq_rounds ? kScanRoundThreads : kScanThreads) * 4 <=
                            kLdsBudget
                    ? 1u
                    : 0u;
    if (p->nprobe == 0) {
        if ((rc = launch_pad(ctx, d_slots, d_scores, static_cast<uint64_t>(nq) * p->k))) return rc;
        HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        return 0;
    }
    uint32_t cap = 1;
    for (uint32_t b : beams) cap = std::max(cap, b);
    // copied only when they change (they depend on the tree and want_c)
    if (tree && (rc = upload_beams(ctx, beams))) return rc;
    Work& W = ctx->Wk;
    // timed only when the caller asks for measurements
    if (st) HIP_TRY(ctx, hipEventRecord(ctx->ev[0], ctx->stream));
    // small batches with codes over the whole padded dimension: prep, descent and route in one
    // launch (the counters cleared beforehand only when the last pass left them set)
    const bool fused = nq <= ctx->pq_front_max_q && A.W * 64 == A.P;
    if (fused) {
        if (!ctx->counters_clean && (rc = launch_reset(ctx, nq))) return rc;
    } else if ((rc = launch_prep(ctx, K, d_q, kPrepReset))) {
        return rc;
    }
    ctx->counters_clean = false;  // the finish's epilogue clears them again
    for (;;) {
        if (fused) {
            if ((rc = launch_pq_front(ctx, K, d_q, cap))) return rc;
        } else {
            if (tree && (rc = launch_pq_tree(ctx, K, cap))) return rc;
            if ((rc = launch_route(ctx, K))) return rc;
        }
        if ((rc = launch_pq_scan(ctx, K)) || (rc = launch_pq_finish(ctx, K, d_q, d_slots, d_scores))) return rc;
        Ctl ctl{};
        if ((rc = read_ctl(ctx, &ctl))) return rc;
        if (ctl.err_shortlist && K.sort_cap < ctx->max_sort_cap_route) {
            K.sort_cap = ctx->max_sort_cap_route;
            S.reruns++;
            if ((rc = launch_reset(ctx, nq))) return rc;
            continue;
        }
        if (ctl.err_shortlist)
            return fail(ctx, MAIVS_ERR_UNSUPPORTED, "a routing shortlist of %u cells exceeds the on-chip sort capacity %u",
                        ctl.max_shortlist, ctx->max_sort_cap_route);
        // host checks of libm-sensitive decisions, then candidate-buffer growth; each re-runs the scan
        for (int pass = 0; pass < 4; ++pass) {
            bool rerun = false;
            std::vector<float> cs;
            std::vector<uint32_t> ch;
            if (ctl.nflag_route) {
                std::vector<uint32_t> fl(ctl.nflag_route);
                HIP_TRY(ctx, hipMemcpy(fl.data(), W.flag_route, fl.size() * 4, hipMemcpyDeviceToHost));
                for (uint32_t qi : fl) {
                    uint32_t nch;
                    HIP_TRY(ctx, hipMemcpy(&nch, W.nchosen + qi, 4, hipMemcpyDeviceToHost));
                    if ((rc = fetch_probe_list(ctx, qi, p->nprobe, cs, ch))) return rc;
                    uint32_t capn = 0;
                    while (capn < p->nprobe && ch[capn] != kNone) ++capn;
                    const uint32_t exact = host_nucleus(cs.data(), capn, p->target_confidence, p->beta);
                    S.host_checks++;
                    if (exact != nch) {
                        S.host_fixes++;
                        HIP_TRY(ctx, hipMemcpy(W.nchosen + qi, &exact, 4, hipMemcpyHostToDevice));
                        rerun = true;
                    }
                }
            }
            if (ctl.nflag_prune) {
                // the bounds of a flagged query with the host's libm acos / cos (src/index.rs:1476-1483)
                std::vector<uint32_t> fl(ctl.nflag_prune);
                HIP_TRY(ctx, hipMemcpy(fl.data(), W.flag_prune, fl.size() * 4, hipMemcpyDeviceToHost));
                for (uint32_t qi : fl) {
                    uint32_t nch;
                    HIP_TRY(ctx, hipMemcpy(&nch, W.nchosen + qi, 4, hipMemcpyDeviceToHost));
                    if ((rc = fetch_probe_list(ctx, qi, p->nprobe, cs, ch))) return rc;
                    std::vector<float> b(nch);
                    for (uint32_t i = 0; i < nch; ++i) {
                        const float c = std::fmin(std::fmax(cs[i], -1.0f), 1.0f);
                        b[i] = std::cos(std::fmax(std::acos(c) - ctx->h_r_bound[ch[i]], 0.0f));
                    }
                    if (nch)
                        HIP_TRY(ctx, hipMemcpy(W.bnd + static_cast<uint64_t>(qi) * p->nprobe, b.data(), nch * 4,
                                               hipMemcpyHostToDevice));
                    S.host_checks++;
                }
                K.pq_noflag = 1;
                rerun = true;
            }
            if (ctl.pq_overflow) {
                ctx->pq_cap_min = std::max(ctx->pq_cap_min, 2 * ctl.pq_overflow);
                if ((rc = ensure_pq(ctx, nq, K.tcap, ctx->pq_cap_min))) return rc;
                K.pq_cap = ctx->cap_pq;
                rerun = true;
            }
            if (ctl.max_cand > ctx->cap_cand) {
                // the Hamming branch keeps every tie at tau, possibly more than the candidate room
                if ((rc = ensure_cand(ctx, ctl.max_cand + ctl.max_cand / 4 + 64))) return rc;
                K.cand_cap = ctx->cap_cand;
                K.fin_cap = ctx->cap_fin;
                K.key_cap = ctx->cap_key;
                rerun = true;
            }
            if (!rerun) break;
            S.reruns++;
            if ((rc = launch_reset(ctx, nq)) || (rc = launch_pq_scan(ctx, K)) ||
                (rc = launch_pq_finish(ctx, K, d_q, d_slots, d_scores)) || (rc = read_ctl(ctx, &ctl)))
                return rc;
            ctl.nflag_route = 0;  // decided above; nucleus flags are raised only by the route
        }
        if (ctl.pq_overflow || ctl.max_cand > ctx->cap_cand)
            return fail(ctx, MAIVS_ERR_HIP, "per-query candidate buffer still overflows");
        break;
    }
    if (st) {
        HIP_TRY(ctx, hipEventRecord(ctx->ev[6], ctx->stream));
        HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        float ms;
        if (hipEventElapsedTime(&ms, ctx->ev[0], ctx->ev[6]) == hipSuccess) S.ms_total = ms;
        (void)hipGetLastError();
    }
    ctx->last_nq = nq;
    ctx->last_K = K;
    ctx->last_pq = true;
    return 0;
}

}  // namespace

// ================================================================ the fixed scratch array

// The work area of maivs_gpu_search_batch_device_noalloc: every work buffer of a batched call is
// carved from it, so that entry point allocates nothing. Each GPU the library runs on holds its
// own copy at its own address, from the code object's load until the process ends. In host code
// the name is only a stand-in for the symbol: kernels and copies get the per-device address that
// hipGetSymbolAddress returns (kept in ScratchSlot::ptr), never `scratch` itself.
static __device__ __align__(256) uint8_t scratch[MAIVS_GPU_SCRATCH_BYTES];

namespace {

struct ScratchSlot {
    uint8_t* ptr = nullptr;  // this device's copy of `scratch`
    hipError_t lookup = hipSuccess;
    std::mutex run;          // calls on one GPU share the array: they run one at a time
};

// This device's scratch slot; the symbol's address is looked up once per device, with that device
// current (maivs_gpu_create calls this after hipSetDevice).
ScratchSlot* scratch_slot(int device) {
    static std::mutex mu;
    static std::map<int, ScratchSlot*> slots;  // never freed: the array lives as long as the process
    std::lock_guard<std::mutex> lk(mu);
    ScratchSlot*& s = slots[device];
    if (!s) {
        s = new ScratchSlot();
        void* p = nullptr;
        s->lookup = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        s->ptr = s->lookup == hipSuccess ? static_cast<uint8_t*>(p) : nullptr;
        (void)hipGetLastError();
    }
    return s;
}

}  // namespace

// ================================================================ C ABI

extern "C" {

int maivs_gpu_create(int device, maivs_gpu_ctx** out) {
    if (!out) return MAIVS_ERR_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return MAIVS_ERR_HIP;
    auto* ctx = new (std::nothrow) maivs_gpu_ctx();
    if (!ctx) return MAIVS_ERR_OOM;
    ctx->device = device;
    // the main pass launched kernel by kernel (default: two to five launches cost less than one
    // graph replay here), or replayed as one captured HIP graph (MAIVS_GPU_GRAPH=1)
    if (const char* g = std::getenv("MAIVS_GPU_GRAPH")) ctx->use_graph = std::strcmp(g, "1") == 0;
    // the first candidate buffer's room per query (it grows to the exact need on overflow)
    if (const char* c = std::getenv("MAIVS_GPU_CAND_CAP")) ctx->initial_cand_cap = std::max(16, std::atoi(c));
    // the seed stage's own rest scan: unset = by cell sharing, else a fixed count of ranks (0 or 8)
    if (const char* f = std::getenv("MAIVS_GPU_FRONT_REST")) ctx->front_rest_mode = std::max(0, std::atoi(f));
    // the matrix-core scan: unset = by cell sharing, 0 = off, else the least queries of its work items
    if (const char* m = std::getenv("MAIVS_GPU_MMA_MIN")) ctx->mma_min_mode = std::max(0, std::atoi(m));
    // the per-query tree descent by a workgroup per query up to this many queries (else a wave each)
    if (const char* t = std::getenv("MAIVS_GPU_PQ_TREE_BLOCK")) ctx->pq_tree_block_max_q = static_cast<uint32_t>(std::max(0, std::atoi(t)));
    // the per-query scan in rounds of cells (a 1024-thread workgroup per query) up to this many queries
    if (const char* r = std::getenv("MAIVS_GPU_PQ_ROUNDS")) ctx->pq_rounds_max_q = static_cast<uint32_t>(std::max(0, std::atoi(r)));
    // the Hamming rows of indexes with more cells than the route keeps in LDS: by popcounts (0, the
    // default) or on the matrix cores (1); both write the same rows, and both are bound by writing them
    if (const char* hm = std::getenv("MAIVS_GPU_HAM_MMA")) ctx->ham_mma = std::strcmp(hm, "0") != 0;
    // the batched pass by Hamming rows (prep, rows, route + seed) at any cell count
    if (const char* rp = std::getenv("MAIVS_GPU_ROWS")) ctx->rows_pass = std::strcmp(rp, "0") != 0;
    // the per-query path's prep, tree descent and route in one launch up to this many queries
    if (const char* pf = std::getenv("MAIVS_GPU_PQ_FRONT")) ctx->pq_front_max_q = static_cast<uint32_t>(std::max(0, std::atoi(pf)));
    // the per-query path's rerank over workgroups of 8 rows, then the top k, up to this many queries
    if (const char* fs = std::getenv("MAIVS_GPU_PQ_FINISH_SPLIT")) ctx->pq_finish_split_max_q = static_cast<uint32_t>(std::max(0, std::atoi(fs)));
    // the finish with a 1024-thread workgroup per query up to this many queries
    if (const char* fw = std::getenv("MAIVS_GPU_FINISH_WIDE")) ctx->finish_wide_max_q = static_cast<uint32_t>(std::max(0, std::atoi(fw)));
    // the split per-query scan (a workgroup per probed cell, then the bucket queue replayed) up to this many queries
    if (const char* sp = std::getenv("MAIVS_GPU_PQ_SPLIT")) ctx->pq_split_max_q = static_cast<uint32_t>(std::max(0, std::atoi(sp)));
    // the matrix-core scan's items in cell order, a contiguous chunk per XCD: 1 (default) or 0
    if (const char* x = std::getenv("MAIVS_GPU_XCD_ORDER")) ctx->xcd_order = std::strcmp(x, "0") != 0;
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return MAIVS_ERR_HIP;
    }
    for (auto& e : ctx->ev) {
        if (hipEventCreate(&e) != hipSuccess) {
            maivs_gpu_destroy(ctx);
            return MAIVS_ERR_HIP;
        }
    }
    // the control block's host mirror in pinned memory, written by the last kernel of each pass
    void* dev_ctl = nullptr;
    if (hipHostMalloc(reinterpret_cast<void**>(&ctx->h_ctl), sizeof(Ctl), hipHostMallocDefault) != hipSuccess) {
        ctx->h_ctl = nullptr;
        maivs_gpu_destroy(ctx);
        return MAIVS_ERR_OOM;
    }
    if (hipHostGetDevicePointer(&dev_ctl, ctx->h_ctl, 0) != hipSuccess || !dev_ctl) {
        maivs_gpu_destroy(ctx);
        return MAIVS_ERR_HIP;
    }
    std::memset(ctx->h_ctl, 0, sizeof(Ctl));
    ctx->Wk.h_ctl = static_cast<Ctl*>(dev_ctl);
    // the no-allocation entry point's array on this device (device current)
    ctx->scratch = scratch_slot(device);
    *out = ctx;
    return 0;
}

void maivs_gpu_destroy(maivs_gpu_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->gexec) (void)hipGraphExecDestroy(ctx->gexec);
    free_all(ctx->work_allocs);
    free_all(ctx->cand_allocs);
    free_all(ctx->pq_allocs);
    free_all(ctx->split_allocs);
    free_all(ctx->arena_allocs);
    free_all(ctx->store.allocs);
    for (auto& e : ctx->ev)
        if (e) (void)hipEventDestroy(e);
    if (ctx->h_ctl) (void)hipHostFree(ctx->h_ctl);
    if (ctx->h_stage) (void)hipHostFree(ctx->h_stage);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

const char* maivs_gpu_last_error(const maivs_gpu_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int maivs_gpu_upload_arena(maivs_gpu_ctx* ctx, const maivs_arena_desc* a) {
    if (!ctx || !a) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    // this context's row store holds the arena's rows in slot order: they are read there (no H2D),
    // and the description may then leave vecs_f32, sq8_codes, fs_codes and slot_codes out
    const RowStore& R = ctx->store;
    const bool from_store = a->store_token != 0 && a->store_token == R.token && R.n == a->n_slots &&
                            R.dim == a->dim && R.W == a->n_words && (R.flags & MAIVS_STORE_BITS) &&
                            (a->rerank_mode == MAIVS_RERANK_F32 ? (R.flags & MAIVS_STORE_F32) != 0
                                                                : (R.flags & MAIVS_STORE_CODES) != 0);
    const bool fs_arena = a->fs_off && (a->fs_codes || from_store);
    if (!(fs_arena || a->slot_codes || from_store) || !a->mem_off || !a->members || !a->rot_signs || !a->r_bound)
        return fail(ctx, MAIVS_ERR_ARG, "arena is missing its codes (FastScan blocks or per-slot codes), members, "
                                        "rotation or radii");
    if (a->n_cells == 0) return fail(ctx, MAIVS_ERR_ARG, "the arena has no cells");
    if (!supported_nw(a->n_words)) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "n_words %u not in {1,2,4,8,16}", a->n_words);
    // (the Hamming rows address the cell codes with 32-bit byte offsets)
    if (static_cast<uint64_t>(a->n_cells) * a->n_words * 8 >= (1ull << 32))
        return fail(ctx, MAIVS_ERR_UNSUPPORTED, "%u cells of %u-word codes exceed 4 GiB of cell codes", a->n_cells,
                    a->n_words);
    if (a->max_assign > 1 && !a->slot_cells) return fail(ctx, MAIVS_ERR_ARG, "slot_cells missing");
    if (a->max_assign > 1) {
        // homes index per-cell bitsets on the device: every one must name a cell
        const uint64_t nh = static_cast<uint64_t>(a->n_slots) * a->max_assign;
        for (uint64_t i = 0; i < nh; ++i)
            if (a->slot_cells[i] != UINT32_MAX && a->slot_cells[i] >= a->n_cells)
                return fail(ctx, MAIVS_ERR_ARG, "slot_cells names cell %u of %u", a->slot_cells[i], a->n_cells);
    }
    if (!a->cent_sq8 && !a->centroids) return fail(ctx, MAIVS_ERR_ARG, "no centroid store for the rescore");
    if (a->cent_sq8 && (!a->csq_min || !a->csq_step)) return fail(ctx, MAIVS_ERR_ARG, "csq_min/csq_step missing");
    if (a->rerank_mode == MAIVS_RERANK_F32 && !a->vecs_f32 && !from_store) return fail(ctx, MAIVS_ERR_ARG, "f32 rows missing");
    if (a->rerank_mode == MAIVS_RERANK_SQ8 && ((!a->sq8_codes && !from_store) || !a->sq_min || !a->sq_step))
        return fail(ctx, MAIVS_ERR_ARG, "SQ8 rows missing");
    if (a->rerank_mode > MAIVS_RERANK_SQ8) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "rerank mode %u", a->rerank_mode);
    if (a->dim == 0 || a->dim > a->dim_pad || a->dim_pad > 4096 || (a->dim_pad & (a->dim_pad - 1)))
        return fail(ctx, MAIVS_ERR_UNSUPPORTED, "dim %u / dim_pad %u", a->dim, a->dim_pad);
    if (a->n_words * 64 > a->dim_pad) return fail(ctx, MAIVS_ERR_ARG, "n_words exceeds dim_pad");
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    drop_graph(ctx);
    free_all(ctx->work_allocs);
    free_all(ctx->cand_allocs);
    free_all(ctx->pq_allocs);
    free_all(ctx->split_allocs);
    free_all(ctx->arena_allocs);
    ctx->cap_nq = ctx->cap_nprobe = ctx->cap_k = ctx->cap_cand = ctx->cap_seed = ctx->cand_nq = 0;
    ctx->cap_pq_nq = ctx->cap_tcap = ctx->cap_pq = ctx->pq_cap_min = 0;
    ctx->cap_split_e = ctx->cap_split_h = ctx->cap_split_n = 0;
    ctx->d_beams = nullptr;
    ctx->beams_on_device.clear();
    ctx->uploaded = false;
    ctx->last_nq = 0;

    DevArena& A = ctx->A;
    A = DevArena{};
    A.d = a->dim;
    A.P = a->dim_pad;
    A.W = a->n_words;
    A.M = a->n_cells;
    A.N = a->n_slots;
    A.ma = std::max<uint32_t>(a->max_assign, 1);
    A.rerank_mode = a->rerank_mode;
    A.npos = A.W * 16;
    A.maxk = 255 * A.npos;
    A.MW = (A.M + 31) / 32;
    A.Mp = (A.M + 7) & ~7u;
    A.E = a->mem_off[A.M];
    A.fht_scale = 1.0f / std::sqrt(static_cast<float>(A.P));
    A.cf = make_chain(A.d, 4);
    A.cu = make_chain(A.d, 16);
    std::vector<uint32_t> dead;
    uint32_t max_len = 0, n_live = 0;
    for (uint32_t c = 0; c < A.M; ++c) {
        uint32_t len = a->mem_off[c + 1] - a->mem_off[c];
        if (len == 0) dead.push_back(c);
        n_live += len > 0;
        max_len = std::max(max_len, len);
        if (fs_arena && a->fs_off[c + 1] - a->fs_off[c] != (len + 31) / 32)
            return fail(ctx, MAIVS_ERR_ARG, "fs_off does not match the member lists at cell %u", c);
    }
    // members index per-slot arrays on the device (codes, rows, homes, tags)
    for (uint64_t e = 0; e < A.E; ++e)
        if (a->members[e] >= A.N) return fail(ctx, MAIVS_ERR_ARG, "member %llu names slot %u of %u",
                                              static_cast<unsigned long long>(e), a->members[e], A.N);
    A.fs = fs_arena ? 1u : 0u;
    A.n_live = n_live;
    A.n_dead = static_cast<uint32_t>(dead.size());
    A.max_cell_len = max_len;
    // a seed set holds the members of at most SEED_CELLS cells: bound it by the largest ones
    uint32_t seed_cap = 0;
    {
        std::vector<uint32_t> lens(A.M);
        for (uint32_t c = 0; c < A.M; ++c) lens[c] = a->mem_off[c + 1] - a->mem_off[c];
        const uint32_t top = std::min<uint32_t>(kSeedCells, A.M);
        std::partial_sort(lens.begin(), lens.begin() + top, lens.end(), std::greater<uint32_t>());
        uint64_t sum = 0;
        for (uint32_t i = 0; i < top; ++i) sum += lens[i];
        seed_cap = static_cast<uint32_t>(std::min<uint64_t>(std::max<uint64_t>(sum, 1), 1ull << 20));
    }
    if (fs_arena && (seed_cap > 65536 || seed_lds(A, seed_cap) + A.W * 256 > kLdsBudget))
        return fail(ctx, MAIVS_ERR_UNSUPPORTED, "the %u largest cells (%u members) exceed the on-chip seed set", kSeedCells,
                    seed_cap);
    if (prep_lds(A) > kLdsBudget) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "dim_pad %u too large for query prep", A.P);

    std::vector<void*> tmp;  // row-major staging, freed once the chain-major copies exist
    auto stage = [&](auto* src, size_t count, auto** out) -> int {
        int r = dalloc(ctx, tmp, out, count);
        if (r) return r;
        HIP_TRY(ctx, hipMemcpyAsync(*out, src, count * sizeof(**out), hipMemcpyHostToDevice, ctx->stream));
        return 0;
    };
    auto run = [&]() -> int {
        int rc = 0;
        uint8_t* fs = nullptr;
        uint32_t* ddead = nullptr;
        uint32_t *fs_off = nullptr, *codes = nullptr, *members = nullptr, *mem_off = nullptr, *slot_cells = nullptr,
                 *alt = nullptr;
        uint64_t* cent_bits = nullptr;
        float *csq_min = nullptr, *csq_step = nullptr, *r_bound = nullptr, *signs = nullptr, *sq_min = nullptr,
              *sq_step = nullptr;
        uint64_t* scodes = nullptr;
        if (from_store) {
            scodes = R.bits;  // the members' codes are gathered from the store's sign codes
        } else if (fs_arena) {
            const uint64_t nblocks = a->fs_off[A.M];
            if ((rc = stage(a->fs_codes, nblocks * A.W * 256, &fs))) return rc;
            if ((rc = stage(a->fs_off, static_cast<uint64_t>(A.M) + 1, &fs_off))) return rc;
        } else if ((rc = stage(a->slot_codes, static_cast<uint64_t>(A.N) * A.W, &scodes))) {
            return rc;
        }
        if ((rc = dalloc(ctx, ctx->arena_allocs, &codes, A.E * 2 * A.W))) return rc;
        // cos(pi * t / dp) for t = 0 .. dp with the f32 operations of score_to_cos(hamming_score(t))
        // (src/index.rs:1139-1158, src/quantize.rs:206) and this host's libm: the Hamming branch's
        // adaptive-stop threshold, exact on the device
        {
            const uint32_t dp = A.W * 64;
            std::vector<float> hc(dp + 1);
            const float dpf = static_cast<float>(dp);
            for (uint32_t t = 0; t <= dp; ++t) {
                const float sc = dpf - 2.0f * static_cast<float>(t);
                const float hh = (dpf - sc) * 0.5f;
                hc[t] = std::cos(static_cast<float>(M_PI) * hh / dpf);
            }
            float* dhc = nullptr;
            if ((rc = dupload(ctx, hc.data(), hc.size(), &dhc))) return rc;
            HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));  // hc is about to go
            A.ham_cos = dhc;
        }
        if ((rc = dupload(ctx, a->members, A.E, &members))) return rc;
        if ((rc = dupload(ctx, a->mem_off, static_cast<uint64_t>(A.M) + 1, &mem_off))) return rc;
        if ((rc = dalloc(ctx, ctx->arena_allocs, &alt, A.E))) return rc;
        if (A.ma > 1 && (rc = dupload(ctx, a->slot_cells, static_cast<uint64_t>(A.N) * A.ma, &slot_cells))) return rc;
        if (a->cent_bits && (rc = dupload(ctx, a->cent_bits, static_cast<uint64_t>(A.M) * A.W, &cent_bits))) return rc;
        if ((rc = dupload(ctx, a->r_bound, A.M, &r_bound))) return rc;
        if ((rc = dupload(ctx, a->rot_signs, 2ull * A.P, &signs))) return rc;
        if (!dead.empty() && (rc = dupload(ctx, dead.data(), dead.size(), &ddead))) return rc;
        if (fs_arena && !from_store) {
            hipLaunchKernelGGL(fs_to_codes_kernel, dim3(std::max<uint32_t>(A.M, 1)), dim3(256), 0, ctx->stream, fs,
                               fs_off, mem_off, A.M, A.W, codes);
        } else if (A.E) {
            const uint32_t blocks = static_cast<uint32_t>(std::min<uint64_t>((A.E * A.W + 255) / 256, 65535));
            hipLaunchKernelGGL(gather_codes_kernel, dim3(blocks), dim3(256), 0, ctx->stream, scodes, members, A.E, A.W,
                               reinterpret_cast<uint64_t*>(codes));
        }
        if (A.ma == 2)
            hipLaunchKernelGGL(entry_alt_kernel, dim3(std::max<uint32_t>(A.M, 1)), dim3(256), 0, ctx->stream, mem_off,
                               members, slot_cells, A.M, alt);
        uint32_t* etag = nullptr;
        if (a->tags && A.E) {
            uint32_t* tags = nullptr;
            if ((rc = stage(a->tags, A.N, &tags))) return rc;
            if ((rc = dalloc(ctx, ctx->arena_allocs, &etag, A.E))) return rc;
            hipLaunchKernelGGL(entry_tag_kernel, dim3(static_cast<uint32_t>(std::min<uint64_t>((A.E + 255) / 256, 65535))),
                               dim3(256), 0, ctx->stream, members, tags, A.E, etag);
        }
        A.entry_tag = etag;
        // the centroid tree of the per-query path's routing
        if ((rc = upload_tree(ctx, ctx->arena_allocs, a->tree, A.W, A.M, &ctx->tree, &ctx->tree_level_n))) return rc;
        ctx->tree_beam_frac = a->tree ? a->tree->beam_frac : 0.5f;
        ctx->tree_min_beam = a->tree ? a->tree->min_beam : 32u;
        HIP_TRY(ctx, hipGetLastError());
        // chain-major copies of the rows the 8-lane dots read
        // dev: the rows already in HBM (the row store), else src is staged
        auto chain_f32 = [&](const float* src, uint64_t rows, const float** out, const float* dev = nullptr) -> int {
            float *raw = const_cast<float*>(dev), *cm = nullptr;
            int r;
            if (!raw && (r = stage(src, rows * A.d, &raw))) return r;
            if ((r = dalloc(ctx, ctx->arena_allocs, &cm, rows * A.cf.stride))) return r;
            hipLaunchKernelGGL(to_chain_kernel<float>, dim3(static_cast<uint32_t>(std::min<uint64_t>(rows, 65535))),
                               dim3(256), 0, ctx->stream, raw, rows, A.d, A.cf, cm);
            *out = cm;
            return 0;
        };
        auto chain_u8 = [&](const uint8_t* src, uint64_t rows, const uint8_t** out, const uint8_t* dev = nullptr) -> int {
            uint8_t *raw = const_cast<uint8_t*>(dev), *cm = nullptr;
            int r;
            if (!raw && (r = stage(src, rows * A.d, &raw))) return r;
            if ((r = dalloc(ctx, ctx->arena_allocs, &cm, rows * A.cu.stride))) return r;
            hipLaunchKernelGGL(to_chain_kernel<uint8_t>, dim3(static_cast<uint32_t>(std::min<uint64_t>(rows, 65535))),
                               dim3(256), 0, ctx->stream, raw, rows, A.d, A.cu, cm);
            *out = cm;
            return 0;
        };
        if (a->cent_sq8) {
            if ((rc = chain_u8(a->cent_sq8, A.M, &A.cent_sq8))) return rc;
            if ((rc = dupload(ctx, a->csq_min, A.d, &csq_min))) return rc;
            if ((rc = dupload(ctx, a->csq_step, A.d, &csq_step))) return rc;
        } else {
            if ((rc = chain_f32(a->centroids, A.M, &A.cents))) return rc;
        }
        if (A.rerank_mode == MAIVS_RERANK_F32) {
            if ((rc = chain_f32(a->vecs_f32, A.N, &A.vecs, from_store ? R.f32 : nullptr))) return rc;
        } else {
            if ((rc = chain_u8(a->sq8_codes, A.N, &A.sq8, from_store ? reinterpret_cast<const uint8_t*>(R.codes) : nullptr)))
                return rc;
            if ((rc = dupload(ctx, a->sq_min, A.d, &sq_min))) return rc;
            if ((rc = dupload(ctx, a->sq_step, A.d, &sq_step))) return rc;
        }
        HIP_TRY(ctx, hipGetLastError());
        HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        A.codes = codes;
        A.members = members;
        A.entry_alt = alt;
        A.mem_off = mem_off;
        A.slot_cells = slot_cells;
        A.cent_bits = cent_bits;
        A.csq_min = csq_min;
        A.csq_step = csq_step;
        A.r_bound = r_bound;
        A.rot_signs = signs;
        A.sq_min = sq_min;
        A.sq_step = sq_step;
        A.dead = ddead;
        return 0;
    };
    int rc = run();
    (void)hipStreamSynchronize(ctx->stream);
    free_all(tmp);
    if (rc) {
        free_all(ctx->arena_allocs);
        return rc;
    }
    ctx->h_r_bound.assign(a->r_bound, a->r_bound + A.M);
    // LDS plan: the route's shortlist sort size is per call (12 bytes per entry: key + weight)
    // (the fused front kernel also holds one query's prep region beside the route's)
    const size_t route_fixed = route_lds(A, 0, 0) + (fused_front(A) ? prep1_lds(A) : 0);
    size_t room = kLdsBudget - 8192 > route_fixed ? (kLdsBudget - 8192 - route_fixed) / 12 : 0;
    if (room < 1024) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "routing tables do not fit in LDS");
    uint32_t sc = 1024;
    while (static_cast<size_t>(sc) * 2 <= room && sc < 16384) sc <<= 1;
    ctx->max_sort_cap_route = sc;
    ctx->seed_cap = seed_cap;
    ctx->lds_prep = prep_lds(A);
    ctx->lds_seed = seed_lds(A, seed_cap);
    ctx->lds_finish = finish_lds(A);
    // every kernel's dynamic-LDS limit only grows (another context's smaller arena must not lower
    // the limit this one's launches rely on), and a failure is an error
    auto raise = [&](const void* fn, size_t lds) { return raise_lds_limit(ctx, fn, lds); };
    if ((rc = raise(reinterpret_cast<const void*>(finish_kernel<kFinishThreads>), ctx->lds_finish)) ||
        (rc = raise(reinterpret_cast<const void*>(finish_kernel<kFinishWideThreads>), ctx->lds_finish)))
        return rc;
    DISPATCH_EPL(A.P / 64, rc = raise(reinterpret_cast<const void*>(prep_kernel<EPL>), ctx->lds_prep));
    if (rc) return rc;
    DISPATCH_NW(A.W, {
        const size_t rs = std::max(route_lds(A, sc, sc), ctx->lds_seed);
        if ((rc = raise(reinterpret_cast<const void*>(route_kernel<NW>), route_lds(A, sc, sc))) ||
            (rc = raise(reinterpret_cast<const void*>(seed_kernel<NW>), ctx->lds_seed)) ||
            (rc = raise(reinterpret_cast<const void*>(route_seed_kernel<NW, false>), rs)) ||
            (rc = raise(reinterpret_cast<const void*>(route_seed_kernel<NW, true>), rs)) ||
            (rc = raise(reinterpret_cast<const void*>(front_kernel<NW>),
                        std::max(route_lds(A, sc, sc) + prep1_lds(A), ctx->lds_seed))))
            return rc;
    });
    ctx->uploaded = true;
    return 0;
}

int maivs_gpu_search_batch_device(maivs_gpu_ctx* ctx, const float* d_q, uint32_t nq, const maivs_search_params* p,
                                  uint32_t* d_slots, float* d_scores, maivs_gpu_stats* st) {
    if (!ctx || !p || (nq && (!d_q || !d_slots || !d_scores))) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    return run_search(ctx, d_q, nq, p, d_slots, d_scores, st);
}

int maivs_gpu_search_batch_device_noalloc(maivs_gpu_ctx* ctx, const float* d_q, uint32_t nq,
                                          const maivs_search_params* p, uint32_t* d_slots, float* d_scores,
                                          maivs_gpu_stats* st) {
    if (!ctx || !p || (nq && (!d_q || !d_slots || !d_scores))) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (!ctx->uploaded) return fail(ctx, MAIVS_ERR_NOT_UPLOADED, "no arena uploaded");
    if (p->k == 0) return fail(ctx, MAIVS_ERR_ARG, "k must be > 0");
    ScratchSlot* slot = static_cast<ScratchSlot*>(ctx->scratch);
    if (!slot || !slot->ptr)
        return fail(ctx, MAIVS_ERR_HIP, "the scratch array of device %d is unavailable: hipGetSymbolAddress: %s",
                    ctx->device, hipGetErrorString(slot ? slot->lookup : hipErrorInvalidValue));
    if (st) *st = maivs_gpu_stats{};
    if (nq == 0) return 0;
    const DevArena& A = ctx->A;
    const uint32_t nprobe = std::max<uint32_t>(p->nprobe, 1), k = std::max<uint32_t>(p->k, 1);
    const size_t bytes = MAIVS_GPU_SCRATCH_BYTES;
    const uint32_t cand_cap = std::max<uint32_t>(ctx->initial_cand_cap, 64);
    // routing through the centroid tree also needs the descent's leaf lists and beams
    KParams Kr = make_params(ctx, 1, p);
    int rc = route_setup(ctx, p, true, Kr, nullptr);
    if (rc) return rc;
    const uint32_t tcap = Kr.tree_list ? Kr.tcap : 0u;
    // A chunk of n queries: its work buffers (and the tree's), then its candidate buffers at the
    // room the context starts with (an overflow re-carves them within the array).
    auto carve_front = [&](uint32_t n, Carver& c, Work& w, uint32_t** beams) {
        carve_work(A, n, nprobe, k, ctx->seed_cap, bucket_cap_for(A, n, nprobe), false, c, w);
        if (tcap) {
            c.take(&w.tlist, static_cast<uint64_t>(n) * tcap);
            c.take(&w.tcount, n);
            c.take(beams, kPqMaxLevels);
        }
    };
    auto need = [&](uint32_t n, size_t* cand_off) {
        Work tmp{};
        Carver c{nullptr};
        uint32_t* b = nullptr;
        carve_front(n, c, tmp, &b);
        if (cand_off) *cand_off = c.used;
        carve_cand(n, ctx->seed_cap, cand_cap, c, tmp);
        return c.used;
    };
    // Queries are independent, so a batch larger than the array holds runs as equal chunks of the
    // largest size that fits, with results identical to one pass.
    uint32_t chunk = nq;
    if (need(chunk, nullptr) > bytes) {
        uint32_t lo = 0, hi = nq;  // need(lo) fits (lo = 0 meaning none), need(hi) does not
        while (hi - lo > 1) {
            const uint32_t mid = lo + (hi - lo) / 2;
            (need(mid, nullptr) <= bytes ? lo : hi) = mid;
        }
        if (lo == 0)
            return fail(ctx, MAIVS_ERR_UNSUPPORTED,
                        "one query at nprobe %u needs %zu bytes of work buffers, more than the %zu-byte scratch "
                        "(use maivs_gpu_search_batch_device)",
                        nprobe, need(1, nullptr), bytes);
        const uint32_t parts = (nq + lo - 1) / lo;
        chunk = (nq + parts - 1) / parts;
    }

    // one call at a time on this GPU's array; the call returns only after its kernels are done
    std::lock_guard<std::mutex> run(slot->run);
    // the context's own buffers and their state are set aside and restored afterwards
    const Work own = ctx->Wk;
    const uint32_t s_nq = ctx->cap_nq, s_np = ctx->cap_nprobe, s_k = ctx->cap_k, s_cand = ctx->cap_cand,
                   s_seed = ctx->cap_seed, s_fin = ctx->cap_fin, s_key = ctx->cap_key, s_b = ctx->cap_bucket,
                   s_cnq = ctx->cand_nq;
    const bool s_clean = ctx->counters_clean;
    uint32_t* const s_beams = ctx->d_beams;
    const std::vector<uint32_t> s_beams_dev = ctx->beams_on_device;
    for (uint32_t q0 = 0; q0 < nq && rc == 0; q0 += chunk) {
        const uint32_t n = std::min(chunk, nq - q0);
        const uint32_t bcap = bucket_cap_for(A, n, nprobe);
        size_t cand_off = 0;
        need(n, &cand_off);
        Work W = own;  // keeps the pinned control-block mirror and the per-query path's fields
        Carver cw{slot->ptr};
        uint32_t* beams = nullptr;
        carve_front(n, cw, W, &beams);
        if (tcap) {
            ctx->d_beams = beams;  // the array's beams: unknown contents, copied by the pass
            ctx->beams_on_device.clear();
        }
        Carver cc{slot->ptr};
        cc.used = cand_off;
        carve_cand(n, ctx->seed_cap, cand_cap, cc, W);
        ctx->Wk = W;
        ctx->cap_nq = n;
        ctx->cap_nprobe = nprobe;
        ctx->cap_k = k;
        ctx->cap_seed = ctx->seed_cap;
        ctx->cap_bucket = bcap;
        ctx->cap_cand = cand_cap;
        ctx->cand_nq = n;
        cand_caps(ctx->cap_seed, cand_cap, &ctx->cap_fin, &ctx->cap_key);
        ctx->counters_clean = false;  // the array holds the last call's contents: clear the counters first
        const Scratch sc{slot->ptr, bytes, cand_off};
        maivs_gpu_stats part{};
        rc = run_search(ctx, d_q + static_cast<uint64_t>(q0) * A.d, n, p, d_slots + static_cast<uint64_t>(q0) * p->k,
                        d_scores + static_cast<uint64_t>(q0) * p->k, st ? &part : nullptr, &sc);
        if (st && rc == 0) {
            st->ms_total += part.ms_total;
            st->ms_prep += part.ms_prep;
            st->ms_route += part.ms_route;
            st->ms_seed += part.ms_seed;
            st->ms_invert += part.ms_invert;
            st->ms_scan += part.ms_scan;
            st->ms_select += part.ms_select;
            st->ms_rerank += part.ms_rerank;
            st->host_checks += part.host_checks;
            st->host_fixes += part.host_fixes;
            st->reruns += part.reruns;
        }
    }
    const hipError_t sync = hipStreamSynchronize(ctx->stream);
    ctx->Wk = own;
    ctx->d_beams = s_beams;
    ctx->beams_on_device = s_beams_dev;
    ctx->cap_nq = s_nq;
    ctx->cap_nprobe = s_np;
    ctx->cap_k = s_k;
    ctx->cap_cand = s_cand;
    ctx->cap_seed = s_seed;
    ctx->cap_fin = s_fin;
    ctx->cap_key = s_key;
    ctx->cap_bucket = s_b;
    ctx->cand_nq = s_cnq;
    ctx->counters_clean = s_clean;
    ctx->last_nq = 0;  // the stage read-backs read the context's own buffers, which this call left alone
    if (rc) return rc;
    if (sync != hipSuccess) return fail(ctx, MAIVS_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(sync));
    return 0;
}

// The host-buffer entry points' copies: the queries through the context's pinned staging buffer to
// the device, `run` on them, and the slots and scores back through the same buffer (a pinned copy
// runs at the link's rate; a pageable one goes through the runtime's own staging in pieces).
extern "C++" template <class Run>
static int staged_search(maivs_gpu_ctx* ctx, const float* q, uint32_t nq, uint32_t k, uint32_t* out_slots,
                         float* out_scores, Run run) {
    const size_t qb = static_cast<size_t>(nq) * ctx->A.d * 4, ob = static_cast<size_t>(nq) * k * 4;
    const size_t need = std::max(qb, 2 * ob);
    if (need > ctx->h_stage_bytes) {
        // (no copy of an earlier call may still read the old buffer)
        if (ctx->h_stage) HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->h_stage) HIP_TRY(ctx, hipHostFree(ctx->h_stage));
        ctx->h_stage = nullptr;
        ctx->h_stage_bytes = 0;
        if (hipHostMalloc(&ctx->h_stage, need, hipHostMallocDefault) != hipSuccess) {
            ctx->h_stage = nullptr;
            return fail(ctx, MAIVS_ERR_OOM, "pinned staging of %zu bytes", need);
        }
        ctx->h_stage_bytes = need;
    }
    uint8_t* h = static_cast<uint8_t*>(ctx->h_stage);
    std::memcpy(h, q, qb);
    HIP_TRY(ctx, hipMemcpyAsync(ctx->Wk.q, h, qb, hipMemcpyHostToDevice, ctx->stream));
    int rc = run();
    if (rc) {
        (void)hipStreamSynchronize(ctx->stream);  // the queries' copy out of the buffer is done
        return rc;
    }
    // (the queries' copy has finished before the kernels that read them, so the buffer is free)
    HIP_TRY(ctx, hipMemcpyAsync(h, ctx->Wk.out_slots, ob, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(h + ob, ctx->Wk.out_scores, ob, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    std::memcpy(out_slots, h, ob);
    std::memcpy(out_scores, h + ob, ob);
    return 0;
}

int maivs_gpu_search_batch(maivs_gpu_ctx* ctx, const float* q, uint32_t nq, const maivs_search_params* p,
                           uint32_t* out_slots, float* out_scores, maivs_gpu_stats* st) {
    if (!ctx || !p || (nq && (!q || !out_slots || !out_scores))) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (!ctx->uploaded) return fail(ctx, MAIVS_ERR_NOT_UPLOADED, "no arena uploaded");
    if (nq == 0) return 0;
    int rc = ensure_all(ctx, nq, p->nprobe, p->k);
    if (rc) return rc;
    return staged_search(ctx, q, nq, p->k, out_slots, out_scores, [&] {
        return run_search(ctx, ctx->Wk.q, nq, p, ctx->Wk.out_slots, ctx->Wk.out_scores, st);
    });
}

int maivs_gpu_search_queries_device(maivs_gpu_ctx* ctx, const float* d_q, uint32_t nq, const maivs_search_params* p,
                                    uint32_t* d_slots, float* d_scores, maivs_gpu_stats* st) {
    if (!ctx || !p || (nq && (!d_q || !d_slots || !d_scores))) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    return run_search_pq(ctx, d_q, nq, p, d_slots, d_scores, st);
}

int maivs_gpu_search_queries(maivs_gpu_ctx* ctx, const float* q, uint32_t nq, const maivs_search_params* p,
                             uint32_t* out_slots, float* out_scores, maivs_gpu_stats* st) {
    if (!ctx || !p || (nq && (!q || !out_slots || !out_scores))) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (!ctx->uploaded) return fail(ctx, MAIVS_ERR_NOT_UPLOADED, "no arena uploaded");
    if (nq == 0) return 0;
    int rc = ensure_all(ctx, nq, p->nprobe, p->k);
    if (rc) return rc;
    return staged_search(ctx, q, nq, p->k, out_slots, out_scores, [&] {
        return run_search_pq(ctx, ctx->Wk.q, nq, p, ctx->Wk.out_slots, ctx->Wk.out_scores, st);
    });
}

int maivs_gpu_query_prep(maivs_gpu_ctx* ctx, const float* q, uint32_t nq, uint64_t* out_bits, uint8_t* out_lut,
                         float* out_delta, float* out_bias) {
    if (!ctx || (nq && (!q || !out_bits || !out_lut || !out_delta || !out_bias))) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (!ctx->uploaded) return fail(ctx, MAIVS_ERR_NOT_UPLOADED, "no arena uploaded");
    if (nq == 0) return 0;
    int rc = ensure_all(ctx, nq, ctx->cap_nprobe, ctx->cap_k);
    if (rc) return rc;
    const DevArena& A = ctx->A;
    maivs_search_params p{};
    p.k = 1;
    p.nprobe = 1;
    p.target_confidence = 1.0f;
    KParams K = make_params(ctx, nq, &p);
    HIP_TRY(ctx, hipMemcpyAsync(ctx->Wk.q, q, static_cast<size_t>(nq) * A.d * 4, hipMemcpyHostToDevice, ctx->stream));
    if ((rc = launch_prep(ctx, K, ctx->Wk.q, 0))) return rc;
    HIP_TRY(ctx, hipMemcpyAsync(out_bits, ctx->Wk.qbits, static_cast<size_t>(nq) * A.W * 8, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(out_lut, ctx->Wk.lut, static_cast<size_t>(nq) * A.npos * 16, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(out_delta, ctx->Wk.delta, nq * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(out_bias, ctx->Wk.bias, nq * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

int maivs_gpu_block_sums(maivs_gpu_ctx* ctx, uint32_t n_words, const uint8_t* blocks, const uint8_t* luts, uint32_t nb,
                         uint16_t* out) {
    if (!ctx || (nb && (!blocks || !luts || !out))) return MAIVS_ERR_ARG;
    if (!supported_nw(n_words)) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "n_words %u", n_words);
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (nb == 0) return 0;
    const uint64_t bb = n_words * 256ull, ne = 32ull * nb;
    std::vector<void*> tmp;
    uint8_t *dblk = nullptr, *dlut = nullptr;
    uint32_t *doff = nullptr, *dmem = nullptr, *dcodes = nullptr;
    uint16_t* dout = nullptr;
    std::vector<uint32_t> off(nb + 1), moff(nb + 1);
    for (uint32_t i = 0; i <= nb; ++i) {
        off[i] = i;
        moff[i] = 32 * i;
    }
    int rc = 0;
    rc |= dalloc(ctx, tmp, &dblk, nb * bb);
    rc |= dalloc(ctx, tmp, &dlut, nb * bb);
    rc |= dalloc(ctx, tmp, &doff, nb + 1ull);
    rc |= dalloc(ctx, tmp, &dmem, nb + 1ull);
    rc |= dalloc(ctx, tmp, &dcodes, ne * 2 * n_words);
    rc |= dalloc(ctx, tmp, &dout, ne);
    if (rc) {
        free_all(tmp);
        return rc;
    }
    auto run = [&]() -> int {
        HIP_TRY(ctx, hipMemcpyAsync(dblk, blocks, nb * bb, hipMemcpyHostToDevice, ctx->stream));
        HIP_TRY(ctx, hipMemcpyAsync(dlut, luts, nb * bb, hipMemcpyHostToDevice, ctx->stream));
        HIP_TRY(ctx, hipMemcpyAsync(doff, off.data(), (nb + 1) * 4, hipMemcpyHostToDevice, ctx->stream));
        HIP_TRY(ctx, hipMemcpyAsync(dmem, moff.data(), (nb + 1) * 4, hipMemcpyHostToDevice, ctx->stream));
        hipLaunchKernelGGL(fs_to_codes_kernel, dim3(nb), dim3(64), 0, ctx->stream, dblk, doff, dmem, nb, n_words, dcodes);
        DISPATCH_NW(n_words, hipLaunchKernelGGL(entry_sums_kernel<NW>, dim3(nb), dim3(64), NW * 256, ctx->stream,
                                                dcodes, dlut, static_cast<uint32_t>(ne), dout));
        HIP_TRY(ctx, hipGetLastError());
        HIP_TRY(ctx, hipMemcpyAsync(out, dout, ne * 2, hipMemcpyDeviceToHost, ctx->stream));
        HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        return 0;
    };
    rc = run();
    free_all(tmp);
    return rc;
}

int maivs_gpu_route(maivs_gpu_ctx* ctx, const float* q, uint32_t nq, const maivs_search_params* p, uint32_t* out_chosen,
                    float* out_cscore, uint32_t* out_nchosen) {
    if (!ctx || !p || (nq && (!q || !out_chosen || !out_cscore || !out_nchosen))) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (!ctx->uploaded) return fail(ctx, MAIVS_ERR_NOT_UPLOADED, "no arena uploaded");
    if (nq == 0 || p->nprobe == 0) return 0;
    int rc = ensure_all(ctx, nq, p->nprobe, p->k);
    if (rc) return rc;
    KParams K = make_params(ctx, nq, p);
    std::vector<uint32_t> beams;
    if ((rc = route_setup(ctx, p, true, K, &beams))) return rc;
    uint32_t tree_cap = 1;
    for (uint32_t b : beams) tree_cap = std::max(tree_cap, b);
    if (K.tree_list && ((rc = ensure_pq(ctx, nq, K.tcap, 0)) || (rc = upload_beams(ctx, beams)))) return rc;
    Work& W = ctx->Wk;
    if (K.want_c == 0) {
        std::fill(out_chosen, out_chosen + static_cast<size_t>(nq) * p->nprobe, kNone);
        std::fill(out_cscore, out_cscore + static_cast<size_t>(nq) * p->nprobe, NAN);
        std::fill(out_nchosen, out_nchosen + nq, 0u);
        return 0;
    }
    HIP_TRY(ctx, hipMemcpyAsync(W.q, q, static_cast<size_t>(nq) * ctx->A.d * 4, hipMemcpyHostToDevice, ctx->stream));
    ctx->counters_clean = false;  // the route sets control counters that no epilogue clears
    if ((rc = launch_prep(ctx, K, W.q, kPrepReset))) return rc;
    if (K.tree_list && (rc = launch_pq_tree(ctx, K, tree_cap))) return rc;
    if ((rc = launch_route(ctx, K))) return rc;
    Ctl ctl{};
    HIP_TRY(ctx, hipMemcpyAsync(&ctl, W.ctl, sizeof(Ctl), hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(out_chosen, W.chosen, static_cast<size_t>(nq) * p->nprobe * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(out_cscore, W.cscore, static_cast<size_t>(nq) * p->nprobe * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(out_nchosen, W.nchosen, nq * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    if (ctl.err_shortlist)
        return fail(ctx, MAIVS_ERR_UNSUPPORTED, "a routing shortlist of %u cells exceeds the on-chip sort capacity %u",
                    ctl.max_shortlist, K.sort_cap);
    if (ctl.nflag_route) {
        std::vector<uint32_t> fl(ctl.nflag_route);
        HIP_TRY(ctx, hipMemcpy(fl.data(), W.flag_route, fl.size() * 4, hipMemcpyDeviceToHost));
        for (uint32_t qi : fl) {
            const float* cs = out_cscore + static_cast<size_t>(qi) * p->nprobe;
            const uint32_t* ch = out_chosen + static_cast<size_t>(qi) * p->nprobe;
            uint32_t cap = 0;
            while (cap < p->nprobe && ch[cap] != kNone) ++cap;
            out_nchosen[qi] = host_nucleus(cs, cap, p->target_confidence, p->beta);
        }
    }
    return 0;
}

int maivs_gpu_last_counters(maivs_gpu_ctx* ctx, maivs_gpu_stats* stats) {
    if (!ctx || !stats) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    stats->seed_blocks = stats->scan_blocks = stats->scan_pairs = stats->survivors = stats->rerank_rows = 0;
    if (ctx->last_nq == 0) return 0;
    if (ctx->last_pq)
        return fail(ctx, MAIVS_ERR_UNSUPPORTED, "the last search ran the per-query path, which keeps no work counters");
    hipLaunchKernelGGL(counters_kernel, dim3(1), dim3(1024), 0, ctx->stream, ctx->A, ctx->Wk, ctx->last_K);
    HIP_TRY(ctx, hipGetLastError());
    Ctl ctl{};
    int rc = read_ctl_live(ctx, &ctl);
    if (rc) return rc;
    stats->seed_blocks = ctl.seed_blocks;
    stats->scan_blocks = ctl.scan_blocks;
    stats->scan_pairs = ctl.scan_pairs;
    stats->survivors = ctl.survivors;
    stats->rerank_rows = ctl.rerank_rows;
    return 0;
}

int maivs_gpu_last_candidates(maivs_gpu_ctx* ctx, uint32_t* tau, uint32_t* rest_end, uint32_t* cut, uint32_t* ncand,
                              uint32_t* cand_slots, uint32_t* cand_d, uint64_t cap) {
    if (!ctx) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    const uint32_t nq = ctx->last_nq;
    if (nq == 0) return 0;
    if (ctx->last_pq)
        return fail(ctx, MAIVS_ERR_UNSUPPORTED, "the last search ran the per-query path, which keeps no seed cut-offs");
    Work& W = ctx->Wk;
    std::vector<uint32_t> n(nq);
    HIP_TRY(ctx, hipMemcpy(n.data(), W.ncand, nq * 4, hipMemcpyDeviceToHost));
    if (tau) HIP_TRY(ctx, hipMemcpy(tau, W.tau, nq * 4, hipMemcpyDeviceToHost));
    if (rest_end) HIP_TRY(ctx, hipMemcpy(rest_end, W.rest_end, nq * 4, hipMemcpyDeviceToHost));
    if (cut) HIP_TRY(ctx, hipMemcpy(cut, W.cut, nq * 4, hipMemcpyDeviceToHost));
    if (ncand) std::memcpy(ncand, n.data(), nq * 4);
    if (!cand_slots && !cand_d) return 0;
    uint64_t total = 0;
    for (uint32_t x : n) total += x;
    if (total > cap) return fail(ctx, MAIVS_ERR_ARG, "candidate arrays hold %llu, need %llu",
                                 static_cast<unsigned long long>(cap), static_cast<unsigned long long>(total));
    std::vector<uint2> buf;
    uint64_t pos = 0;
    for (uint32_t qi = 0; qi < nq; ++qi) {
        buf.resize(n[qi]);
        if (n[qi])
            HIP_TRY(ctx, hipMemcpy(buf.data(), W.fin + static_cast<uint64_t>(qi) * ctx->cap_fin, n[qi] * sizeof(uint2),
                                   hipMemcpyDeviceToHost));
        std::sort(buf.begin(), buf.end(), [](const uint2& a, const uint2& b) { return a.x != b.x ? a.x < b.x : a.y < b.y; });
        for (auto& e : buf) {
            if (cand_slots) cand_slots[pos] = e.y;
            if (cand_d) cand_d[pos] = e.x;
            ++pos;
        }
    }
    return 0;
}

}  // extern "C"
