/*
 * maivs_gpu.h - C ABI of libmaivs_gpu.so, the MI355X (gfx950) batched cell-major search.
 *
 * This is the surface a Rust `build.rs` + `extern "C"` block binds, and what the C++
 * `FlatCellIndex` host mirror calls. Plain pointers and sizes only; no C++ types cross it
 * and no exceptions escape it. Every function returns 0 on success or a negative
 * maivs_status; the message of the last failure on a context is kept per context.
 *
 * Reference interfaces replaced (file:line in V47VANSH/MAIVS):
 *   maivs_gpu_search_batch   FlatCellIndex::search_batch_cellmajor, src/index.rs:1999-2311
 *                            (route_batch :1873-1980, rerank_exact :1309-1378), reached from
 *                            the pyo3 FlatCellIndex.search_batch, src/index.rs:3316-3362
 *   maivs_gpu_upload_arena   the compacted arena fields read by that path, src/index.rs:431-566
 *                            in the state compact_arena (:929-1112) leaves
 *   maivs_gpu_query_prep     rotate + pack_signs_trunc + FsQuery::new, src/quantize.rs:57-313
 *   maivs_gpu_block_sums     FsQuery::block_sums, src/quantize.rs:323-386
 *   maivs_gpu_route          route_batch, src/index.rs:1873-1980
 *   maivs_gpu_search_queries FlatCellIndex::search_one + route_query, src/index.rs:1168-1305,
 *                            1381-1864, reached from search (:3283-3305) and the per-query
 *                            branch of search_batch (:3363-3391)
 *   maivs_gpu_kmeans         kmeans_spherical, src/tree.rs:179-248, as run by train_centroids'
 *                            two-level k-means (src/tree.rs:257-348, src/index.rs:2762-2804) and
 *                            by the centroid tree build (src/tree.rs:354-460)
 *   maivs_gpu_place          add_batch's per-vector work, src/index.rs:2442-2610: rotation and
 *                            sign code, the centroid-tree descent (src/tree.rs:120-159, 559-628),
 *                            exact centroid scores and the home choice (assign_cells,
 *                            pick_orthogonal, :2480-2560), the i8 / SQ8 copy (:3083-3123),
 *                            and the primary cell sums (:2643-2667, 3186-3196)
 *   maivs_gpu_store_radii    recompute_radii, src/index.rs:817-861 (the dots and order statistics)
 *   maivs_gpu_store_compact  compact_arena's row moves and FastScan packing, src/index.rs:929-1112
 *   maivs_gpu_store_reset / _info: the row store those two read (no counterpart: see below)
 */
#ifndef MAIVS_GPU_H
#define MAIVS_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum maivs_status {
    MAIVS_OK = 0,
    MAIVS_ERR_ARG = -1,          /* bad argument (null pointer, size mismatch, k == 0 ...) */
    MAIVS_ERR_NOT_UPLOADED = -2, /* search before maivs_gpu_upload_arena */
    MAIVS_ERR_HIP = -3,          /* a HIP runtime call failed */
    MAIVS_ERR_OOM = -4,          /* device allocation failed */
    MAIVS_ERR_UNSUPPORTED = -5,  /* configuration this library does not run */
} maivs_status;

/* Rerank stores (src/index.rs:1309-1378). */
enum {
    MAIVS_RERANK_F32 = 0,   /* `quality`: f32 rows, dot_f32 */
    MAIVS_RERANK_SQ8 = 1,   /* `memory`: per-dimension SQ8 rows, base + dot_f32_u8 */
};

/*
 * The index, as host pointers (compacted with FastScan blocks, or else with per-slot codes). Caller-owned; maivs_gpu_upload_arena copies every
 * array to HBM and keeps nothing of the caller's. Shapes use d = dim, P = dim_pad,
 * W = n_words, M = n_cells, N = n_slots, E = mem_off[M], B = fs_off[M].
 */
typedef struct maivs_arena_desc {
    uint32_t dim;          /* d, a multiple of 8 is not required */
    uint32_t dim_pad;      /* P = next power of two >= d, >= 64 (src/quantize.rs:38-40) */
    uint32_t n_words;      /* W = 64-bit words per sign code (8 at d = 384) */
    uint32_t n_cells;      /* M */
    uint32_t n_slots;      /* N, length of the per-slot arrays */
    uint32_t max_assign;   /* homes per slot (2 with orthogonal polysemy) */
    uint32_t rerank_mode;  /* MAIVS_RERANK_* */
    uint32_t reserved0;
    /* FastScan blocks: 32 vectors x W*64 bytes each, cell-major in member order */
    const uint8_t* fs_codes;    /* B * W * 256 bytes */
    const uint32_t* fs_off;     /* M + 1, in blocks */
    /* member lists: cell c owns members[mem_off[c] .. mem_off[c+1]), primaries then replicas */
    const uint32_t* mem_off;    /* M + 1 */
    const uint32_t* members;    /* E slots */
    const uint32_t* slot_cells; /* N * max_assign, UINT32_MAX = unused */
    /* routing */
    const uint64_t* cent_bits;  /* M * W, or NULL when two-stage routing is off (route_mode 1 only) */
    const uint8_t* cent_sq8;    /* M * d, or NULL to score the f32 centroids */
    const float* centroids;     /* M * d (used when cent_sq8 is NULL) */
    const float* csq_min;       /* d */
    const float* csq_step;      /* d */
    const float* r_bound;       /* M, p99 member angle per cell */
    const float* rot_signs;     /* 2 * P, the +-1 rotation signs */
    /* rerank */
    const float* vecs_f32;      /* N * d (MAIVS_RERANK_F32) */
    const uint8_t* sq8_codes;   /* N * d (MAIVS_RERANK_SQ8) */
    const float* sq_min;        /* d (MAIVS_RERANK_SQ8) */
    const float* sq_step;       /* d (MAIVS_RERANK_SQ8) */
    /* filtering: one u32 attribute per slot (src/index.rs:551-555), or NULL when unused */
    const uint32_t* tags;       /* N */
    /* the centroid tree the per-query path routes with (n_levels 0: none); defined below */
    const struct maivs_tree_desc* tree;
    /* Per-slot sign codes, N * W. An index that is not compacted, or has no FastScan blocks, is
     * uploaded with fs_codes and fs_off NULL and these instead: its cells' members are then in any
     * order, and only the per-query path runs, scanning them with Hamming distances (search_one's
     * Hamming branch, src/index.rs:1694-1760). Ignored when fs_codes is given. */
    const uint64_t* slot_codes;
    /* Nonzero: the token maivs_gpu_store_info gave for this context's row store, which holds this
     * arena's N rows in slot order. The f32 rows, the SQ8 rows and the sign codes are then read from
     * that store in HBM instead of from vecs_f32, sq8_codes and fs_codes / slot_codes (which may
     * still be given and are ignored). A token of another store, or of an older state of this one,
     * is ignored and the host arrays are used. */
    uint64_t store_token;
} maivs_arena_desc;

/* Query-time settings of search_batch (src/index.rs:3316-3326 and the index setters). */
typedef struct maivs_search_params {
    uint32_t k;
    uint32_t nprobe;
    float target_confidence;  /* >= 1 probes all nprobe; < 1 nucleus over exp(beta*(s-max)) */
    float beta;
    uint32_t rerank_factor;   /* survivors reranked = k * rerank_factor */
    uint32_t shortlist_mult;  /* two-stage shortlist = nprobe * max(mult, 2) */
    uint32_t adaptive;        /* adaptive probe cut (set_adaptive) */
    float at_margin;          /* its margin */
    /* Inclusive tag range [tag_lo, tag_hi] (set_filter, src/index.rs:3553-3558). With filter != 0
     * and uploaded tags, a member counts only when its slot's tag is in range: the reference's
     * keep! predicate (:1428-1439), applied in the seed and cell-major scans beside the canonical
     * test, before tau and the cut-offs. (The reference runs filtered searches per query,
     * :3343-3348; this is the same predicate on the batched path.) */
    uint32_t filter;
    uint32_t tag_lo;
    uint32_t tag_hi;
    /* Routing (src/index.rs:1168-1305, 1873-1877). 0: two-stage routing is on (set_two_stage with
     * centroid codes): the batched path routes with route_batch's Hamming shortlist and exact
     * rescore; the per-query path with the tree when the arena has one, else route_query's
     * two-stage shortlist. 1: two-stage routing is off: both paths route as route_query does, with
     * the tree when the arena has one, else over every live cell scored exactly. */
    uint32_t route_mode;
} maivs_search_params;

/* Per-call measurements. maivs_gpu_search_batch* fills the times and host_* / reruns fields
 * (HIP events on the context's stream, recorded only when a stats struct is passed; no extra
 * device work). The main pass is launched stage by stage and each stage is timed; a context
 * created with the environment variable MAIVS_GPU_GRAPH=1 replays it as one captured HIP graph
 * instead, timed as a whole (ms_total; the stage fields stay 0). The work counters (the *_blocks,
 * scan_pairs, survivors, rerank_rows fields) are filled on demand by maivs_gpu_last_counters. */
typedef struct maivs_gpu_stats {
    float ms_total;       /* device time of the whole pipeline (hipEvents) */
    float ms_prep;        /* per-call counter reset; with the query prep (rotation, sign codes,
                             FastScan tables) when that runs as its own kernel */
    float ms_route;       /* Hamming shortlist + SQ8 rescore + probe-list sort and the seed scan,
                             cut-off and adaptive cut; with the query prep when the codes cover the
                             whole padded dimension (one fused kernel) */
    float ms_seed;        /* the seed stage when it runs as its own kernel (0: fused with the route) */
    float ms_invert;      /* query -> cell inversion */
    float ms_scan;        /* the cell-major scan kernel */
    float ms_select;      /* tie-inclusive cut at k * rerank_factor */
    float ms_rerank;      /* exact rerank + top-k */
    uint64_t scan_pairs;      /* (query, cell) pairs in the rest scan */
    uint64_t scan_blocks;     /* sum over those pairs of the cell's 32-vector blocks */
    uint64_t seed_blocks;     /* same for the seed scan */
    uint64_t survivors;       /* candidates the rest scan emitted */
    uint64_t rerank_rows;     /* rows the rerank read */
    uint32_t host_checks;     /* queries whose libm-sensitive decision the host re-evaluated */
    uint32_t host_fixes;      /* of those, how many changed the device's decision */
    uint32_t reruns;          /* pipeline re-runs (buffer growth or host fixes) */
    uint32_t reserved;
} maivs_gpu_stats;

typedef struct maivs_gpu_ctx maivs_gpu_ctx;

/* One context per (device, arena). Creates a HIP stream on `device`. */
int maivs_gpu_create(int device, maivs_gpu_ctx** out);
void maivs_gpu_destroy(maivs_gpu_ctx* ctx);
const char* maivs_gpu_last_error(const maivs_gpu_ctx* ctx);

/* Copy the compacted arena to HBM (replaces any previous one). An arena without cells is refused
 * (MAIVS_ERR_ARG), and so is one whose cell codes exceed 4 GiB (MAIVS_ERR_UNSUPPORTED). */
int maivs_gpu_upload_arena(maivs_gpu_ctx* ctx, const maivs_arena_desc* arena);

/*
 * Batched cell-major search. Host buffers: queries nq x dim (f32, row-major), outputs nq x k.
 * out_slots[q*k + i] is the arena slot of the i-th best result of query q, best first, ties by
 * ascending slot; rows with fewer than k results are padded with UINT32_MAX / -inf. The copies
 * go through a pinned staging buffer the context allocates on first use and keeps (grown to the
 * largest call).
 */
int maivs_gpu_search_batch(maivs_gpu_ctx* ctx, const float* queries, uint32_t nq,
                           const maivs_search_params* params, uint32_t* out_slots,
                           float* out_scores, maivs_gpu_stats* stats);

/* Same, with queries and outputs already in device memory (HBM-resident inputs). */
int maivs_gpu_search_batch_device(maivs_gpu_ctx* ctx, const float* d_queries, uint32_t nq,
                                  const maivs_search_params* params, uint32_t* d_out_slots,
                                  float* d_out_scores, maivs_gpu_stats* stats);

/* Bytes of the fixed device array maivs_gpu_search_batch_device_noalloc works in (one per GPU). */
#define MAIVS_GPU_SCRATCH_BYTES ((size_t)128 << 20)

/*
 * No counterpart in the reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the same search as
 * maivs_gpu_search_batch_device, with identical results, that allocates nothing. Every work buffer
 * is carved from a fixed array of MAIVS_GPU_SCRATCH_BYTES that the library holds on each GPU it
 * runs on until the process ends; queries and outputs stay the caller's. A batch whose buffers do
 * not fit runs as equal chunks of the largest size that does (queries are independent, so results
 * do not change); MAIVS_ERR_UNSUPPORTED when even one query does not fit (very long probe lists or
 * indexes of more than 8,192 cells, whose Hamming rows live in global memory). Calls on one GPU
 * share its array and keep the last call's contents: the library runs them one at a time within a
 * process, and each call clears what must start at zero. The call runs its stages without a HIP
 * graph and leaves the context's own buffers, and what maivs_gpu_last_candidates /
 * maivs_gpu_last_counters read, untouched (they report nothing after it).
 */
int maivs_gpu_search_batch_device_noalloc(maivs_gpu_ctx* ctx, const float* d_queries, uint32_t nq,
                                          const maivs_search_params* params, uint32_t* d_out_slots,
                                          float* d_out_scores, maivs_gpu_stats* stats);

/*
 * The per-query path: the reference's search_one (src/index.rs:1381-1864) for every query on its
 * own, as its search() and its search_batch for small batches, filtered searches and
 * cell_major=False run it (:3283-3392). Each query is routed by route_query (:1168-1305: the
 * centroid tree when the arena has one, else the two-stage Hamming shortlist of nprobe *
 * shortlist_mult cells), then its probed cells are scanned in probe order with the FastScan
 * bucket queue on d >> 6, the rule that a multi-home vector counts at its first-ranked probed home,
 * the tag filter and the adaptive stop; the k * rerank_factor smallest d (ties by ascending slot)
 * are reranked exactly. Same buffers and results layout as maivs_gpu_search_batch.
 */
int maivs_gpu_search_queries(maivs_gpu_ctx* ctx, const float* queries, uint32_t nq,
                             const maivs_search_params* params, uint32_t* out_slots,
                             float* out_scores, maivs_gpu_stats* stats);
int maivs_gpu_search_queries_device(maivs_gpu_ctx* ctx, const float* d_queries, uint32_t nq,
                                    const maivs_search_params* params, uint32_t* d_out_slots,
                                    float* d_out_scores, maivs_gpu_stats* stats);

/* ---- stage entry points for parity tests (host buffers) ---- */

/* Rotation, sign code and FastScan table of nq queries: bits nq x W, lut nq x (W*256),
 * delta nq, bias nq. Needs an uploaded arena (for the rotation signs). */
int maivs_gpu_query_prep(maivs_gpu_ctx* ctx, const float* queries, uint32_t nq,
                         uint64_t* out_bits, uint8_t* out_lut, float* out_delta,
                         float* out_bias);

/* FastScan sums of nb blocks against one table each: blocks nb x (W*256) bytes, luts
 * nb x (W*256) bytes, out nb x 32 u16. Needs a context (arena not required); n_words = W. */
int maivs_gpu_block_sums(maivs_gpu_ctx* ctx, uint32_t n_words, const uint8_t* blocks,
                         const uint8_t* luts, uint32_t nb, uint16_t* out);

/* Routing of nq queries: chosen nq x nprobe cell ids (best first), cscore nq x nprobe,
 * nchosen nq. Unused tail entries are UINT32_MAX / NaN. */
int maivs_gpu_route(maivs_gpu_ctx* ctx, const float* queries, uint32_t nq,
                    const maivs_search_params* params, uint32_t* out_chosen,
                    float* out_cscore, uint32_t* out_nchosen);

/* Work counters of the last maivs_gpu_search_batch* call into `stats` (other fields untouched):
 * seed_blocks / scan_blocks = 32-vector FastScan blocks scored by the seed and cell-major scans
 * (one per (query, block) pair), scan_pairs = (query, cell) pairs of the cell-major scan,
 * survivors = candidates it emitted, rerank_rows = rows the rerank read. */
int maivs_gpu_last_counters(maivs_gpu_ctx* ctx, maivs_gpu_stats* stats);

/*
 * Intermediates of the last maivs_gpu_search_batch* call (host buffers, NULL to skip):
 * tau nq (seed cut-off), rest_end nq (probe-list index where the scan stopped),
 * cut nq (final tie-inclusive cut-off G), ncand nq (candidates reranked),
 * cand_slots / cand_d: for each query its candidates, sorted by (d, slot), packed
 * back to back in query order; cap = capacity of those two arrays (entries).
 */
int maivs_gpu_last_candidates(maivs_gpu_ctx* ctx, uint32_t* tau, uint32_t* rest_end,
                              uint32_t* cut, uint32_t* ncand, uint32_t* cand_slots,
                              uint32_t* cand_d, uint64_t cap);

/* ---- index build ---- */

/* One spherical k-means problem of a batch. Its points are rows[first .. first + n) of the
 * batch's row list; jobs tile the row list in order (first = sum of the earlier jobs' n). */
typedef struct maivs_kmeans_job {
    uint32_t first;
    uint32_t n;       /* points, >= 1 */
    uint32_t k;       /* clusters, 1 <= k <= n */
    uint32_t iters;   /* Lloyd iterations (0 leaves the initial centroids and assignment 0) */
    uint64_t seed;    /* the empty-cluster reseeding state starts at seed | 1 */
} maivs_kmeans_job;

/*
 * Batched spherical Lloyd k-means over rows of one host matrix x (n_rows x dim f32, row-major),
 * bit-identical to the reference's CPU k-means: initial centroid c = point min(c*stride, n-1)
 * with stride = max(n/k, 1); each iteration assigns every point to the first best centroid by
 * the 8-lane FMA dot, sums each cluster's points in point order, normalises the sums, and
 * reseeds empty clusters with xorshift64 picks. rows: the batch's row ids (NULL = 0, 1, 2, ...);
 * dim <= 2048. Outputs (host): assign[sum n] = cluster within the job at the last iteration,
 * cents[sum k x dim], the jobs' centroids back to back.
 */
int maivs_gpu_kmeans(maivs_gpu_ctx* ctx, const float* x, uint64_t n_rows, uint32_t dim,
                     const uint32_t* rows, const maivs_kmeans_job* jobs, uint32_t n_jobs,
                     uint32_t* assign, float* cents);

/* The centroid tree (src/tree.rs) in its compacted layout: every node's children are contiguous
 * in the next level (or the leaves), child_start / child_len give the range. A descent that
 * wants `want` leaves keeps, per level from the finest up, clamp(ceil(need * beam_frac),
 * min_beam, level size) nodes, need starting at want (src/tree.rs:559-570). */
typedef struct maivs_tree_desc {
    uint32_t n_levels;            /* 0 = no tree */
    uint32_t n_leaf;
    float beam_frac;              /* set_tree_route's beam_frac (0.5 by default) */
    uint32_t min_beam;            /* MIN_BEAM, 32 */
    const uint32_t* level_n;      /* n_levels: nodes per level, coarsest first */
    const uint64_t* level_codes;  /* sum(level_n) x n_words, level by level */
    const uint32_t* child_start;  /* sum(level_n) */
    const uint32_t* child_len;    /* sum(level_n) */
    const uint64_t* leaf_codes;   /* n_leaf x n_words */
    const uint32_t* leaf_cells;   /* n_leaf: the cell of each leaf */
} maivs_tree_desc;

/* What placing a vector reads from the index (host pointers). */
typedef struct maivs_place_desc {
    uint32_t dim, dim_pad, n_words, n_cells;
    uint32_t max_assign;          /* homes per vector, 1..64 */
    float spill_lambda;           /* > 0: orthogonal polysemy strength */
    float spill_margin;           /* else: homes within this score of the best */
    uint32_t code_mode;           /* 0: none, 1: per-dimension SQ8, 2: global int8 (quant_scale) */
    float quant_scale;
    uint32_t tree_want;           /* leaves the descent keeps, max(64, 8 * max_assign) (src/index.rs:2452) */
    const float* rot_signs;       /* 2 x dim_pad */
    const float* centroids;       /* n_cells x dim (f32) */
    const float* sq_min;          /* dim (code_mode 1) */
    const float* sq_step;         /* dim (code_mode 1) */
    maivs_tree_desc tree;         /* n_levels 0: every cell is a candidate */
    /* Optional, n entries: vector i's rows (the f32 row, the sign code and the i8 / SQ8 copy, as
     * the context's row store keeps them) are also written to the store at slot store_slots[i],
     * the slot add_batch gives it (src/index.rs:3077-3199, 2566-2667). */
    const uint32_t* store_slots;
    /* Optional, n_cells x dim, in and out: vector i's f32 row is added to the sum of its primary
     * home (homes[i * max_assign]), the vectors of a cell in input order (add_batch's primary
     * sums, src/index.rs:2643-2667, 3186-3196). */
    float* sums;
} maivs_place_desc;

/*
 * Place n vectors (host, n x dim f32), bit-identical to the reference's CPU placement: homes
 * n x max_assign (cell ids, primary first, UINT32_MAX padded), bits n x n_words (the 1-bit
 * code), codes n x dim (the i8 / SQ8 copy; may be NULL when code_mode is 0).
 */
int maivs_gpu_place(maivs_gpu_ctx* ctx, const maivs_place_desc* desc, const float* x, uint32_t n,
                    uint32_t* homes, uint64_t* bits, int8_t* codes);

/*
 * The row store: the index's per-slot rows kept in HBM through the build. No counterpart in the
 * reference, whose rows live in host memory only. Placement writes each vector's rows once
 * (maivs_place_desc.store_slots); the cell radii, the compaction and the arena upload then read
 * them where they are, so the build moves each row over PCIe once instead of at every step.
 * One store per context; its layout is fixed by maivs_gpu_store_reset.
 */
enum {
    MAIVS_STORE_F32 = 1,    /* f32 rows, dim floats per slot (keep_f32) */
    MAIVS_STORE_CODES = 2,  /* i8 / SQ8 rows, dim bytes per slot (scan_i8) */
    MAIVS_STORE_BITS = 4,   /* sign codes, n_words u64 per slot (bits) */
};

/* Empties the store and sets its layout (flags: MAIVS_STORE_*). */
int maivs_gpu_store_reset(maivs_gpu_ctx* ctx, uint32_t dim, uint32_t n_words, uint32_t flags);

/* The store's token (nonzero after a reset, new after every write) and its slot count. */
int maivs_gpu_store_info(maivs_gpu_ctx* ctx, uint64_t* token, uint32_t* n_slots);

/* What recompute_radii reads (src/index.rs:817-861), besides the store's rows. */
typedef struct maivs_radii_desc {
    uint32_t n_cells, dim;
    uint32_t mode;            /* 0: f32 rows, 1: per-dimension SQ8 rows, 2: global int8 rows */
    float inv_scale;          /* mode 2: 1 / quant_scale */
    const uint32_t* mem_off;  /* n_cells + 1 */
    const uint32_t* members;  /* mem_off[n_cells] slots of the store, any order within a cell */
    const float* centroids;   /* n_cells x dim */
    const float* sq_min;      /* dim (mode 1) */
    const float* sq_step;     /* dim (mode 1) */
} maivs_radii_desc;

/*
 * recompute_radii's order statistics (src/index.rs:817-861): for every cell with members, the
 * member dots with its centroid clamped to [-1, 1] (the reference's arithmetic for each mode),
 * and of those p99_dot = the (p99 + 1)-th largest, p99 = min(ceil(len * 0.99) - 1, len - 1) in
 * f32, and min_dot = the smallest. acos is non-increasing on [-1, 1] (checked for every f32 input
 * of the host's libm by the tests), so r_bound = acos(p99_dot) and r_max = acos(min_dot) are the
 * reference's select_nth_unstable and max over the angles. Cells without members get 0.
 */
int maivs_gpu_store_radii(maivs_gpu_ctx* ctx, const maivs_radii_desc* desc, float* p99_dot, float* min_dot);

/*
 * compact_arena's row moves and FastScan packing (src/index.rs:929-1112) in the store: slot s of
 * the compacted store is old slot old_of_new[s]; then, when fs_codes is given, every cell's members
 * (mem_off / members, in compacted slots and final member order) are packed into FastScan blocks
 * from the store's sign codes (fs_pack_block, src/quantize.rs:238-265), cell c's blocks at
 * fs_off[c]. The compacted rows are also copied to rows_out / codes_out / bits_out where given.
 */
int maivs_gpu_store_compact(maivs_gpu_ctx* ctx, const uint32_t* old_of_new, uint32_t n_new, uint32_t n_cells,
                            const uint32_t* mem_off, const uint32_t* members, const uint32_t* fs_off,
                            uint8_t* fs_codes, float* rows_out, int8_t* codes_out, uint64_t* bits_out);

#ifdef __cplusplus
}
#endif
#endif /* MAIVS_GPU_H */
