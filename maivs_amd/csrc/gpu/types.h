// Constants and plain structs shared by the search kernels and the host side of the library
// (the arena in HBM, the per-call work buffers, the control block and the launch parameters).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../../include/maivs_gpu.h"

namespace maivs_dev {

constexpr uint32_t kSeedCells = 8;       // SEED_CELLS, src/index.rs:2018
constexpr uint32_t kFrontRestMax = 8;    // rest cells the seed stage may scan itself (<= kSeedCells)
constexpr double kFrontRestShare = 8.0;  // ... when the batch's rest probes per live cell are fewer
constexpr uint32_t kPrepWaves = 4;       // queries per prep workgroup, one wave each
constexpr uint32_t kPrepReset = 1;
constexpr uint32_t kHdLdsCells = 8192;  // the route keeps its Hamming row in LDS up to this many cells
constexpr uint32_t kHamQ = 16, kHamC = 256;  // hamming_kernel's tile: queries x cells
constexpr uint32_t kRouteThreads = 256;
constexpr uint32_t kSeedThreads = 256;
constexpr uint32_t kScanThreads = 256;
constexpr uint32_t kFinishThreads = 256;
constexpr uint32_t kFinishWideThreads = 1024;  // the finish of small batches
constexpr uint32_t kG = 4;               // queries interleaved per cell_scan table pass
constexpr uint32_t kItemQ = 2 * kG;      // queries per scan work item (two interleaved tables)
constexpr uint32_t kBucketQ = 32;       // bucket entries per scan work item (one matrix-core query tile)
constexpr uint32_t kItemGroups = 1024;   // work items per cell in a scan work item id (bucket_cap <= 4096)
constexpr uint32_t kHistBins = 256;
constexpr uint32_t kFinishLdsCap = 2048; // final candidates kept and sorted in LDS up to this many
constexpr uint32_t kNoAlt = 0xFFFFFFFEu; // entry_alt: the slot has no other home
constexpr uint32_t kNoD = 0xFFFFu;        // seed score buffer: member not scored here (d <= 255 * 256 < kNoD)
constexpr uint32_t kThrBins = 256;       // a query's running-cut histogram: bins of d >> 8 (d < 65536)
constexpr uint32_t kThrEvery = 512;      // its cut is recomputed each time this many more candidates are appended

// Chain-major row layout for the 8-lane FMA dots: element 8t + l (t < T) of a row is stored at
// l*Tp + t, the d - 8T tail elements at 8*Tp + i. Lane l of a group of 8 then reads its whole
// accumulation chain with wide loads, in the reference's order.
struct Chain {
    uint32_t T, Tp, tail, stride;
};

struct DevArena {
    uint32_t d, P, W, M, N, ma, rerank_mode, npos, maxk, n_live, n_dead, max_cell_len, MW, Mp;
    uint64_t E;
    float fht_scale;
    Chain cf, cu;               // f32 and u8 chain layouts
    const uint32_t* codes;      // E x 2W dwords, entry-major 1-bit codes in member order
    const uint32_t* members;    // E slots
    const uint32_t* entry_alt;  // E: the entry's other home (max_assign == 2), kNoAlt if none
    const uint32_t* mem_off;    // M + 1
    const uint32_t* slot_cells; // N x ma
    const uint64_t* cent_bits;  // M x W (null: the arena routes by the tree or every live cell only)
    const uint8_t* cent_sq8;    // M x cu.stride (chain-major) or null
    const float* cents;         // M x cf.stride (chain-major f32 centroids, when cent_sq8 is null)
    const float* csq_min;
    const float* csq_step;
    const float* r_bound;       // M
    const float* rot_signs;     // 2P
    const float* vecs;          // N x cf.stride (chain-major f32 rows)
    const uint8_t* sq8;         // N x cu.stride (chain-major SQ8 rows)
    const float* sq_min;
    const float* sq_step;
    const uint32_t* dead;       // n_dead: the cells with no members, ascending
    const uint32_t* entry_tag;  // E: the tag of the entry's slot (null without tags)
    uint32_t fs;                // 1: codes came from FastScan blocks (compacted); 0: from per-slot codes
    const float* ham_cos;       // W*64 + 1: cos(pi * t / dp) in f32 by the host's libm (Hamming branch)
};

struct Ctl {
    uint32_t nflag_route;
    uint32_t nflag_prune;
    uint32_t max_cand;        // largest candidate count past the buffer capacity (0 = none)
    uint32_t err_shortlist;   // a shortlist exceeded the sort capacity
    uint32_t max_shortlist;
    uint32_t err_seed;        // a seed set exceeded its on-chip capacity
    uint32_t bucket_overflow; // a cell's query bucket was full (the pass falls back to the counting sort)
    uint32_t n_active;        // scan work items: (cell, block of kBucketQ bucket entries) (bucket mode)
    uint32_t n_active8;       // the same by groups of kItemQ bucket entries (the lookup scan's items)
    uint32_t pq_overflow;     // per-query path: largest candidate count past its buffer (0 = none)
    unsigned long long seed_blocks, scan_blocks, scan_pairs, survivors, rerank_rows;
};

// Bytes of the route's LDS layout: cqs[d4] | ex[np4] | keys[sort_cap] u64 | hist[nbins4] |
// scratch[16] | hd[Mp] u16 (hd only up to kHdLdsCells cells). A multiple of 16.
__host__ __device__ inline size_t route_lds_bytes(uint32_t d, uint32_t W, uint32_t Mp, uint32_t sort_cap,
                                                  uint32_t nprobe) {
    const size_t d4 = (d + 3) & ~3u;
    const size_t np4 = ((nprobe + 3) & ~3u) < sort_cap ? ((nprobe + 3) & ~3u) : sort_cap;
    const size_t nbins4 = ((W * 64 + 1) + 3) & ~3u;
    return d4 * 4 + np4 * 4 + static_cast<size_t>(sort_cap) * 8 + nbins4 * 4 + 16 * 4 +
           (Mp <= kHdLdsCells ? static_cast<size_t>(Mp) * 2 : 0);
}

struct Work {
    float* q;              // nq x d (host-input calls)
    uint64_t* qbits;       // nq x W
    uint16_t* hs;          // nq x Mp Hamming rows, only when Mp > kHdLdsCells (else in LDS)
    uint8_t* lut;          // nq x npos*16
    float* delta;          // nq
    float* bias;           // nq
    float* cqs;            // nq x d: rescore operand q * csq_step (q itself for f32 centroids)
    float* cqbase;         // nq: sum(q * csq_min), sequential
    float* rbase;          // nq: SQ8 rerank base sum(q * sq_min), sequential (MAIVS_RERANK_SQ8)
    float* bnd;            // nq x nprobe: adaptive-cut bounds of the probe list (i >= SEED_CELLS)
    uint32_t* chosen;      // nq x nprobe
    float* cscore;         // nq x nprobe
    uint32_t* nchosen;     // nq
    uint32_t* probed;      // nq x MW
    uint2* seed;           // nq x seed_cap (d, slot): seed members with d <= tau
    uint32_t* seed_cnt;    // nq
    uint32_t* tau;         // nq
    uint32_t* rest_end;    // nq
    uint2* cand;           // nq x cand_cap
    uint32_t* cand_cnt;    // nq
    uint32_t* cand_n;      // nq: each query's candidate count as the finish read it (kept after the clear)
    uint32_t* done;        // 1: finished workgroups of the pass's last kernel (pass_epilogue)
    uint2* fin;            // nq x fin_cap (d, slot) final candidates
    uint64_t* keys;        // nq x key_cap (global sort when a final list is large)
    uint32_t* cut;         // nq
    uint32_t* ncand;       // nq
    uint32_t* out_slots;   // nq x k (host-output calls)
    float* out_scores;     // nq x k
    uint32_t* cell_cnt;    // M + 1
    uint32_t* cell_off;    // M + 1
    uint32_t* cell_cur;    // M
    uint32_t* qof;         // nq x nprobe
    uint32_t* qbuck;       // M x bucket_cap: the queries probing each cell (bucket mode)
    uint32_t* active;      // scan work items, cell * kItemGroups + group of kBucketQ, in arrival order (bucket mode)
    uint32_t* active8;     // the same by groups of kItemQ (cell * kItemGroups + group)
    uint32_t* active_cs;   // the kBucketQ items again, in cell order (order_items_kernel)
    uint32_t* flag_route;  // nq
    uint32_t* flag_prune;  // nq
    // per-query path
    uint32_t* tlist;       // nq x tcap: the centroid tree's leaf cells for each query
    uint32_t* tcount;      // nq
    uint64_t* pqc;         // nq x pq_cap: scanned candidates (d << 32 | slot)
    // the split per-query scan (small batches): each probed cell's admitted entries (nq x nprobe x
    // pq_room, d << 32 | slot), their bucket-queue histogram (nq x nprobe x bins4) and count (nq x nprobe)
    uint64_t* pqe;
    uint32_t* pqh;
    uint32_t* pqn;
    // The cell-major scans' running cut of each query: starts at tau, and drops to the upper edge of
    // the d >> 8 bin holding the target-th smallest d among the entries counted so far in dhist
    // (the seed's scored members, then every appended candidate). Those are entries of the query's
    // scanned cells, so the cut never falls below the final cut G and the candidate set at G is
    // unchanged; it only stops the scans appending entries G would drop.
    uint32_t* thr;         // nq
    uint32_t* dhist;       // nq x kThrBins
    uint32_t* thr_at;      // nq: the query's candidate count when its running cut was last lowered
    Ctl* ctl;
    Ctl* h_ctl;            // pinned host mirror of ctl, written by pass_epilogue (device address)
};

struct KParams {
    uint32_t nq, k, nprobe, want_c, target, adaptive, sort_cap, use_nucleus;
    uint32_t seed_cap, cand_cap, fin_cap, key_cap, bucket_cap;
    uint32_t filter, tag_lo, tag_hi;  // keep!: tag in [tag_lo, tag_hi] (filter != 0 only with tags)
    // per-query path: routing from the tree's list, bounds from this probe rank on, buffer sizes
    uint32_t tree_list, bnd_from, tcap, pq_cap, pq_room, pq_noflag;
    // per-query scan: look up byte pairs of positions in a 256-entry table per pair (small batches)
    uint32_t pq_pair;
    // batched path: rest cells (probe ranks SEED_CELLS on) the seed stage scans itself, query-major
    uint32_t front_rest;
    // bucket work items with at least this many queries go to the matrix-core scan (0: none)
    uint32_t mma_min;
    // per-query path: the Hamming branch (no FastScan blocks)
    uint32_t pq_ham;
    // per-query scan: probed cells in rounds scanned together (small batches)
    uint32_t pq_rounds;
    // per-query scan: every probed cell scored by its own workgroup, then the bucket queue replayed
    uint32_t pq_split;
    // matrix-core scan: items in cell order, a contiguous chunk per XCD (else arrival order)
    uint32_t xcd_order;
    // routing: every live cell is rescored (no tree, no two-stage shortlist)
    uint32_t flat_route;
    // the scans' cut: 0 tau; 1 the running cut Wk.thr, counted and lowered as candidates are
    // appended (the seed stage starts it); 2 the running cut as it stands, not updated (a re-run
    // over the same cells, whose entries were counted already)
    uint32_t run_thr;
    float tc, beta, at_margin, norm, prune_band, nucleus_band;
};

}  // namespace maivs_dev
