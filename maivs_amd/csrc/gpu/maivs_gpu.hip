// libmaivs_gpu.so: MI355X (gfx950) batched cell-major search behind the C ABI of
// include/maivs_gpu.h. Restates MAIVS's FlatCellIndex::search_batch_cellmajor
// (src/index.rs:1999-2311) with route_batch (:1873-1980) and rerank_exact (:1309-1378).
//
// Pipeline of one batch (one HIP stream, no host round trip until the end):
//   prep_route   one workgroup per query: rotation (2 x sign flip + FWHT), 1-bit code,
//                FastScan table, Hamming against every centroid code, tie-inclusive
//                shortlist, exact SQ8 rescore, probe list sorted (score desc, cell asc)
//   seed         one workgroup per query: scan of the first 8 probed cells, seed cut-off
//                tau, adaptive probe cut
//   invert       count / scan / fill: cell -> probing queries
//   cell_scan    one workgroup per probed cell: each lane holds one member's code in
//                registers; groups of 4 probing queries' tables are interleaved in LDS so one
//                ds_read_b32 looks up a nibble for 4 queries; survivors d <= tau appended
//   finish       one workgroup per query: exact tie-inclusive cut at k*rerank_factor, exact
//                f32 / SQ8 rerank, top-k (score desc, slot asc)
// The host reads a small control block at the end; rare events (candidate buffer overflow,
// libm-sensitive decisions near their threshold) re-run the affected stages.
//
// Compiled with -ffp-contract=off: every FMA below is an explicit __builtin_fmaf standing
// for one of the reference's _mm256_fmadd_ps.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../../include/maivs_gpu.h"
#include "device_common.h"

using namespace maivs_dev;

namespace {

constexpr uint32_t kSeedCells = 8;       // SEED_CELLS, src/index.rs:2018
constexpr uint32_t kRouteThreads = 256;
constexpr uint32_t kScanThreads = 256;
constexpr uint32_t kG = 4;               // queries interleaved per cell_scan table pass
constexpr uint32_t kHistBins = 256;
constexpr uint32_t kFinishSortCap = 2048;  // final candidates sorted in LDS up to this many
constexpr size_t kLdsBudget = 160 * 1024;
// Host re-evaluation bands around libm-sensitive thresholds (see host_check_* below).
constexpr float kPruneBand = 4e-6f;
constexpr float kNucleusBand = 2e-3f;

// ---------------------------------------------------------------- arena / params on device

struct DevArena {
    uint32_t d, P, W, M, N, ma, rerank_mode, npos, maxk, n_live, max_cell_len, MW;
    uint64_t E;
    float fht_scale;
    const uint32_t* codes;      // E x (2W) dwords, entry-major 1-bit codes
    const uint32_t* members;    // E
    const uint32_t* mem_off;    // M + 1
    const uint32_t* slot_cells; // N x ma
    const uint64_t* cent_bits;  // M x W
    const uint8_t* cent_sq8;    // M x d or null
    const float* centroids;     // M x d (used when cent_sq8 is null)
    const float* csq_min;
    const float* csq_step;
    const float* r_bound;       // M
    const float* rot_signs;     // 2P
    const float* vecs;          // N x d (f32 rerank)
    const uint8_t* sq8;         // N x d (SQ8 rerank)
    const float* sq_min;
    const float* sq_step;
    const uint8_t* live;        // M
};

struct Ctl {
    uint32_t nflag_route;
    uint32_t nflag_prune;
    uint32_t max_cand;
    uint32_t err_shortlist;   // a shortlist exceeded the sort capacity
    uint32_t max_shortlist;
    uint32_t pad[3];
    unsigned long long seed_blocks;  // 32-vector blocks the seed scan read (work counter)
    unsigned long long scan_blocks;  // 32-vector blocks the cell-major scan scored, per query
    unsigned long long scan_pairs;   // (query, cell) pairs of the cell-major scan
    unsigned long long survivors;    // candidates the cell-major scan emitted
    unsigned long long rerank_rows;  // rows the rerank read
};

struct Work {
    // per query
    float* q;              // nq x d (host-input calls)
    uint64_t* qbits;       // nq x W
    uint8_t* lut;          // nq x npos*16
    float* delta;          // nq
    float* bias;           // nq
    uint32_t* chosen;      // nq x nprobe
    float* cscore;         // nq x nprobe
    uint32_t* nchosen;     // nq
    uint32_t* probed;      // nq x MW
    uint2* seed;           // nq x seed_cap (d, slot)
    uint32_t* seed_cnt;    // nq
    uint32_t* tau;         // nq
    uint32_t* rest_end;    // nq
    uint2* cand;           // nq x cand_cap
    uint32_t* cand_cnt;    // nq
    uint2* fin;            // nq x fin_cap (d, slot) final candidates
    uint64_t* keys;        // nq x key_cap (global sort fallback)
    uint32_t* cut;         // nq
    uint32_t* ncand;       // nq
    uint32_t* out_slots;   // nq x k (host-output calls)
    float* out_scores;     // nq x k
    // per cell
    uint32_t* cell_cnt;    // M + 1
    uint32_t* cell_off;    // M + 1
    uint32_t* cell_cur;    // M
    uint32_t* qof;         // nq x nprobe
    uint32_t* flag_route;  // nq
    uint32_t* flag_prune;  // nq
    Ctl* ctl;
};

struct KParams {
    uint32_t nq, k, nprobe, want_c, target, adaptive, sort_cap, use_nucleus;
    uint32_t seed_cap, cand_cap, fin_cap, key_cap, fin_sort_cap;
    float tc, beta, at_margin, norm, prune_band, nucleus_band;
};

// ---------------------------------------------------------------- small device pieces

// One member's nibble sums against a FastScan table of G interleaved queries in LDS.
// `code` = the member's entry-major code (2*NW dwords; nibble j at dword j/8, bits 4*(j%8)),
// streamed 16 bytes (32 positions) at a time with the next chunk prefetched. Table byte
// [(j*16 + e)*G + g] = query g's entry e of position j.
template <int G>
__device__ __forceinline__ void lut_chunk(uint32_t dw0, uint32_t dw1, uint32_t dw2, uint32_t dw3, int npos,
                                          const uint8_t* tk, uint32_t& S, uint32_t& T) {
#pragma unroll
    for (int t = 0; t < 32; ++t) {
        if (t < npos) {
            const uint32_t dw = t < 8 ? dw0 : t < 16 ? dw1 : t < 24 ? dw2 : dw3;
            const uint32_t nib = (dw >> (4 * (t & 7))) & 0xFu;
            if constexpr (G == 1) {
                S += tk[t * 16 + nib];
            } else {
                const uint32_t v = reinterpret_cast<const uint32_t*>(tk)[t * 16 + nib];
                S += v;
                T += __builtin_amdgcn_perm(0u, v, 0x0c030c01u);  // bytes 1,3 -> u16 lanes
            }
        }
    }
}

template <int NW, int G>
__device__ __forceinline__ void lut_sums(const uint32_t* __restrict__ code, const uint8_t* table, uint32_t (&sum)[G]) {
    static_assert(G == 1 || G == 4, "G is 1 or 4");
    // S accumulates table words; for G = 4 it is b0 + 256 b1 + 65536 b2 + 2^24 b3 (mod 2^32) and T
    // the odd bytes as u16 lanes (b1 + 65536 b3). Every per-query sum is at most 255 * 16 * NW
    // < 65536, so both un-mix exactly at the end.
    uint32_t S = 0, T = 0;
    if constexpr (NW == 1) {
        uint2 v = *reinterpret_cast<const uint2*>(code);
        lut_chunk<G>(v.x, v.y, 0u, 0u, 16, table, S, T);
    } else {
        constexpr int NCH = NW / 2;  // 16-byte chunks of 32 positions
        const uint4* p = reinterpret_cast<const uint4*>(code);
        uint4 v = p[0];
#pragma unroll 1
        for (int k = 0; k < NCH; ++k) {
            uint4 vn = (k + 1 < NCH) ? p[k + 1] : v;
            lut_chunk<G>(v.x, v.y, v.z, v.w, 32, table + static_cast<uint32_t>(k) * 32 * 16 * G, S, T);
            v = vn;
        }
    }
    if constexpr (G == 1) {
        sum[0] = S;
    } else {
        uint32_t b1 = T & 0xFFFFu, b3 = T >> 16;
        uint32_t r = S - (b1 << 8) - (b3 << 24);
        sum[0] = r & 0xFFFFu;
        sum[1] = b1;
        sum[2] = r >> 16;
        sum[3] = b3;
    }
}

// canonical(slot, c, probed) of src/index.rs:2036-2045: false when another home h < c of the
// slot was probed by the query.
__device__ __forceinline__ bool canonical(const DevArena& A, uint32_t slot, uint32_t c, const uint32_t* probed) {
    if (A.ma <= 1) return true;
    const uint32_t* h = A.slot_cells + static_cast<uint64_t>(slot) * A.ma;
    for (uint32_t j = 0; j < A.ma; ++j) {
        uint32_t hc = h[j];
        if (hc != kNone && hc < c && ((probed[hc >> 5] >> (hc & 31)) & 1u)) return false;
    }
    return true;
}

// Exact target-th smallest of d values (1-based `want`) supplied by get(i), i < n, d < 65536.
// Two 256-bin LDS histogram passes; every thread returns the value.
template <class Get>
__device__ uint32_t select_kth(uint32_t n, uint32_t want, Get get, uint32_t* hist, uint32_t* scratch) {
    for (uint32_t i = threadIdx.x; i < kHistBins; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) atomicAdd(&hist[get(i) >> 8], 1u);
    __syncthreads();
    // find the high byte: first bin where the inclusive prefix reaches want
    uint32_t hb = 0, below = 0;
    {
        uint32_t v = threadIdx.x < kHistBins ? hist[threadIdx.x] : 0u;
        uint32_t total;
        uint32_t ex = block_excl_scan_u32(v, scratch, &total);
        uint32_t cand = (threadIdx.x < kHistBins && ex < want && ex + v >= want) ? threadIdx.x : kNone;
        hb = block_min_u32(cand, scratch);
        // exclusive prefix at hb
        uint32_t exb = (threadIdx.x == hb) ? ex : 0u;
        below = block_sum_u32(exb, scratch);
    }
    for (uint32_t i = threadIdx.x; i < kHistBins; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        uint32_t d = get(i);
        if ((d >> 8) == hb) atomicAdd(&hist[d & 0xFFu], 1u);
    }
    __syncthreads();
    uint32_t need = want - below;
    uint32_t v = threadIdx.x < kHistBins ? hist[threadIdx.x] : 0u;
    uint32_t total;
    uint32_t ex = block_excl_scan_u32(v, scratch, &total);
    uint32_t cand = (threadIdx.x < kHistBins && ex < need && ex + v >= need) ? threadIdx.x : kNone;
    uint32_t lb = block_min_u32(cand, scratch);
    return (hb << 8) | lb;
}

// f32 acos / cos / exp evaluated in f64 and rounded once. glibc's acosf / cosf / expf (what the
// reference's f32::acos / cos / exp call) are not correctly rounded, so a decision that lands
// within a small band of its threshold is flagged and re-evaluated on the host with libm.
__device__ __forceinline__ float acos_f(float x) { return static_cast<float>(acos(static_cast<double>(x))); }
__device__ __forceinline__ float cos_f(float x) { return static_cast<float>(cos(static_cast<double>(x))); }
__device__ __forceinline__ float exp_f(float x) { return static_cast<float>(exp(static_cast<double>(x))); }

// ---------------------------------------------------------------- upload: FastScan -> entry-major

// Entry e of cell c (member position i) lives in block fs_off[c] + i/32, lane i%32; nibble j
// is byte [(j/2)*32 + (j%2)*16 + lane%16], low half for lanes < 16 (src/quantize.rs:238-265).
__global__ void fs_to_codes_kernel(const uint8_t* __restrict__ fs, const uint32_t* __restrict__ fs_off,
                                   const uint32_t* __restrict__ mem_off, uint32_t M, uint32_t W,
                                   uint32_t* __restrict__ codes) {
    uint32_t c = blockIdx.x;
    if (c >= M) return;
    uint32_t e0 = mem_off[c], len = mem_off[c + 1] - e0;
    const uint32_t bb = W * 256, nd = 2 * W;
    for (uint32_t i = threadIdx.x; i < len; i += blockDim.x) {
        const uint8_t* blk = fs + static_cast<uint64_t>(fs_off[c] + i / 32) * bb;
        uint32_t lane = i % 32, li = lane % 16;
        bool hi = lane >= 16;
        for (uint32_t w = 0; w < nd; ++w) {
            uint32_t dw = 0;
            for (uint32_t t = 0; t < 8; ++t) {
                uint32_t j = w * 8 + t;
                uint8_t byte = blk[(j / 2) * 32 + (j % 2) * 16 + li];
                uint32_t nib = hi ? (byte >> 4) : (byte & 0xFu);
                dw |= nib << (4 * t);
            }
            codes[(static_cast<uint64_t>(e0) + i) * nd + w] = dw;
        }
    }
}

// Test entry point: nibble sums of nb entry-major codes (32 per block) against per-block tables.
template <int NW>
__global__ void entry_sums_kernel(const uint32_t* __restrict__ codes, const uint8_t* __restrict__ luts,
                                  uint32_t n_entries, uint16_t* __restrict__ out) {
    extern __shared__ uint8_t smem[];
    constexpr uint32_t TB = NW * 256;
    uint32_t b = blockIdx.x;  // one FastScan block = 32 entries
    for (uint32_t i = threadIdx.x; i < TB; i += blockDim.x) smem[i] = luts[static_cast<uint64_t>(b) * TB + i];
    __syncthreads();
    uint32_t e = b * 32 + threadIdx.x;
    if (threadIdx.x < 32 && e < n_entries) {
        uint32_t s[1];
        lut_sums<NW, 1>(codes + static_cast<uint64_t>(e) * (2 * NW), smem, s);
        out[e] = static_cast<uint16_t>(s[0]);
    }
}

// ---------------------------------------------------------------- prep + route

// LDS layout of prep_route (dynamic): x[P] f32 | cqs[d] f32 | hs[M] u16 (padded) | keys[sort_cap] u64
// | mins[npos] f32 | hist[P/ ... 513] u32 | scratch[16] u32
template <int NW>
__global__ void __launch_bounds__(kRouteThreads)
prep_route_kernel(DevArena A, Work Wk, KParams K, const float* __restrict__ queries, uint32_t route_only) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t qi = blockIdx.x;
    if (qi >= K.nq) return;
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    const uint32_t d = A.d, P = A.P, M = A.M, npos = A.npos;
    constexpr uint32_t W = NW;
    float* x = reinterpret_cast<float*>(smem);
    float* cqs = x + P;
    uint16_t* hs = reinterpret_cast<uint16_t*>(cqs + ((d + 3) & ~3u));
    uint64_t* keys = reinterpret_cast<uint64_t*>(hs + ((M + 7) & ~7u));
    float* mins = reinterpret_cast<float*>(keys + K.sort_cap);
    uint32_t* hist = reinterpret_cast<uint32_t*>(mins + npos);
    const uint32_t nbins = W * 64 + 1;
    uint32_t* scratch = hist + ((nbins + 3) & ~3u);
    __shared__ float s_cqbase;
    __shared__ uint32_t s_cut, s_nsl;

    const float* q = queries + static_cast<uint64_t>(qi) * d;
    // ---- rotation: copy, zero-pad, 2 x (sign flip, FWHT, x 1/sqrt(P)) (src/quantize.rs:152-163)
    for (uint32_t i = tid; i < P; i += nt) x[i] = i < d ? q[i] : 0.0f;
    for (int r = 0; r < 2; ++r) {
        __syncthreads();
        for (uint32_t i = tid; i < P; i += nt) x[i] *= A.rot_signs[r * P + i];
        for (uint32_t h = 1; h < P; h <<= 1) {
            __syncthreads();
            for (uint32_t t = tid; t < P / 2; t += nt) {
                uint32_t j = (t / h) * 2 * h + (t % h);
                float u = x[j], v = x[j + h];
                x[j] = u + v;
                x[j + h] = u - v;
            }
        }
        __syncthreads();
        for (uint32_t i = tid; i < P; i += nt) x[i] *= A.fht_scale;
    }
    __syncthreads();
    // ---- 1-bit code: bit i = x[i] < 0 over the first W*64 coordinates (src/quantize.rs:57-67)
    uint64_t* qb_out = Wk.qbits + static_cast<uint64_t>(qi) * W;
    for (uint32_t base = 0; base < W * 64; base += nt) {
        uint32_t i = base + tid;
        bool neg = i < W * 64 && i < P && x[i] < 0.0f;
        uint64_t m = __ballot(neg);
        if (lane_id() == 0 && i < W * 64) qb_out[i >> 6] = m;
    }
    // ---- FastScan table (src/quantize.rs:279-313): position j uses x[4j .. 4j+3]
    float lo = INFINITY, hi = -INFINITY;
    float raw[16];
    const bool own = tid < npos;
    if (own) {
        float xs[4];
        for (int t = 0; t < 4; ++t) {
            uint32_t dd = 4 * tid + t;
            xs[t] = dd < P ? x[dd] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            float v = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; ++t) v += ((e >> t) & 1) ? -xs[t] : xs[t];
            raw[e] = v;
            lo = fminf(lo, v);
            hi = fmaxf(hi, v);
        }
        mins[tid] = lo;
    }
    float range = block_max_f32(own ? hi - lo : 0.0f, reinterpret_cast<float*>(scratch));
    range = fmaxf(range, 0.0f);
    const float delta = fmaxf(range / 255.0f, 1e-12f);
    if (own) {
        uint8_t* lut = Wk.lut + static_cast<uint64_t>(qi) * npos * 16 + tid * 16;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            float qv = roundf((raw[e] - lo) / delta);
            qv = fminf(fmaxf(qv, 0.0f), 255.0f);
            lut[e] = static_cast<uint8_t>(qv);
        }
    }
    __syncthreads();
    if (tid == 0) {
        float b = -0.0f;  // Rust's f32 Sum folds from -0.0
        for (uint32_t j = 0; j < npos; ++j) b += mins[j];
        Wk.bias[qi] = b;
        Wk.delta[qi] = delta;
    }
    if (route_only == 2) return;  // query_prep test entry point
    // ---- SQ8 rescore prep: cqs = q * csq_step, cqbase = sum q * csq_min (src/index.rs:1934-1942)
    const bool sq8 = A.cent_sq8 != nullptr;
    if (sq8) {
        for (uint32_t j = tid; j < d; j += nt) cqs[j] = q[j] * A.csq_step[j];
        if (tid == 0) {
            float b = 0.0f;
            for (uint32_t j = 0; j < d; ++j) b += q[j] * A.csq_min[j];
            s_cqbase = b;
        }
    }
    // ---- Hamming against every centroid code + live histogram (src/index.rs:1901-1923)
    for (uint32_t i = tid; i < nbins; i += nt) hist[i] = 0;
    __syncthreads();
    uint64_t qw[W];
#pragma unroll
    for (int w = 0; w < (int)W; ++w) qw[w] = qb_out[w];
    for (uint32_t c = tid; c < M; c += nt) {
        const uint64_t* cb = A.cent_bits + static_cast<uint64_t>(c) * W;
        uint32_t h = 0;
#pragma unroll
        for (int w = 0; w < (int)W; ++w) h += __popcll(qw[w] ^ cb[w]);
        hs[c] = static_cast<uint16_t>(h);
        if (A.live[c]) atomicAdd(&hist[h], 1u);
    }
    __syncthreads();
    // cut = smallest t whose cumulative live count reaches want_c (hamming_cutoff, :86-104)
    {
        uint32_t per = (nbins + nt - 1) / nt, b0 = tid * per, loc = 0;
        for (uint32_t i = b0; i < min(b0 + per, nbins); ++i) loc += hist[i];
        uint32_t total;
        uint32_t ex = block_excl_scan_u32(loc, scratch, &total);
        uint32_t cand = kNone, cum = ex;
        for (uint32_t i = b0; i < min(b0 + per, nbins); ++i) {
            cum += hist[i];
            if (cum >= K.want_c) {
                cand = i;
                break;
            }
        }
        uint32_t cut = block_min_u32(cand, scratch);
        if (tid == 0) s_cut = cut == kNone ? W * 64 : cut;
    }
    __syncthreads();
    const uint32_t cut = s_cut;
    // ---- shortlist: live cells with h <= cut, ascending id, via a block-wide compaction
    {
        uint32_t per = (M + nt - 1) / nt, c0 = tid * per, c1 = min(c0 + per, M), cnt = 0;
        for (uint32_t c = c0; c < c1; ++c) cnt += (A.live[c] && hs[c] <= cut);
        uint32_t total;
        uint32_t pos = block_excl_scan_u32(cnt, scratch, &total);
        if (tid == 0) {
            s_nsl = total;
            atomicMax(&Wk.ctl->max_shortlist, total);
        }
        if (total <= K.sort_cap) {
            for (uint32_t c = c0; c < c1; ++c)
                if (A.live[c] && hs[c] <= cut) keys[pos++] = c;  // id for now; score below
        }
    }
    __syncthreads();
    const uint32_t nsl = s_nsl;
    uint32_t* chosen = Wk.chosen + static_cast<uint64_t>(qi) * K.nprobe;
    float* cscore = Wk.cscore + static_cast<uint64_t>(qi) * K.nprobe;
    if (nsl > K.sort_cap) {
        if (tid == 0) {
            atomicAdd(&Wk.ctl->err_shortlist, 1u);
            Wk.nchosen[qi] = 0;
        }
        return;
    }
    // ---- exact rescore: 8 lanes per cell, the reference's 8-lane FMA order (:777-800)
    const float cqbase = sq8 ? s_cqbase : 0.0f;
    {
        const uint32_t l = tid & 7, grp = tid >> 3, ngrp = nt >> 3;
        const uint32_t rounds = (nsl + ngrp - 1) / ngrp;
        for (uint32_t rr = 0; rr < rounds; ++rr) {
            uint32_t i = rr * ngrp + grp;
            uint32_t c = i < nsl ? static_cast<uint32_t>(keys[i]) : 0u;
            float s;
            if (sq8) {
                const uint8_t* code = A.cent_sq8 + static_cast<uint64_t>(c) * d;
                s = dot8_group(d, l, [&](uint32_t j) { return cqs[j]; },
                               [&](uint32_t j) { return static_cast<float>(code[j]); }) + cqbase;
            } else {
                const float* cen = A.centroids + static_cast<uint64_t>(c) * d;
                s = dot8_group(d, l, [&](uint32_t j) { return q[j]; }, [&](uint32_t j) { return cen[j]; });
            }
            __syncthreads();  // all reads of keys[] in this round happen before the writes
            if (i < nsl && l == 0) keys[i] = desc_score_key(s, c);
        }
    }
    // pad to a power of two with max keys, sort ascending = (score desc, id asc)
    uint32_t n2 = 1;
    while (n2 < nsl) n2 <<= 1;
    __syncthreads();
    for (uint32_t i = nsl + tid; i < n2; i += nt) keys[i] = kKeyMax;
    bitonic_sort_u64(keys, n2);
    const uint32_t cap = min(K.nprobe, nsl);
    for (uint32_t i = tid; i < K.nprobe; i += nt) {
        bool ok = i < cap;
        chosen[i] = ok ? static_cast<uint32_t>(keys[i]) : kNone;
        cscore[i] = ok ? key_score(keys[i]) : __uint_as_float(0x7fc00000u);
    }
    // ---- nucleus over the capped list (:1960-1973); tc >= 1 keeps all cap cells
    if (tid == 0) {
        uint32_t nch = cap;
        if (K.use_nucleus && cap > 0) {
            float max_s = key_score(keys[0]);
            float z = -0.0f;
            for (uint32_t i = 0; i < cap; ++i) z += exp_f((key_score(keys[i]) - max_s) * K.beta);
            float cum = 0.0f;
            bool near = false;
            nch = cap;
            for (uint32_t i = 0; i < cap; ++i) {
                cum += exp_f((key_score(keys[i]) - max_s) * K.beta) / (z + 1e-9f);
                if (fabsf(cum - K.tc) <= K.nucleus_band) near = true;
                if (cum >= K.tc) {
                    nch = i + 1;
                    break;
                }
            }
            if (near) {
                uint32_t slot = atomicAdd(&Wk.ctl->nflag_route, 1u);
                Wk.flag_route[slot] = qi;
            }
        }
        Wk.nchosen[qi] = nch;
    }
}

// ---------------------------------------------------------------- seed scan + tau + adaptive cut

template <int NW>
__global__ void __launch_bounds__(kScanThreads)
seed_kernel(DevArena A, Work Wk, KParams K) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t qi = blockIdx.x;
    if (qi >= K.nq) return;
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    constexpr uint32_t TB = NW * 256;
    uint8_t* table = smem;
    uint32_t* probed = reinterpret_cast<uint32_t*>(smem + TB);
    uint32_t* hist = probed + ((A.MW + 3) & ~3u);
    uint32_t* scratch = hist + kHistBins;
    float* fsc = reinterpret_cast<float*>(scratch + 16);
    __shared__ uint32_t s_cnt;

    const uint32_t nch = Wk.nchosen[qi];
    const uint32_t* chosen = Wk.chosen + static_cast<uint64_t>(qi) * K.nprobe;
    const float* cscore = Wk.cscore + static_cast<uint64_t>(qi) * K.nprobe;
    const uint8_t* lut = Wk.lut + static_cast<uint64_t>(qi) * TB;
    for (uint32_t i = tid; i < TB / 4; i += nt) reinterpret_cast<uint32_t*>(table)[i] = reinterpret_cast<const uint32_t*>(lut)[i];
    for (uint32_t i = tid; i < A.MW; i += nt) probed[i] = 0;
    if (tid == 0) s_cnt = 0;
    __syncthreads();
    for (uint32_t i = tid; i < nch; i += nt) atomicOr(&probed[chosen[i] >> 5], 1u << (chosen[i] & 31));
    __syncthreads();
    uint32_t* gprobed = Wk.probed + static_cast<uint64_t>(qi) * A.MW;
    for (uint32_t i = tid; i < A.MW; i += nt) gprobed[i] = probed[i];

    // ---- seed: every canonical member of the first ns probed cells (src/index.rs:2150-2154)
    const uint32_t ns = min(kSeedCells, nch);
    uint2* seed = Wk.seed + static_cast<uint64_t>(qi) * K.seed_cap;
    if (tid < ns) {
        const uint32_t c = chosen[tid];
        atomicAdd(&Wk.ctl->seed_blocks, static_cast<unsigned long long>((A.mem_off[c + 1] - A.mem_off[c] + 31) / 32));
    }
    for (uint32_t si = 0; si < ns; ++si) {
        const uint32_t c = chosen[si];
        const uint32_t e0 = A.mem_off[c], len = A.mem_off[c + 1] - e0;
        for (uint32_t base = 0; base < len; base += nt) {
            uint32_t i = base + tid;
            bool pass = false;
            uint32_t dv = 0, slot = 0;
            if (i < len) {
                uint32_t s[1];
                lut_sums<NW, 1>(A.codes + (static_cast<uint64_t>(e0) + i) * (2 * NW), table, s);
                dv = A.maxk - s[0];
                slot = A.members[e0 + i];
                pass = canonical(A, slot, c, probed);
            }
            uint64_t m = __ballot(pass);
            uint32_t wbase = 0;
            if (lane_id() == 0 && m) wbase = atomicAdd(&s_cnt, static_cast<uint32_t>(__popcll(m)));
            wbase = __shfl(wbase, 0, kWave);
            if (pass) seed[wbase + lanes_below(m)] = make_uint2(dv, slot);
        }
    }
    __syncthreads();
    const uint32_t cnt = s_cnt;
    __threadfence_block();
    // ---- tau = target-th smallest seed d (src/index.rs:2155-2160)
    uint32_t tau = A.maxk;
    if (cnt >= K.target) tau = select_kth(cnt, K.target, [&](uint32_t i) { return seed[i].x; }, hist, scratch);
    // ---- adaptive cut (src/index.rs:2166-2188): b_i = cos(max(acos(clamp(cs_i)) - r_c, 0)),
    // suffix max from the end, rest_end = first i >= ns with suffix_i < thr - margin
    uint32_t rest_end = nch;
    if (K.adaptive && cnt >= K.target && ns < nch) {
        const float delta = Wk.delta[qi], bias = Wk.bias[qi];
        const float est = delta * static_cast<float>(A.maxk - tau) + bias;
        const float thr = fminf(fmaxf(est / K.norm, -1.0f), 1.0f);
        const float T = thr - K.at_margin;
        // suffix max over [i, nch): chunked, each thread owns a contiguous run
        const uint32_t m = nch - ns, per = (m + nt - 1) / nt;
        const uint32_t i0 = ns + tid * per, i1 = min(i0 + per, nch);
        float run_max = -INFINITY;
        for (uint32_t i = i1; i-- > i0;) {
            float cs = fminf(fmaxf(cscore[i], -1.0f), 1.0f);
            float b = cos_f(fmaxf(acos_f(cs) - A.r_bound[chosen[i]], 0.0f));
            run_max = fmaxf(run_max, b);
        }
        // exclusive suffix of the run maxima of later threads
        fsc[tid] = run_max;
        __syncthreads();
        float later = -INFINITY;
        for (uint32_t t = tid + 1; t < nt; ++t) later = fmaxf(later, fsc[t]);
        // walk own run forward: suffix_i = max(b_i.., later)
        uint32_t first = kNone;
        bool near = false;
        {
            // recompute suffix values from the end of the run
            float sfx = later;
            // need forward order of the first crossing: collect in reverse, remember the smallest i
            for (uint32_t i = i1; i-- > i0;) {
                float cs = fminf(fmaxf(cscore[i], -1.0f), 1.0f);
                float b = cos_f(fmaxf(acos_f(cs) - A.r_bound[chosen[i]], 0.0f));
                sfx = fmaxf(sfx, b);
                if (sfx < T) first = i;
                if (fabsf(sfx - T) <= K.prune_band) near = true;
            }
        }
        uint32_t fe = block_min_u32(first, scratch);
        uint32_t any_near = block_sum_u32(near ? 1u : 0u, scratch);
        if (fe != kNone) rest_end = fe;
        if (tid == 0 && any_near) {
            uint32_t slot = atomicAdd(&Wk.ctl->nflag_prune, 1u);
            Wk.flag_prune[slot] = qi;
        }
    }
    if (tid == 0) {
        Wk.seed_cnt[qi] = cnt;
        Wk.tau[qi] = tau;
        Wk.rest_end[qi] = rest_end;
    }
}

// ---------------------------------------------------------------- inversion: cell -> queries

__global__ void invert_count_kernel(Work Wk, KParams K, const uint32_t* __restrict__ mem_off) {
    uint32_t qi = blockIdx.x;
    if (qi >= K.nq) return;
    uint32_t ns = min(kSeedCells, Wk.nchosen[qi]), re = Wk.rest_end[qi];
    const uint32_t* chosen = Wk.chosen + static_cast<uint64_t>(qi) * K.nprobe;
    uint32_t blocks = 0;
    for (uint32_t i = ns + threadIdx.x; i < re; i += blockDim.x) {
        uint32_t c = chosen[i];
        atomicAdd(&Wk.cell_cnt[c], 1u);
        blocks += (mem_off[c + 1] - mem_off[c] + 31) / 32;
    }
    blocks = wave_sum_u32(blocks);
    if (threadIdx.x == 0 && blocks) {
        atomicAdd(&Wk.ctl->scan_blocks, static_cast<unsigned long long>(blocks));
        atomicAdd(&Wk.ctl->scan_pairs, static_cast<unsigned long long>(re - ns));
    }
}

// Single workgroup: exclusive scan of cell_cnt[0..M) -> cell_off[0..M], cell_cur = cell_off.
__global__ void invert_scan_kernel(Work Wk, uint32_t M) {
    __shared__ uint32_t scratch[32];
    __shared__ uint32_t carry;
    if (threadIdx.x == 0) carry = 0;
    __syncthreads();
    for (uint32_t base = 0; base < M; base += blockDim.x) {
        uint32_t i = base + threadIdx.x;
        uint32_t v = i < M ? Wk.cell_cnt[i] : 0u;
        uint32_t total;
        uint32_t ex = block_excl_scan_u32(v, scratch, &total);
        uint32_t c0 = carry;
        if (i < M) {
            Wk.cell_off[i] = c0 + ex;
            Wk.cell_cur[i] = c0 + ex;
        }
        __syncthreads();
        if (threadIdx.x == 0) carry = c0 + total;
        __syncthreads();
    }
    if (threadIdx.x == 0) Wk.cell_off[M] = carry;
}

__global__ void invert_fill_kernel(Work Wk, KParams K) {
    uint32_t qi = blockIdx.x;
    if (qi >= K.nq) return;
    uint32_t ns = min(kSeedCells, Wk.nchosen[qi]), re = Wk.rest_end[qi];
    const uint32_t* chosen = Wk.chosen + static_cast<uint64_t>(qi) * K.nprobe;
    for (uint32_t i = ns + threadIdx.x; i < re; i += blockDim.x) {
        uint32_t c = chosen[i];
        uint32_t pos = atomicAdd(&Wk.cell_cur[c], 1u);
        Wk.qof[pos] = qi;
    }
}

// ---------------------------------------------------------------- the cell-major scan

// One workgroup per cell (src/index.rs:2231-2275 is the CPU loop this replaces). Lanes own
// members; their codes stay in registers while groups of kG probing queries stream through.
template <int NW>
__global__ void __launch_bounds__(kScanThreads)
cell_scan_kernel(DevArena A, Work Wk, KParams K) {
    constexpr uint32_t TB = NW * 256;
    __shared__ __align__(16) uint8_t table[kG * TB];
    __shared__ uint32_t s_q[kG], s_t[kG];
    const uint32_t c = blockIdx.x;
    if (c >= A.M) return;
    const uint32_t q0 = Wk.cell_off[c], nqc = Wk.cell_off[c + 1] - q0;
    const uint32_t e0 = A.mem_off[c], len = A.mem_off[c + 1] - e0;
    if (nqc == 0 || len == 0) return;
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    for (uint32_t ebase = 0; ebase < len; ebase += nt) {
        const uint32_t i = ebase + tid;
        const bool have = i < len;
        // lanes past the end read the cell's first member (in bounds) and emit nothing
        const uint32_t* code = A.codes + (static_cast<uint64_t>(e0) + (have ? i : 0u)) * (2 * NW);
        const uint32_t slot = have ? A.members[e0 + i] : 0u;
        for (uint32_t g0 = 0; g0 < nqc; g0 += kG) {
            const uint32_t ng = min(kG, nqc - g0);
            __syncthreads();
            if (tid < kG) {
                uint32_t qq = tid < ng ? Wk.qof[q0 + g0 + tid] : kNone;
                s_q[tid] = qq;
                s_t[tid] = qq != kNone ? Wk.tau[qq] : 0u;
            }
            // interleave the group's tables: table[x*4 + g] = lut_g[x]
            for (uint32_t x4 = tid; x4 < TB / 4; x4 += nt) {
                uint32_t v[kG];
#pragma unroll
                for (uint32_t g = 0; g < kG; ++g) {
                    uint32_t qq = g < ng ? Wk.qof[q0 + g0 + g] : kNone;
                    v[g] = qq != kNone ? reinterpret_cast<const uint32_t*>(Wk.lut + static_cast<uint64_t>(qq) * TB)[x4] : 0u;
                }
                // 4x4 byte transpose: out[b] = (v0.b, v1.b, v2.b, v3.b)
                uint32_t lo01 = __builtin_amdgcn_perm(v[1], v[0], 0x05010400u);  // v0.b0 v1.b0 v0.b1 v1.b1
                uint32_t hi01 = __builtin_amdgcn_perm(v[1], v[0], 0x07030602u);  // v0.b2 v1.b2 v0.b3 v1.b3
                uint32_t lo23 = __builtin_amdgcn_perm(v[3], v[2], 0x05010400u);
                uint32_t hi23 = __builtin_amdgcn_perm(v[3], v[2], 0x07030602u);
                uint4 o;
                o.x = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
                o.y = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
                o.z = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
                o.w = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
                reinterpret_cast<uint4*>(table)[x4] = o;
            }
            __syncthreads();
            uint32_t sums[kG];
            lut_sums<NW, kG>(code, table, sums);
#pragma unroll
            for (uint32_t g = 0; g < kG; ++g) {
                const uint32_t qq = s_q[g];
                bool pass = false;
                uint32_t dv = 0;
                if (have && qq != kNone) {
                    dv = A.maxk - sums[g];
                    if (dv <= s_t[g]) pass = canonical(A, slot, c, Wk.probed + static_cast<uint64_t>(qq) * A.MW);
                }
                uint64_t m = __ballot(pass);
                if (m) {
                    uint32_t wbase = 0;
                    if (lane_id() == 0) wbase = atomicAdd(&Wk.cand_cnt[qq], static_cast<uint32_t>(__popcll(m)));
                    wbase = __shfl(wbase, 0, kWave);
                    uint32_t pos = wbase + lanes_below(m);
                    if (pass && pos < K.cand_cap) Wk.cand[static_cast<uint64_t>(qq) * K.cand_cap + pos] = make_uint2(dv, slot);
                }
            }
        }
    }
}

// ---------------------------------------------------------------- finish: cut + rerank + top-k

__global__ void __launch_bounds__(kScanThreads)
finish_kernel(DevArena A, Work Wk, KParams K, const float* __restrict__ queries, uint32_t* __restrict__ out_slots,
              float* __restrict__ out_scores) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t qi = blockIdx.x;
    if (qi >= K.nq) return;
    const uint32_t tid = threadIdx.x, nt = blockDim.x, d = A.d;
    uint32_t* hist = reinterpret_cast<uint32_t*>(smem);
    uint32_t* scratch = hist + kHistBins;
    float* qs = reinterpret_cast<float*>(scratch + 32);
    uint64_t* keys = reinterpret_cast<uint64_t*>(qs + ((d + 3) & ~3u));
    __shared__ uint32_t s_n;
    __shared__ float s_base;

    const uint32_t ns_cnt = Wk.seed_cnt[qi];
    const uint32_t nc = min(Wk.cand_cnt[qi], K.cand_cap);
    const uint2* seed = Wk.seed + static_cast<uint64_t>(qi) * K.seed_cap;
    const uint2* cand = Wk.cand + static_cast<uint64_t>(qi) * K.cand_cap;
    const uint32_t total = ns_cnt + nc;
    auto get_d = [&](uint32_t i) { return i < ns_cnt ? seed[i].x : cand[i - ns_cnt].x; };
    // ---- exact cut at target, every tie kept (src/index.rs:2281-2293)
    // G = target-th smallest d; with fewer than target candidates every one is kept
    uint32_t cutv = A.maxk;
    if (total >= K.target) cutv = select_kth(total, K.target, get_d, hist, scratch);
    // ---- compact the survivors into fin[]
    uint2* fin = Wk.fin + static_cast<uint64_t>(qi) * K.fin_cap;
    if (tid == 0) s_n = 0;
    __syncthreads();
    for (uint32_t base = 0; base < total; base += nt) {
        uint32_t i = base + tid;
        uint2 e = make_uint2(0, 0);
        bool pass = false;
        if (i < total) {
            e = i < ns_cnt ? seed[i] : cand[i - ns_cnt];
            pass = e.x <= cutv;
        }
        uint64_t m = __ballot(pass);
        uint32_t wbase = 0;
        if (lane_id() == 0 && m) wbase = atomicAdd(&s_n, static_cast<uint32_t>(__popcll(m)));
        wbase = __shfl(wbase, 0, kWave);
        if (pass) fin[wbase + lanes_below(m)] = e;
    }
    __syncthreads();
    const uint32_t n = s_n;
    __threadfence_block();
    // ---- exact rerank (src/index.rs:1309-1378): f32 dot_f32, or SQ8 base + dot_f32_u8
    const float* q = queries + static_cast<uint64_t>(qi) * d;
    const bool sq8 = A.rerank_mode == MAIVS_RERANK_SQ8;
    if (sq8) {
        for (uint32_t j = tid; j < d; j += nt) qs[j] = q[j] * A.sq_step[j];
        if (tid == 0) {
            float b = 0.0f;
            for (uint32_t j = 0; j < d; ++j) b += q[j] * A.sq_min[j];
            s_base = b;
        }
    } else {
        for (uint32_t j = tid; j < d; j += nt) qs[j] = q[j];
    }
    __syncthreads();
    uint32_t n2 = 1;
    while (n2 < n) n2 <<= 1;
    const bool in_lds = n2 <= K.fin_sort_cap;
    uint64_t* kk = in_lds ? keys : (Wk.keys + static_cast<uint64_t>(qi) * K.key_cap);
    {
        const uint32_t l = tid & 7, grp = tid >> 3, ngrp = nt >> 3;
        const uint32_t rounds = (n + ngrp - 1) / ngrp;
        const float base = sq8 ? s_base : 0.0f;
        for (uint32_t rr = 0; rr < rounds; ++rr) {
            uint32_t i = rr * ngrp + grp;
            uint32_t slot = i < n ? fin[i].y : 0u;
            float s;
            if (sq8) {
                const uint8_t* code = A.sq8 + static_cast<uint64_t>(slot) * d;
                s = base + dot8_group(d, l, [&](uint32_t j) { return qs[j]; },
                                      [&](uint32_t j) { return static_cast<float>(code[j]); });
            } else {
                const float* row = A.vecs + static_cast<uint64_t>(slot) * d;
                s = dot8_group(d, l, [&](uint32_t j) { return qs[j]; }, [&](uint32_t j) { return row[j]; });
            }
            if (i < n && l == 0) kk[i] = desc_score_key(s, slot);
        }
    }
    __syncthreads();
    for (uint32_t i = n + tid; i < n2; i += nt) kk[i] = kKeyMax;
    bitonic_sort_u64(kk, n2);
    for (uint32_t i = tid; i < K.k; i += nt) {
        bool ok = i < n;
        out_slots[static_cast<uint64_t>(qi) * K.k + i] = ok ? static_cast<uint32_t>(kk[i]) : kNone;
        out_scores[static_cast<uint64_t>(qi) * K.k + i] = ok ? key_score(kk[i]) : -INFINITY;
    }
    if (tid == 0) {
        Wk.cut[qi] = cutv;
        Wk.ncand[qi] = n;
        atomicMax(&Wk.ctl->max_cand, Wk.cand_cnt[qi]);
        atomicAdd(&Wk.ctl->survivors, static_cast<unsigned long long>(Wk.cand_cnt[qi]));
        atomicAdd(&Wk.ctl->rerank_rows, static_cast<unsigned long long>(n));
    }
}

}  // namespace

// ================================================================ host side

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
    uint32_t cap_nq = 0, cap_nprobe = 0, cap_k = 0, cap_cand = 0, cap_seed = 0, cap_fin = 0, cap_key = 0;
    uint32_t cand_nq = 0;
    uint32_t max_sort_cap_route = 0;  // largest shortlist sort the route kernel's LDS can hold
    size_t lds_route_fixed = 0, lds_seed = 0, lds_finish = 0;
    hipEvent_t ev[8] = {};
    // last call, for maivs_gpu_last_candidates
    uint32_t last_nq = 0, last_fin_cap = 0;
    uint32_t initial_cand_cap = 4096;
};

namespace {

int fail(maivs_gpu_ctx* ctx, int code, const char* fmt, ...) {
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
int dalloc(maivs_gpu_ctx* ctx, std::vector<void*>& owner, T** p, size_t count) {
    *p = nullptr;
    if (count == 0) count = 1;
    void* v = nullptr;
    HIP_TRY(ctx, hipMalloc(&v, count * sizeof(T)));
    owner.push_back(v);
    *p = static_cast<T*>(v);
    return 0;
}

template <class T>
int dupload(maivs_gpu_ctx* ctx, const T* src, size_t count, T** out) {
    int rc = dalloc(ctx, ctx->arena_allocs, out, count);
    if (rc) return rc;
    if (src && count) HIP_TRY(ctx, hipMemcpyAsync(*out, src, count * sizeof(T), hipMemcpyHostToDevice, ctx->stream));
    return 0;
}

void free_all(std::vector<void*>& v) {
    for (void* p : v) (void)hipFree(p);
    v.clear();
}

bool supported_nw(uint32_t w) { return w == 1 || w == 2 || w == 4 || w == 8 || w == 16; }

#define DISPATCH_NW(W, ...)                              \
    switch (W) {                                         \
        case 1: { constexpr int NW = 1; __VA_ARGS__; break; } \
        case 2: { constexpr int NW = 2; __VA_ARGS__; break; } \
        case 4: { constexpr int NW = 4; __VA_ARGS__; break; } \
        case 8: { constexpr int NW = 8; __VA_ARGS__; break; } \
        default: { constexpr int NW = 16; __VA_ARGS__; break; } \
    }

size_t route_lds(const DevArena& A, uint32_t sort_cap) {
    size_t b = A.P * 4 + ((A.d + 3) & ~3u) * 4 + ((A.M + 7) & ~7u) * 2 + static_cast<size_t>(sort_cap) * 8 +
               A.npos * 4 + (((A.W * 64 + 1) + 3) & ~3u) * 4 + 16 * 4;
    return b;
}

// Per-query and per-cell work buffers for (nq, nprobe, k); grows only. Candidate buffers are
// separate (ensure_cand) so that growing them never moves the staged queries or outputs.
int ensure_work(maivs_gpu_ctx* ctx, uint32_t nq, uint32_t nprobe, uint32_t k) {
    const DevArena& A = ctx->A;
    uint32_t seed_cap = kSeedCells * std::max<uint32_t>(A.max_cell_len, 1);
    if (nq <= ctx->cap_nq && nprobe <= ctx->cap_nprobe && k <= ctx->cap_k && seed_cap <= ctx->cap_seed) return 0;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    free_all(ctx->work_allocs);
    free_all(ctx->cand_allocs);
    ctx->cand_nq = 0;
    nq = std::max(nq, ctx->cap_nq);
    nprobe = std::max(nprobe, ctx->cap_nprobe);
    k = std::max(k, ctx->cap_k);
    Work& W = ctx->Wk;
    auto& o = ctx->work_allocs;
    const uint64_t nql = nq;
    int rc = 0;
    rc |= dalloc(ctx, o, &W.q, nql * A.d);
    rc |= dalloc(ctx, o, &W.qbits, nql * A.W);
    rc |= dalloc(ctx, o, &W.lut, nql * A.npos * 16);
    rc |= dalloc(ctx, o, &W.delta, nql);
    rc |= dalloc(ctx, o, &W.bias, nql);
    rc |= dalloc(ctx, o, &W.chosen, nql * nprobe);
    rc |= dalloc(ctx, o, &W.cscore, nql * nprobe);
    rc |= dalloc(ctx, o, &W.nchosen, nql);
    rc |= dalloc(ctx, o, &W.probed, nql * A.MW);
    rc |= dalloc(ctx, o, &W.seed, nql * seed_cap);
    rc |= dalloc(ctx, o, &W.seed_cnt, nql);
    rc |= dalloc(ctx, o, &W.tau, nql);
    rc |= dalloc(ctx, o, &W.rest_end, nql);
    rc |= dalloc(ctx, o, &W.cand_cnt, nql);
    rc |= dalloc(ctx, o, &W.cut, nql);
    rc |= dalloc(ctx, o, &W.ncand, nql);
    rc |= dalloc(ctx, o, &W.out_slots, nql * k);
    rc |= dalloc(ctx, o, &W.out_scores, nql * k);
    rc |= dalloc(ctx, o, &W.cell_cnt, static_cast<uint64_t>(A.M) + 1);
    rc |= dalloc(ctx, o, &W.cell_off, static_cast<uint64_t>(A.M) + 1);
    rc |= dalloc(ctx, o, &W.cell_cur, static_cast<uint64_t>(A.M) + 1);
    rc |= dalloc(ctx, o, &W.qof, nql * nprobe);
    rc |= dalloc(ctx, o, &W.flag_route, nql);
    rc |= dalloc(ctx, o, &W.flag_prune, nql);
    rc |= dalloc(ctx, o, &W.ctl, 1);
    if (rc) {
        free_all(ctx->work_allocs);
        ctx->cap_nq = ctx->cap_nprobe = ctx->cap_k = ctx->cap_seed = 0;
        return rc;
    }
    ctx->cap_nq = nq;
    ctx->cap_nprobe = nprobe;
    ctx->cap_k = k;
    ctx->cap_seed = seed_cap;
    return 0;
}

// Candidate, final-list and sort-key buffers for (cap_nq, cand_cap); grows only.
int ensure_cand(maivs_gpu_ctx* ctx, uint32_t cand_cap) {
    if (ctx->cand_nq >= ctx->cap_nq && cand_cap <= ctx->cap_cand && ctx->cand_nq) return 0;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    free_all(ctx->cand_allocs);
    cand_cap = std::max(cand_cap, ctx->cap_cand);
    uint32_t fin_cap = ctx->cap_seed + cand_cap;
    uint32_t key_cap = 1;
    while (key_cap < fin_cap) key_cap <<= 1;
    Work& W = ctx->Wk;
    auto& o = ctx->cand_allocs;
    const uint64_t nql = ctx->cap_nq;
    int rc = 0;
    rc |= dalloc(ctx, o, &W.cand, nql * cand_cap);
    rc |= dalloc(ctx, o, &W.fin, nql * fin_cap);
    rc |= dalloc(ctx, o, &W.keys, nql * key_cap);
    if (rc) {
        free_all(ctx->cand_allocs);
        ctx->cand_nq = 0;
        ctx->cap_cand = 0;
        return rc;
    }
    ctx->cand_nq = ctx->cap_nq;
    ctx->cap_cand = cand_cap;
    ctx->cap_fin = fin_cap;
    ctx->cap_key = key_cap;
    return 0;
}

int ensure_all(maivs_gpu_ctx* ctx, uint32_t nq, uint32_t nprobe, uint32_t k) {
    int rc = ensure_work(ctx, nq, std::max<uint32_t>(nprobe, 1), std::max<uint32_t>(k, 1));
    if (rc) return rc;
    return ensure_cand(ctx, std::max(ctx->cap_cand, ctx->initial_cand_cap));
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
    K.cand_cap = ctx->cap_cand;
    K.fin_cap = ctx->cap_fin;
    K.key_cap = ctx->cap_key;
    K.fin_sort_cap = kFinishSortCap;
    K.tc = p->target_confidence;
    K.beta = p->beta;
    K.at_margin = p->at_margin;
    // norm = sqrt(2 * dim_pad / pi) in f32 (src/index.rs:2169)
    K.norm = std::sqrt(2.0f * static_cast<float>(A.P) / static_cast<float>(M_PI));
    K.prune_band = kPruneBand;
    K.nucleus_band = kNucleusBand;
    return K;
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

int launch_route(maivs_gpu_ctx* ctx, const KParams& K, const float* d_q, uint32_t mode) {
    const DevArena& A = ctx->A;
    const size_t lds = ctx->lds_route_fixed + static_cast<size_t>(K.sort_cap) * 8;
    DISPATCH_NW(A.W, hipLaunchKernelGGL(prep_route_kernel<NW>, dim3(K.nq), dim3(kRouteThreads), lds, ctx->stream, A,
                                        ctx->Wk, K, d_q, mode));
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

int launch_seed(maivs_gpu_ctx* ctx, const KParams& K) {
    const DevArena& A = ctx->A;
    DISPATCH_NW(A.W, hipLaunchKernelGGL(seed_kernel<NW>, dim3(K.nq), dim3(kScanThreads), ctx->lds_seed,
                                        ctx->stream, A, ctx->Wk, K));
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

int launch_scan(maivs_gpu_ctx* ctx, const KParams& K) {
    const DevArena& A = ctx->A;
    Work& W = ctx->Wk;
    HIP_TRY(ctx, hipMemsetAsync(W.cell_cnt, 0, (A.M + 1) * sizeof(uint32_t), ctx->stream));
    HIP_TRY(ctx, hipMemsetAsync(W.cand_cnt, 0, K.nq * sizeof(uint32_t), ctx->stream));
    hipLaunchKernelGGL(invert_count_kernel, dim3(K.nq), dim3(64), 0, ctx->stream, W, K, A.mem_off);
    hipLaunchKernelGGL(invert_scan_kernel, dim3(1), dim3(1024), 0, ctx->stream, W, A.M);
    hipLaunchKernelGGL(invert_fill_kernel, dim3(K.nq), dim3(64), 0, ctx->stream, W, K);
    HIP_TRY(ctx, hipGetLastError());
    HIP_TRY(ctx, hipEventRecord(ctx->ev[4], ctx->stream));
    DISPATCH_NW(A.W, hipLaunchKernelGGL(cell_scan_kernel<NW>, dim3(A.M), dim3(kScanThreads), 0, ctx->stream, A,
                                        W, K));
    HIP_TRY(ctx, hipGetLastError());
    return 0;
}

int launch_finish(maivs_gpu_ctx* ctx, const KParams& K, const float* d_q, uint32_t* d_slots, float* d_scores) {
    hipLaunchKernelGGL(finish_kernel, dim3(K.nq), dim3(kScanThreads), ctx->lds_finish, ctx->stream, ctx->A, ctx->Wk,
                       K, d_q, d_slots, d_scores);
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

int read_ctl(maivs_gpu_ctx* ctx, Ctl* ctl) {
    HIP_TRY(ctx, hipMemcpyAsync(ctl, ctx->Wk.ctl, sizeof(Ctl), hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

// The whole batch. Stages after the first pass only re-run when the control block asks:
// (1) a nucleus decision within kNucleusBand of tc, (2) an adaptive cut within kPruneBand of its
// threshold (both re-evaluated with the host libm the reference uses), (3) a candidate buffer
// overflow (grown to the exact count), (4) a shortlist larger than the on-chip sort.
int run_search(maivs_gpu_ctx* ctx, const float* d_q, uint32_t nq, const maivs_search_params* p, uint32_t* d_slots,
               float* d_scores, maivs_gpu_stats* st) {
    if (!ctx->uploaded) return fail(ctx, MAIVS_ERR_NOT_UPLOADED, "no arena uploaded");
    if (p->k == 0) return fail(ctx, MAIVS_ERR_ARG, "k must be > 0");
    const DevArena& A = ctx->A;
    int rc = ensure_all(ctx, nq, p->nprobe, p->k);
    if (rc) return rc;
    Work& W = ctx->Wk;
    maivs_gpu_stats local{};
    maivs_gpu_stats& S = st ? *st : local;
    S = maivs_gpu_stats{};
    ctx->last_nq = 0;
    if (nq == 0) return 0;
    KParams K = make_params(ctx, nq, p);
    if (p->nprobe == 0 || K.want_c == 0) {
        // route_batch returns empty probe lists (src/index.rs:1887-1889): padded results
        std::vector<uint32_t> s(static_cast<size_t>(nq) * p->k, kNone);
        std::vector<float> f(static_cast<size_t>(nq) * p->k, -INFINITY);
        HIP_TRY(ctx, hipMemcpyAsync(d_slots, s.data(), s.size() * 4, hipMemcpyHostToDevice, ctx->stream));
        HIP_TRY(ctx, hipMemcpyAsync(d_scores, f.data(), f.size() * 4, hipMemcpyHostToDevice, ctx->stream));
        HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        return 0;
    }
    Ctl ctl{};
    for (;;) {
        HIP_TRY(ctx, hipMemsetAsync(W.ctl, 0, sizeof(Ctl), ctx->stream));
        HIP_TRY(ctx, hipEventRecord(ctx->ev[0], ctx->stream));
        if ((rc = launch_route(ctx, K, d_q, 0))) return rc;
        HIP_TRY(ctx, hipEventRecord(ctx->ev[1], ctx->stream));
        if ((rc = launch_seed(ctx, K))) return rc;
        HIP_TRY(ctx, hipEventRecord(ctx->ev[2], ctx->stream));
        if ((rc = launch_scan(ctx, K))) return rc;
        HIP_TRY(ctx, hipEventRecord(ctx->ev[5], ctx->stream));
        if ((rc = launch_finish(ctx, K, d_q, d_slots, d_scores))) return rc;
        HIP_TRY(ctx, hipEventRecord(ctx->ev[6], ctx->stream));
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
    float ms;
    if (hipEventElapsedTime(&ms, ctx->ev[0], ctx->ev[6]) == hipSuccess) S.ms_total = ms;
    if (hipEventElapsedTime(&ms, ctx->ev[0], ctx->ev[1]) == hipSuccess) S.ms_prep = S.ms_route = ms;
    if (hipEventElapsedTime(&ms, ctx->ev[1], ctx->ev[2]) == hipSuccess) S.ms_seed = ms;
    if (hipEventElapsedTime(&ms, ctx->ev[2], ctx->ev[4]) == hipSuccess) S.ms_invert = ms;
    if (hipEventElapsedTime(&ms, ctx->ev[4], ctx->ev[5]) == hipSuccess) S.ms_scan = ms;
    if (hipEventElapsedTime(&ms, ctx->ev[5], ctx->ev[6]) == hipSuccess) S.ms_rerank = ms;
    S.seed_blocks = ctl.seed_blocks;
    S.scan_blocks = ctl.scan_blocks;

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
            HIP_TRY(ctx, hipMemsetAsync(W.ctl, 0, sizeof(Ctl), ctx->stream));
            if ((rc = launch_seed(ctx, K))) return rc;
            if ((rc = launch_scan(ctx, K))) return rc;
            if ((rc = launch_finish(ctx, K, d_q, d_slots, d_scores))) return rc;
            if ((rc = read_ctl(ctx, &ctl))) return rc;
            S.seed_blocks = ctl.seed_blocks;
            S.scan_blocks = ctl.scan_blocks;
        }
    }
    // (2) adaptive cuts near their threshold
    bool rerun_scan = false;
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
            }
        }
    }
    // (3) candidate overflow: grow to the exact count (cand_cnt counts past the capacity)
    if (ctl.max_cand > ctx->cap_cand) {
        uint32_t need = ctl.max_cand + ctl.max_cand / 4 + 64;
        ctx->initial_cand_cap = std::max(ctx->initial_cand_cap, need);
        if ((rc = ensure_cand(ctx, need))) return rc;
        K = make_params(ctx, nq, p);
        rerun_scan = true;
    }
    if (rerun_scan) {
        S.reruns++;
        HIP_TRY(ctx, hipMemsetAsync(W.ctl, 0, sizeof(Ctl), ctx->stream));
        // the seed stage is not re-run: keep its counter
        if ((rc = launch_scan(ctx, K))) return rc;
        if ((rc = launch_finish(ctx, K, d_q, d_slots, d_scores))) return rc;
        if ((rc = read_ctl(ctx, &ctl))) return rc;
        if (ctl.max_cand > ctx->cap_cand) return fail(ctx, MAIVS_ERR_HIP, "candidate count changed between passes");
        S.scan_blocks = ctl.scan_blocks;
    }
    // work counters of the pass that produced the results
    S.scan_pairs = ctl.scan_pairs;
    S.survivors = ctl.survivors;
    S.rerank_rows = ctl.rerank_rows;
    ctx->last_nq = nq;
    return 0;
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
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return MAIVS_ERR_HIP;
    }
    for (auto& e : ctx->ev) {
        if (hipEventCreate(&e) != hipSuccess) {
            delete ctx;
            return MAIVS_ERR_HIP;
        }
    }
    *out = ctx;
    return 0;
}

void maivs_gpu_destroy(maivs_gpu_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    free_all(ctx->work_allocs);
    free_all(ctx->cand_allocs);
    free_all(ctx->arena_allocs);
    for (auto& e : ctx->ev)
        if (e) (void)hipEventDestroy(e);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

const char* maivs_gpu_last_error(const maivs_gpu_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int maivs_gpu_upload_arena(maivs_gpu_ctx* ctx, const maivs_arena_desc* a) {
    if (!ctx || !a) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (!a->fs_codes || !a->fs_off || !a->mem_off || !a->members || !a->cent_bits || !a->rot_signs || !a->r_bound)
        return fail(ctx, MAIVS_ERR_ARG, "arena is missing FastScan blocks, members, centroid codes or radii");
    if (!supported_nw(a->n_words)) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "n_words %u not in {1,2,4,8,16}", a->n_words);
    if (a->max_assign > 1 && !a->slot_cells) return fail(ctx, MAIVS_ERR_ARG, "slot_cells missing");
    if (!a->cent_sq8 && !a->centroids) return fail(ctx, MAIVS_ERR_ARG, "no centroid store for the rescore");
    if (a->cent_sq8 && (!a->csq_min || !a->csq_step)) return fail(ctx, MAIVS_ERR_ARG, "csq_min/csq_step missing");
    if (a->rerank_mode == MAIVS_RERANK_F32 && !a->vecs_f32) return fail(ctx, MAIVS_ERR_ARG, "f32 rows missing");
    if (a->rerank_mode == MAIVS_RERANK_SQ8 && (!a->sq8_codes || !a->sq_min || !a->sq_step))
        return fail(ctx, MAIVS_ERR_ARG, "SQ8 rows missing");
    if (a->rerank_mode > MAIVS_RERANK_SQ8) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "rerank mode %u", a->rerank_mode);
    if (a->dim == 0 || a->dim > a->dim_pad || a->dim_pad > 4096 || (a->dim_pad & (a->dim_pad - 1)))
        return fail(ctx, MAIVS_ERR_UNSUPPORTED, "dim %u / dim_pad %u", a->dim, a->dim_pad);
    if (a->n_words * 64 > a->dim_pad) return fail(ctx, MAIVS_ERR_ARG, "n_words exceeds dim_pad");
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    free_all(ctx->work_allocs);
    free_all(ctx->cand_allocs);
    free_all(ctx->arena_allocs);
    ctx->cap_nq = ctx->cap_nprobe = ctx->cap_k = ctx->cap_cand = ctx->cap_seed = ctx->cand_nq = 0;
    ctx->uploaded = false;

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
    A.E = a->mem_off[A.M];
    A.fht_scale = 1.0f / std::sqrt(static_cast<float>(A.P));
    std::vector<uint8_t> live(A.M);
    uint32_t max_len = 0, n_live = 0;
    for (uint32_t c = 0; c < A.M; ++c) {
        uint32_t len = a->mem_off[c + 1] - a->mem_off[c];
        live[c] = len > 0;
        n_live += len > 0;
        max_len = std::max(max_len, len);
        if (a->fs_off[c + 1] - a->fs_off[c] != (len + 31) / 32)
            return fail(ctx, MAIVS_ERR_ARG, "fs_off does not match the member lists at cell %u", c);
    }
    A.n_live = n_live;
    A.max_cell_len = max_len;
    if (A.M * 2 > 96 * 1024) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "%u cells exceed the on-chip routing table", A.M);

    int rc = 0;
    uint8_t* fs = nullptr;
    uint32_t* fs_off = nullptr;
    uint32_t *codes = nullptr, *members = nullptr, *mem_off = nullptr, *slot_cells = nullptr;
    uint64_t* cent_bits = nullptr;
    uint8_t *cent_sq8 = nullptr, *sq8 = nullptr, *dlive = nullptr;
    float *cents = nullptr, *csq_min = nullptr, *csq_step = nullptr, *r_bound = nullptr, *signs = nullptr,
          *vecs = nullptr, *sq_min = nullptr, *sq_step = nullptr;
    const uint64_t nblocks = a->fs_off[A.M];
    rc |= dupload(ctx, a->fs_codes, nblocks * A.W * 256, &fs);
    rc |= dupload(ctx, a->fs_off, static_cast<uint64_t>(A.M) + 1, &fs_off);
    rc |= dalloc(ctx, ctx->arena_allocs, &codes, A.E * 2 * A.W);
    rc |= dupload(ctx, a->members, A.E, &members);
    rc |= dupload(ctx, a->mem_off, static_cast<uint64_t>(A.M) + 1, &mem_off);
    if (A.ma > 1) rc |= dupload(ctx, a->slot_cells, static_cast<uint64_t>(A.N) * A.ma, &slot_cells);
    rc |= dupload(ctx, a->cent_bits, static_cast<uint64_t>(A.M) * A.W, &cent_bits);
    if (a->cent_sq8) {
        rc |= dupload(ctx, a->cent_sq8, static_cast<uint64_t>(A.M) * A.d, &cent_sq8);
        rc |= dupload(ctx, a->csq_min, A.d, &csq_min);
        rc |= dupload(ctx, a->csq_step, A.d, &csq_step);
    } else {
        rc |= dupload(ctx, a->centroids, static_cast<uint64_t>(A.M) * A.d, &cents);
    }
    rc |= dupload(ctx, a->r_bound, A.M, &r_bound);
    rc |= dupload(ctx, a->rot_signs, 2ull * A.P, &signs);
    if (A.rerank_mode == MAIVS_RERANK_F32) {
        rc |= dupload(ctx, a->vecs_f32, static_cast<uint64_t>(A.N) * A.d, &vecs);
    } else {
        rc |= dupload(ctx, a->sq8_codes, static_cast<uint64_t>(A.N) * A.d, &sq8);
        rc |= dupload(ctx, a->sq_min, A.d, &sq_min);
        rc |= dupload(ctx, a->sq_step, A.d, &sq_step);
    }
    rc |= dupload(ctx, live.data(), A.M, &dlive);
    if (rc) {
        free_all(ctx->arena_allocs);
        return rc;
    }
    hipLaunchKernelGGL(fs_to_codes_kernel, dim3(std::max<uint32_t>(A.M, 1)), dim3(256), 0, ctx->stream, fs, fs_off,
                       mem_off, A.M, A.W, codes);
    HIP_TRY(ctx, hipGetLastError());
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    A.codes = codes;
    A.members = members;
    A.mem_off = mem_off;
    A.slot_cells = slot_cells;
    A.cent_bits = cent_bits;
    A.cent_sq8 = cent_sq8;
    A.centroids = cents;
    A.csq_min = csq_min;
    A.csq_step = csq_step;
    A.r_bound = r_bound;
    A.rot_signs = signs;
    A.vecs = vecs;
    A.sq8 = sq8;
    A.sq_min = sq_min;
    A.sq_step = sq_step;
    A.live = dlive;
    ctx->h_r_bound.assign(a->r_bound, a->r_bound + A.M);
    // LDS plan: route keeps hs[M] and the shortlist sort on chip (the sort size is per call)
    ctx->lds_route_fixed = route_lds(A, 0);
    size_t room = kLdsBudget - 4096 > ctx->lds_route_fixed ? (kLdsBudget - 4096 - ctx->lds_route_fixed) / 8 : 0;
    if (room < 1024) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "routing tables do not fit in LDS");
    uint32_t sc = 1024;
    while (static_cast<size_t>(sc) * 2 <= room && sc < 16384) sc <<= 1;
    ctx->max_sort_cap_route = sc;
    ctx->lds_seed = A.W * 256 + ((A.MW + 3) & ~3u) * 4 + kHistBins * 4 + 16 * 4 + kScanThreads * 4;
    ctx->lds_finish = kHistBins * 4 + 32 * 4 + ((A.d + 3) & ~3u) * 4 + static_cast<size_t>(kFinishSortCap) * 8;
    if (ctx->lds_finish > kLdsBudget || ctx->lds_seed > kLdsBudget)
        return fail(ctx, MAIVS_ERR_UNSUPPORTED, "LDS plan exceeds 160 KB");
    hipFuncSetAttribute(reinterpret_cast<const void*>(finish_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                        static_cast<int>(ctx->lds_finish));
    DISPATCH_NW(A.W, {
        hipFuncSetAttribute(reinterpret_cast<const void*>(prep_route_kernel<NW>), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(ctx->lds_route_fixed + static_cast<size_t>(sc) * 8));
        hipFuncSetAttribute(reinterpret_cast<const void*>(seed_kernel<NW>), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(ctx->lds_seed));
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

int maivs_gpu_search_batch(maivs_gpu_ctx* ctx, const float* q, uint32_t nq, const maivs_search_params* p,
                           uint32_t* out_slots, float* out_scores, maivs_gpu_stats* st) {
    if (!ctx || !p || (nq && (!q || !out_slots || !out_scores))) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (!ctx->uploaded) return fail(ctx, MAIVS_ERR_NOT_UPLOADED, "no arena uploaded");
    if (nq == 0) return 0;
    int rc = ensure_all(ctx, nq, p->nprobe, p->k);
    if (rc) return rc;
    HIP_TRY(ctx, hipMemcpyAsync(ctx->Wk.q, q, static_cast<size_t>(nq) * ctx->A.d * 4, hipMemcpyHostToDevice, ctx->stream));
    rc = run_search(ctx, ctx->Wk.q, nq, p, ctx->Wk.out_slots, ctx->Wk.out_scores, st);
    if (rc) return rc;
    HIP_TRY(ctx, hipMemcpyAsync(out_slots, ctx->Wk.out_slots, static_cast<size_t>(nq) * p->k * 4, hipMemcpyDeviceToHost,
                                ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(out_scores, ctx->Wk.out_scores, static_cast<size_t>(nq) * p->k * 4,
                                hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
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
    if ((rc = launch_route(ctx, K, ctx->Wk.q, 2))) return rc;
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
    Work& W = ctx->Wk;
    if (K.want_c == 0) {
        std::fill(out_chosen, out_chosen + static_cast<size_t>(nq) * p->nprobe, kNone);
        std::fill(out_cscore, out_cscore + static_cast<size_t>(nq) * p->nprobe, NAN);
        std::fill(out_nchosen, out_nchosen + nq, 0u);
        return 0;
    }
    HIP_TRY(ctx, hipMemcpyAsync(W.q, q, static_cast<size_t>(nq) * ctx->A.d * 4, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(ctx, hipMemsetAsync(W.ctl, 0, sizeof(Ctl), ctx->stream));
    if ((rc = launch_route(ctx, K, W.q, 1))) return rc;
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

int maivs_gpu_last_candidates(maivs_gpu_ctx* ctx, uint32_t* tau, uint32_t* rest_end, uint32_t* cut, uint32_t* ncand,
                              uint32_t* cand_slots, uint32_t* cand_d, uint64_t cap) {
    if (!ctx) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    const uint32_t nq = ctx->last_nq;
    if (nq == 0) return 0;
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
