// Wave-level pieces shared by the index build and the per-query search: LDS ordering inside a
// wave, Hamming distance, the keep_smallest selection (src/tree.rs:120-159) and the beam descent
// of the centroid tree (src/tree.rs:574-628), and the exact one-lane f32 dot.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "device_common.h"

namespace maivs_dev {

constexpr uint32_t kTreeHCache = 2048;  // frontier positions whose distance is kept in LDS per wave

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t hamming_lds(const uint64_t* qb, const uint64_t* code, uint32_t W) {
    uint32_t h = 0;
    for (uint32_t w = 0; w < W; ++w) h += __popcll(qb[w] ^ code[w]);
    return h;
}

// Total-order key of an f32 (ascending), for a first-minimum search.
__device__ __forceinline__ uint32_t asc_f32_key(float f) {
    const uint32_t b = __float_as_uint(f == 0.0f ? 0.0f : f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// t = the smallest distance with count(h <= t) >= keep and below = count(h < t), on every lane of
// the calling wave (keep at most the histogram's total). bits = 64 * W with W <= 16: lane l sums
// bins [l * W, (l + 1) * W) from registers (lane 63 also bin bits), one wave scan, and the lane
// whose run crosses keep walks its registers.
__device__ inline void wave_hist_threshold(const uint32_t* hist, uint32_t bits, uint32_t keep, uint32_t lane,
                                           uint32_t& t, uint32_t& below) {
    const uint32_t per = bits / kWave;
    uint32_t v[16], mine = 0;
#pragma unroll
    for (uint32_t j = 0; j < 16; ++j) {
        v[j] = j < per ? hist[lane * per + j] : 0u;
        mine += v[j];
    }
    mine += lane == kWave - 1 ? hist[bits] : 0u;
    const uint32_t incl = wave_incl_scan_u32(mine), excl = incl - mine;
    const bool here = excl < keep && incl >= keep;
    uint32_t b = bits, cum = excl;
    bool found = false;
#pragma unroll
    for (uint32_t j = 0; j < 16; ++j) {
        if (!found && j < per) {
            if (cum + v[j] >= keep) {
                b = lane * per + j;
                found = true;
            } else {
                cum += v[j];
            }
        }
    }
    // (not found among the registers: lane 63's bin bits, with cum counting all below it)
    const int src = __ffsll(static_cast<long long>(__ballot(here))) - 1;
    t = __shfl(b, src, kWave);
    below = __shfl(cum, src, kWave);
}

// keep_smallest over the frontier positions [0, F) with distance hd(p): emit(k, p) for the kept
// entries in encounter order (k = 0, 1, ...). Returns the number kept = min(keep, F).
// hcache (LDS, hcap entries): the distances of the first hcap positions, computed once.
template <class HD, class EMIT>
__device__ uint32_t wave_keep_smallest(uint32_t F, uint32_t keep, uint32_t bits, uint32_t* hist, HD hd, EMIT emit,
                                       uint16_t* hcache = nullptr, uint32_t hcap = 0) {
    const uint32_t lane = lane_id();
    if (keep >= F) {
        for (uint32_t p = lane; p < F; p += kWave) emit(p, p);
        return F;
    }
    for (uint32_t j = lane; j <= bits; j += kWave) hist[j] = 0;
    wave_sync();
    // four positions per lane at a time, so their code loads are in flight together
    for (uint32_t p0 = lane; p0 < F; p0 += 4 * kWave) {
        uint32_t hv[4];
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t p = p0 + u * kWave;
            hv[u] = p < F ? hd(p) : 0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t p = p0 + u * kWave;
            if (p < F) {
                atomicAdd(&hist[hv[u]], 1u);
                if (p < hcap) hcache[p] = static_cast<uint16_t>(hv[u]);
            }
        }
    }
    wave_sync();
    uint32_t t, below;
    wave_hist_threshold(hist, bits, keep, lane, t, below);
    const uint32_t need_eq = keep - below;
    uint32_t eq_seen = 0, kept = 0;
    for (uint32_t c0 = 0; c0 < F; c0 += kWave) {
        const uint32_t p = c0 + lane;
        const bool valid = p < F;
        const uint32_t h = valid ? (p < hcap ? static_cast<uint32_t>(hcache[p]) : hd(p)) : 0xFFFFFFFFu;
        const uint64_t eqm = __ballot(valid && h == t);
        const bool take = valid && (h < t || (h == t && eq_seen + lanes_below(eqm) < need_eq));
        const uint64_t tm = __ballot(take);
        if (take) emit(kept + lanes_below(tm), p);
        eq_seen += __popcll(eqm);
        kept += __popcll(tm);
    }
    return kept;
}

// Frontier position p -> node id, from the ranges of the kept parents (rpre: prefix of lengths).
__device__ __forceinline__ uint32_t frontier_node(const uint32_t* rbase, const uint32_t* rpre, uint32_t nr, uint32_t p) {
    uint32_t lo = 0, hi = nr;  // the last r with rpre[r] <= p
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (rpre[mid] <= p) lo = mid; else hi = mid;
    }
    return rbase[lo] + (p - rpre[lo]);
}

// Exact dot_f32(a, b) by one lane: 8 accumulators, hsum, sequential tail (src/index.rs:136-152).
template <class LA, class LB>
__device__ __forceinline__ float dot_lane(uint32_t d, LA la, LB lb) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const uint32_t d8 = d & ~7u;
    for (uint32_t t = 0; t < d8; t += 8) {
#pragma unroll
        for (uint32_t l = 0; l < 8; ++l) acc[l] = __builtin_fmaf(la(t + l), lb(t + l), acc[l]);
    }
    float s = ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
    for (uint32_t e = d8; e < d; ++e) s += la(e) * lb(e);
    return s;
}

// The centroid tree in HBM, compacted layout: node j of level l has the children
// [cs[j], cs[j] + cl[j]) of level l + 1 (the leaves after the last level).
struct TreeDev {
    const uint32_t* lv_off;      // n_levels + 1 node offsets, coarsest level first
    const uint64_t* lv_codes;    // sum of level sizes x W
    const uint32_t* lv_cs;
    const uint32_t* lv_cl;
    const uint64_t* leaf_codes;  // n_leaf x W
    const uint32_t* leaf_ids;    // n_leaf: the cell of each leaf
    uint32_t n_levels, n_leaf;
};

// One wave: the beam descent for the code qb (LDS, W words) keeping beams[l] nodes per level and
// `want` leaves, ties in encounter order. Writes the leaves' cells, best first by Hamming, to out
// and returns their number (0: the caller scores every cell, as the reference does on an empty
// result). Per-wave LDS scratch: hist[W*64 + 1], rbase[cap + 1], rpre[cap + 2], knodes[cap] with
// cap >= every beam; out[want]; hcache[hcap] u16 (distances kept between the two passes).
__device__ inline uint32_t tree_descent(const TreeDev& T, const uint32_t* beams, uint32_t want, const uint64_t* qb, uint32_t W,
                                        uint32_t* hist, uint32_t* rbase, uint32_t* rpre, uint32_t* knodes, uint32_t* out,
                                        uint16_t* hcache, uint32_t hcap) {
    const uint32_t lane = lane_id(), bits = W * 64;
    if (T.n_levels == 0) return 0;
    uint32_t nr = 1;
    if (lane == 0) {
        rbase[0] = 0;
        rpre[0] = 0;
        rpre[1] = T.lv_off[1] - T.lv_off[0];
    }
    wave_sync();
    uint32_t F = T.lv_off[1] - T.lv_off[0];
    for (uint32_t li = 0; li < T.n_levels; ++li) {
        const uint64_t* codes = T.lv_codes + static_cast<uint64_t>(T.lv_off[li]) * W;
        const uint32_t keep = min(beams[li], F);
        if (keep == 0) return 0;
        const uint32_t nk = wave_keep_smallest(
            F, keep, bits, hist,
            [&](uint32_t p) {
                const uint32_t node = frontier_node(rbase, rpre, nr, p);
                return hamming_lds(qb, codes + static_cast<uint64_t>(node) * W, W);
            },
            [&](uint32_t k, uint32_t p) { knodes[k] = frontier_node(rbase, rpre, nr, p); }, hcache, hcap);
        wave_sync();
        // children of the kept nodes, in order: the next frontier's ranges
        const uint32_t* cs = T.lv_cs + T.lv_off[li];
        const uint32_t* cl = T.lv_cl + T.lv_off[li];
        uint32_t carry = 0;
        for (uint32_t k0 = 0; k0 < nk; k0 += kWave) {
            const uint32_t k = k0 + lane;
            const uint32_t node = k < nk ? knodes[k] : 0u;
            const uint32_t len = k < nk ? cl[node] : 0u;
            uint32_t incl = wave_incl_scan_u32(len);
            if (k < nk) {
                rbase[k] = cs[node];
                rpre[k] = carry + incl - len;
            }
            carry += __shfl(incl, kWave - 1, kWave);
        }
        if (lane == 0) rpre[nk] = carry;
        wave_sync();
        nr = nk;
        F = carry;
    }
    const uint32_t keep = min(want, F);
    if (keep == 0) return 0;
    const uint32_t nout = wave_keep_smallest(
        F, keep, bits, hist,
        [&](uint32_t p) {
            const uint32_t leaf = frontier_node(rbase, rpre, nr, p);
            return hamming_lds(qb, T.leaf_codes + static_cast<uint64_t>(leaf) * W, W);
        },
        [&](uint32_t k, uint32_t p) { out[k] = T.leaf_ids[frontier_node(rbase, rpre, nr, p)]; }, hcache, hcap);
    wave_sync();
    return nout;
}

// wave_keep_smallest by the whole workgroup (every thread calls it; blockDim.x a multiple of 64, at
// most 1024): the same kept entries, emitted with the same ranks k. hist: bits + 1 counters;
// scratch: 18 words (block scans, then the threshold and its count below).
template <class HD, class EMIT>
__device__ uint32_t block_keep_smallest(uint32_t F, uint32_t keep, uint32_t bits, uint32_t* hist, uint32_t* scratch,
                                        HD hd, EMIT emit, uint16_t* hcache, uint32_t hcap) {
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    if (keep >= F) {
        for (uint32_t p = tid; p < F; p += nt) emit(p, p);
        return F;
    }
    for (uint32_t j = tid; j <= bits; j += nt) hist[j] = 0;
    __syncthreads();
    for (uint32_t p0 = tid; p0 < F; p0 += 4 * nt) {
        uint32_t hv[4];
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t p = p0 + u * nt;
            hv[u] = p < F ? hd(p) : 0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t p = p0 + u * nt;
            if (p < F) {
                atomicAdd(&hist[hv[u]], 1u);
                if (p < hcap) hcache[p] = static_cast<uint16_t>(hv[u]);
            }
        }
    }
    __syncthreads();
    // t = the smallest distance with count(h <= t) >= keep; below = count(h < t): wave 0 alone
    if (tid < kWave) {
        uint32_t t, below;
        wave_hist_threshold(hist, bits, keep, tid, t, below);
        if (tid == 0) {
            scratch[16] = t;
            scratch[17] = below;
        }
    }
    __syncthreads();
    const uint32_t t = scratch[16], below = scratch[17];
    const uint32_t need_eq = keep - below;
    // encounter order: thread tid takes positions [tid * PPT, (tid + 1) * PPT) of each chunk of
    // nt * PPT (PPT by the frontier's size), and one scan counts both the entries below t (low half)
    // and those at t (high half) before its run; the run then walks its positions in order
    uint32_t eq_seen = 0, kept = 0;
    auto emit_runs = [&](auto ppt_tag) {
        constexpr uint32_t PPT = decltype(ppt_tag)::value;
        for (uint32_t c0 = 0; c0 < F; c0 += nt * PPT) {
            uint32_t hv[PPT], cnt = 0;
#pragma unroll
            for (uint32_t i = 0; i < PPT; ++i) {
                const uint32_t p = c0 + tid * PPT + i;
                hv[i] = p < F ? (p < hcap ? static_cast<uint32_t>(hcache[p]) : hd(p)) : 0xFFFFFFFFu;
                cnt += hv[i] < t ? 1u : hv[i] == t ? 0x10000u : 0u;
            }
            uint32_t tot;
            const uint32_t ex = block_excl_scan_u32(cnt, scratch, &tot);
            const uint32_t rem = need_eq > eq_seen ? need_eq - eq_seen : 0u;
            uint32_t lt_before = ex & 0xFFFFu, eq_before = ex >> 16;
#pragma unroll
            for (uint32_t i = 0; i < PPT; ++i) {
                const uint32_t p = c0 + tid * PPT + i;
                if (hv[i] < t) {
                    emit(kept + lt_before + min(eq_before, rem), p);
                    ++lt_before;
                } else if (hv[i] == t) {
                    if (eq_before < rem) emit(kept + lt_before + eq_before, p);
                    ++eq_before;
                }
            }
            kept += (tot & 0xFFFFu) + min(tot >> 16, rem);
            eq_seen += tot >> 16;
        }
    };
    if (F <= nt)
        emit_runs(std::integral_constant<uint32_t, 1>{});
    else if (F <= 2 * nt)
        emit_runs(std::integral_constant<uint32_t, 2>{});
    else
        emit_runs(std::integral_constant<uint32_t, 4>{});
    return kept;
}

// tree_descent by the whole workgroup (every thread calls it): the same leaves in the same order.
// LDS as tree_descent's, plus scratch (18 words), fr and fid (fcap words each: the frontier's nodes
// below the top level, and the leaves' cells, so neither needs a search or a second load), and
// top (top_cs, top_cl): the top level's codes (child ranges) when the caller staged them in LDS
// (else null); out_lds: an LDS copy of out (want words), or null.
__device__ inline uint32_t block_tree_descent(const TreeDev& T, const uint32_t* beams, uint32_t want, const uint64_t* qb,
                                              uint32_t W, uint32_t* hist, uint32_t* rbase, uint32_t* rpre,
                                              uint32_t* knodes, uint32_t* out, uint16_t* hcache, uint32_t hcap,
                                              uint32_t* scratch, uint32_t* fr, uint32_t* fid, uint32_t fcap,
                                              const uint64_t* top, const uint32_t* top_cs = nullptr,
                                              const uint32_t* top_cl = nullptr, uint32_t* out_lds = nullptr) {
    const uint32_t tid = threadIdx.x, nt = blockDim.x, bits = W * 64;
    if (T.n_levels == 0) return 0;
    uint32_t nr = 1;
    if (tid == 0) {
        rbase[0] = 0;
        rpre[0] = 0;
        rpre[1] = T.lv_off[1] - T.lv_off[0];
    }
    __syncthreads();
    uint32_t F = T.lv_off[1] - T.lv_off[0];
    // the node at frontier position p: p itself on the top level, else fr[p] (or the search past fcap)
    auto node_of = [&](uint32_t li, uint32_t p) {
        return li == 0 ? p : p < fcap ? fr[p] : frontier_node(rbase, rpre, nr, p);
    };
    for (uint32_t li = 0; li < T.n_levels; ++li) {
        const uint64_t* codes = li == 0 && top ? top : T.lv_codes + static_cast<uint64_t>(T.lv_off[li]) * W;
        const uint32_t keep = min(beams[li], F);
        if (keep == 0) return 0;
        const uint32_t nk = block_keep_smallest(
            F, keep, bits, hist, scratch,
            [&](uint32_t p) { return hamming_lds(qb, codes + static_cast<uint64_t>(node_of(li, p)) * W, W); },
            [&](uint32_t k, uint32_t p) { knodes[k] = node_of(li, p); }, hcache, hcap);
        __syncthreads();
        // children of the kept nodes, in order: the next frontier's ranges, then its nodes
        const uint32_t* cs = li == 0 && top_cs ? top_cs : T.lv_cs + T.lv_off[li];
        const uint32_t* cl = li == 0 && top_cl ? top_cl : T.lv_cl + T.lv_off[li];
        uint32_t carry = 0;
        for (uint32_t k0 = 0; k0 < nk; k0 += nt) {
            const uint32_t k = k0 + tid;
            const uint32_t node = k < nk ? knodes[k] : 0u;
            const uint32_t len = k < nk ? cl[node] : 0u;
            uint32_t tot;
            const uint32_t ex = block_excl_scan_u32(len, scratch, &tot);
            if (k < nk) {
                rbase[k] = cs[node];
                rpre[k] = carry + ex;
            }
            carry += tot;
        }
        if (tid == 0) rpre[nk] = carry;
        __syncthreads();
        // eight threads per kept node, every eighth child each
        for (uint32_t x = tid; x < nk * 8; x += nt) {
            const uint32_t k = x >> 3, b = rbase[k], p0 = rpre[k], len = rpre[k + 1] - p0;
            for (uint32_t j = x & 7; j < len && p0 + j < fcap; j += 8) fr[p0 + j] = b + j;
        }
        __syncthreads();
        nr = nk;
        F = carry;
    }
    const uint32_t keep = min(want, F);
    if (keep == 0) return 0;
    const uint32_t ll = T.n_levels;  // the leaves: frontier nodes are leaf indices
    const bool every = keep >= F;     // kept without a distance pass: fid is not filled
    const uint32_t nout = block_keep_smallest(
        F, keep, bits, hist, scratch,
        [&](uint32_t p) {
            const uint32_t leaf = node_of(ll, p);
            if (p < fcap) fid[p] = T.leaf_ids[leaf];
            return hamming_lds(qb, T.leaf_codes + static_cast<uint64_t>(leaf) * W, W);
        },
        [&](uint32_t k, uint32_t p) {
            const uint32_t c = !every && p < fcap ? fid[p] : T.leaf_ids[node_of(ll, p)];
            out[k] = c;
            if (out_lds) out_lds[k] = c;
        },
        hcache, hcap);
    __syncthreads();
    return nout;
}

// beams of the descent (src/tree.rs:559-570): from the finest level up, clamp(ceil(need * frac),
// min_beam, level size), need starting at max(want, 1).
__host__ inline void tree_beams(const uint32_t* level_n, uint32_t n_levels, float frac, uint32_t min_beam, uint32_t want,
                                uint32_t* out) {
    uint32_t need = want > 0 ? want : 1;
    for (uint32_t i = n_levels; i-- > 0;) {
        const float raw = static_cast<float>(need) * frac;
        uint32_t b = static_cast<uint32_t>(__builtin_ceilf(raw));
        b = b > min_beam ? b : min_beam;
        b = b < level_n[i] ? b : level_n[i];
        out[i] = b;
        need = b;
    }
}

}  // namespace maivs_dev
