// Device kernels of libmaivs_gpu.so (included by maivs_gpu.hip). They restate MAIVS's batched
// cell-major search (src/index.rs:1873-2311, 1309-1378; src/quantize.rs:57-386) for gfx950.
//
// Compiled with -ffp-contract=off: every FMA below is an explicit __builtin_fmaf standing for one
// of the reference's _mm256_fmadd_ps; every other f32 operation rounds once, in the reference's
// order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../../include/maivs_gpu.h"
#include "device_common.h"

namespace maivs_dev {

constexpr uint32_t kSeedCells = 8;       // SEED_CELLS, src/index.rs:2018
constexpr uint32_t kRouteThreads = 256;
constexpr uint32_t kSeedThreads = 1024;
constexpr uint32_t kScanThreads = 256;
constexpr uint32_t kFinishThreads = 512;
constexpr uint32_t kG = 4;               // queries interleaved per cell_scan table pass
constexpr uint32_t kHistBins = 256;
constexpr uint32_t kFinishLdsCap = 2048; // final candidates kept and sorted in LDS up to this many
constexpr uint32_t kNoAlt = 0xFFFFFFFEu; // entry_alt: the slot has no other home

// Chain-major row layout for the 8-lane FMA dots: element 8t + l (t < T) of a row is stored at
// l*Tp + t, the d - 8T tail elements at 8*Tp + i. Lane l of a group of 8 then reads its whole
// accumulation chain with wide loads, in the reference's order.
struct Chain {
    uint32_t T, Tp, tail, stride;
};

struct DevArena {
    uint32_t d, P, W, M, N, ma, rerank_mode, npos, maxk, n_live, max_cell_len, MW;
    uint64_t E;
    float fht_scale;
    Chain cf, cu;               // f32 and u8 chain layouts
    const uint32_t* codes;      // E x 2W dwords, entry-major 1-bit codes in member order
    const uint32_t* members;    // E slots
    const uint32_t* entry_alt;  // E: the entry's other home (max_assign == 2), kNoAlt if none
    const uint32_t* mem_off;    // M + 1
    const uint32_t* slot_cells; // N x ma
    const uint64_t* cent_bits;  // M x W
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
    const uint8_t* live;        // M
};

struct Ctl {
    uint32_t nflag_route;
    uint32_t nflag_prune;
    uint32_t max_cand;        // largest candidate count past the buffer capacity (0 = none)
    uint32_t err_shortlist;   // a shortlist exceeded the sort capacity
    uint32_t max_shortlist;
    uint32_t err_seed;        // a seed set exceeded its on-chip capacity
    uint32_t pad[2];
    unsigned long long seed_blocks, scan_blocks, scan_pairs, survivors, rerank_rows;
};

struct Work {
    float* q;              // nq x d (host-input calls)
    uint64_t* qbits;       // nq x W
    uint8_t* lut;          // nq x npos*16
    float* delta;          // nq
    float* bias;           // nq
    uint32_t* chosen;      // nq x nprobe
    float* cscore;         // nq x nprobe
    uint32_t* nchosen;     // nq
    uint32_t* probed;      // nq x MW
    uint2* seed;           // nq x seed_cap (d, slot): seed members with d <= tau
    uint32_t* seed_cnt;    // nq
    uint32_t* tau;         // nq
    uint32_t* rest_end;    // nq
    uint32_t* qstat;       // nq x 3: seed blocks, scan blocks, scan pairs
    uint2* cand;           // nq x cand_cap
    uint32_t* cand_cnt;    // nq
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
    uint32_t* flag_route;  // nq
    uint32_t* flag_prune;  // nq
    Ctl* ctl;
};

struct KParams {
    uint32_t nq, k, nprobe, want_c, target, adaptive, sort_cap, use_nucleus;
    uint32_t seed_cap, cand_cap, fin_cap, key_cap;
    float tc, beta, at_margin, norm, prune_band, nucleus_band;
};

// ---------------------------------------------------------------- small pieces

// f32 acos / cos / exp evaluated in f64 and rounded once. glibc's acosf / cosf / expf (what the
// reference's f32::acos / cos / exp call) are not correctly rounded, so a decision that lands
// within a small band of its threshold is flagged and re-evaluated on the host with libm.
__device__ __forceinline__ float acos_f(float x) { return static_cast<float>(acos(static_cast<double>(x))); }
__device__ __forceinline__ float cos_f(float x) { return static_cast<float>(cos(static_cast<double>(x))); }
__device__ __forceinline__ float exp_f(float x) { return static_cast<float>(exp(static_cast<double>(x))); }

// Sequential f32 sum of n LDS values in index order, starting from `init` (one thread).
__device__ __forceinline__ float seq_sum_lds(const float* v, uint32_t n, float init) {
    float s = init;
    uint32_t i = 0;
    for (; i + 16 <= n; i += 16) {
        float4 a = reinterpret_cast<const float4*>(v + i)[0];
        float4 b = reinterpret_cast<const float4*>(v + i)[1];
        float4 c = reinterpret_cast<const float4*>(v + i)[2];
        float4 e = reinterpret_cast<const float4*>(v + i)[3];
        s += a.x; s += a.y; s += a.z; s += a.w;
        s += b.x; s += b.y; s += b.z; s += b.w;
        s += c.x; s += c.y; s += c.z; s += c.w;
        s += e.x; s += e.y; s += e.z; s += e.w;
    }
    for (; i < n; ++i) s += v[i];
    return s;
}

// One group of 8 lanes computes one chain-major f32 row's dot with q(j): lane l owns the chain
// acc_l = fma(q(8t+l), row(8t+l), acc_l) over t ascending; then the hsum order
// ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)); then the tail sequentially (src/index.rs:136-152).
template <class QF>
__device__ __forceinline__ float dot_cm_f32(const float* __restrict__ row, const Chain& C, uint32_t l, QF q) {
    const float* p = row + l * C.Tp;
    float acc = 0.0f;
    uint32_t t = 0;
    for (; t + 48 <= C.T; t += 48) {
        float4 v[12];
#pragma unroll
        for (int i = 0; i < 12; ++i) v[i] = reinterpret_cast<const float4*>(p + t)[i];
#pragma unroll
        for (int i = 0; i < 12; ++i) {
            const uint32_t b = t + 4 * i;
            acc = __builtin_fmaf(q(8 * b + l), v[i].x, acc);
            acc = __builtin_fmaf(q(8 * (b + 1) + l), v[i].y, acc);
            acc = __builtin_fmaf(q(8 * (b + 2) + l), v[i].z, acc);
            acc = __builtin_fmaf(q(8 * (b + 3) + l), v[i].w, acc);
        }
    }
    for (; t + 4 <= C.T; t += 4) {
        float4 v = *reinterpret_cast<const float4*>(p + t);
        acc = __builtin_fmaf(q(8 * t + l), v.x, acc);
        acc = __builtin_fmaf(q(8 * (t + 1) + l), v.y, acc);
        acc = __builtin_fmaf(q(8 * (t + 2) + l), v.z, acc);
        acc = __builtin_fmaf(q(8 * (t + 3) + l), v.w, acc);
    }
    for (; t < C.T; ++t) acc = __builtin_fmaf(q(8 * t + l), p[t], acc);
    float s = acc + __shfl_xor(acc, 4, 8);
    float s2 = __shfl_xor(s, 2, 8);
    float u = s + s2;
    float r = u + __shfl_xor(u, 1, 8);
    const float* tp = row + 8 * C.Tp;
    for (uint32_t i = 0; i < C.tail; ++i) r += q(8 * C.T + i) * tp[i];
    return r;
}

// Same for a chain-major u8 row (dot_f32_u8, src/index.rs:278-294): fma(qs, float(u8), acc).
template <class QF>
__device__ __forceinline__ float dot_cm_u8(const uint8_t* __restrict__ row, const Chain& C, uint32_t l, QF q) {
    const uint8_t* p = row + l * C.Tp;
    float acc = 0.0f;
    uint32_t t = 0;
    for (; t + 48 <= C.T; t += 48) {
        uint4 v[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) v[i] = reinterpret_cast<const uint4*>(p + t)[i];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t b = t + 16 * i + j;
                acc = __builtin_fmaf(q(8 * b + l), static_cast<float>((w[j >> 2] >> (8 * (j & 3))) & 0xFFu), acc);
            }
        }
    }
    for (; t + 16 <= C.T; t += 16) {
        uint4 v = *reinterpret_cast<const uint4*>(p + t);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 16; ++j)
            acc = __builtin_fmaf(q(8 * (t + j) + l), static_cast<float>((w[j >> 2] >> (8 * (j & 3))) & 0xFFu), acc);
    }
    for (; t < C.T; ++t) acc = __builtin_fmaf(q(8 * t + l), static_cast<float>(p[t]), acc);
    float s = acc + __shfl_xor(acc, 4, 8);
    float s2 = __shfl_xor(s, 2, 8);
    float u = s + s2;
    float r = u + __shfl_xor(u, 1, 8);
    const uint8_t* tp = row + 8 * C.Tp;
    for (uint32_t i = 0; i < C.tail; ++i) r += q(8 * C.T + i) * static_cast<float>(tp[i]);
    return r;
}

// Ascending bitonic sort of 64*KPL keys held in one wave: element i = r*64 + lane sits in k[r].
template <int KPL>
__device__ __forceinline__ void wave_sort_u64(uint64_t (&k)[KPL]) {
    constexpr uint32_t N = 64u * KPL;
    const uint32_t lane = lane_id();
#pragma unroll
    for (uint32_t size = 2; size <= N; size <<= 1) {
#pragma unroll
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            if (stride >= 64) {
                const uint32_t rs = stride / 64;
#pragma unroll
                for (int r = 0; r < KPL; ++r) {
                    if ((static_cast<uint32_t>(r) & rs) == 0) {
                        const int r2 = r | static_cast<int>(rs);
                        const bool up = ((static_cast<uint32_t>(r) * 64 + lane) & size) == 0;
                        uint64_t a = k[r], b = k[r2];
                        uint64_t mn = a < b ? a : b, mx = a < b ? b : a;
                        k[r] = up ? mn : mx;
                        k[r2] = up ? mx : mn;
                    }
                }
            } else {
#pragma unroll
                for (int r = 0; r < KPL; ++r) {
                    const uint32_t i = static_cast<uint32_t>(r) * 64 + lane;
                    const bool up = (i & size) == 0;
                    const bool lower = (lane & stride) == 0;
                    uint64_t a = k[r];
                    uint64_t b = __shfl_xor(a, static_cast<int>(stride), 64);
                    uint64_t mn = a < b ? a : b, mx = a < b ? b : a;
                    k[r] = (lower == up) ? mn : mx;
                }
            }
        }
    }
}

// Sort n <= 256 keys from `src` (padded with max keys) in wave 0 and write the first `out_n`
// ascending keys to `dst` (both may alias). Other waves only wait at the caller's barrier.
__device__ __forceinline__ void wave0_sort_prefix(const uint64_t* src, uint32_t n, uint64_t* dst, uint32_t out_n) {
    if (threadIdx.x >= 64) return;
    const uint32_t lane = lane_id();
    auto run = [&](auto kpl_tag) {
        constexpr int KPL = decltype(kpl_tag)::value;
        uint64_t k[KPL];
#pragma unroll
        for (int r = 0; r < KPL; ++r) {
            uint32_t i = static_cast<uint32_t>(r) * 64 + lane;
            k[r] = i < n ? src[i] : kKeyMax;
        }
        wave_sort_u64<KPL>(k);
#pragma unroll
        for (int r = 0; r < KPL; ++r) {
            uint32_t i = static_cast<uint32_t>(r) * 64 + lane;
            if (i < out_n) dst[i] = k[r];
        }
    };
    if (n <= 64)
        run(std::integral_constant<int, 1>{});
    else if (n <= 128)
        run(std::integral_constant<int, 2>{});
    else
        run(std::integral_constant<int, 4>{});
}

// One member's nibble sums against a FastScan table of G interleaved queries in LDS (table byte
// [(j*16 + e)*G + g] = query g's entry e of position j). The member's code (2*NW dwords, nibble j
// at dword j/8, bits 4*(j%8)) is loaded whole before the lookups so its latency is paid once.
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

template <int NW>
struct Code {
    static constexpr int NCH = NW >= 2 ? NW / 2 : 1;  // 16-byte chunks (NW = 1: one 8-byte chunk)
    uint4 v[NCH];
    __device__ __forceinline__ void load(const uint32_t* __restrict__ code) {
        if constexpr (NW == 1) {
            uint2 x = *reinterpret_cast<const uint2*>(code);
            v[0] = make_uint4(x.x, x.y, 0u, 0u);
        } else {
#pragma unroll
            for (int k = 0; k < NCH; ++k) v[k] = reinterpret_cast<const uint4*>(code)[k];
        }
    }
};

template <int NW, int G>
__device__ __forceinline__ void lut_sums(const Code<NW>& c, const uint8_t* table, uint32_t (&sum)[G]) {
    static_assert(G == 1 || G == 4, "G is 1 or 4");
    // S accumulates table words; for G = 4 it is b0 + 256 b1 + 65536 b2 + 2^24 b3 (mod 2^32) and T
    // the odd bytes as u16 lanes (b1 + 65536 b3). Every per-query sum is at most 255 * 16 * NW
    // < 65536, so both un-mix exactly at the end.
    uint32_t S = 0, T = 0;
    if constexpr (NW == 1) {
        lut_chunk<G>(c.v[0].x, c.v[0].y, 0u, 0u, 16, table, S, T);
    } else {
        uint4 v[Code<NW>::NCH];
#pragma unroll
        for (int k = 0; k < Code<NW>::NCH; ++k) v[k] = c.v[k];
#pragma unroll 1
        for (int k = 0; k < Code<NW>::NCH; ++k) {
            lut_chunk<G>(v[0].x, v[0].y, v[0].z, v[0].w, 32, table + static_cast<uint32_t>(k) * 32 * 16 * G, S, T);
#pragma unroll
            for (int r = 0; r + 1 < Code<NW>::NCH; ++r) v[r] = v[r + 1];  // rotate: chunk k+1 to the front
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
// slot was probed by the query. With two homes the other home is precomputed per entry.
__device__ __forceinline__ bool canonical(const DevArena& A, uint64_t e, uint32_t slot, uint32_t c,
                                          const uint32_t* probed) {
    if (A.ma <= 1) return true;
    if (A.ma == 2) {
        const uint32_t h = A.entry_alt[e];
        return !(h < c && ((probed[h >> 5] >> (h & 31)) & 1u));
    }
    const uint32_t* hs = A.slot_cells + static_cast<uint64_t>(slot) * A.ma;
    for (uint32_t j = 0; j < A.ma; ++j) {
        uint32_t hc = hs[j];
        if (hc != kNone && hc < c && ((probed[hc >> 5] >> (hc & 31)) & 1u)) return false;
    }
    return true;
}

// Exact `want`-th smallest (1-based) of n values d < 65536 from get(i). Two 256-bin LDS histogram
// passes; every thread returns the value. Block-uniform call.
template <class Get>
__device__ uint32_t select_kth(uint32_t n, uint32_t want, Get get, uint32_t* hist, uint32_t* scratch) {
    for (uint32_t i = threadIdx.x; i < kHistBins; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) atomicAdd(&hist[get(i) >> 8], 1u);
    __syncthreads();
    uint32_t hb, below;
    {
        uint32_t v = threadIdx.x < kHistBins ? hist[threadIdx.x] : 0u;
        uint32_t total;
        uint32_t ex = block_excl_scan_u32(v, scratch, &total);
        uint32_t cand = (threadIdx.x < kHistBins && ex < want && ex + v >= want) ? threadIdx.x : kNone;
        hb = block_min_u32(cand, scratch);
        below = block_sum_u32(threadIdx.x == hb ? ex : 0u, scratch);
    }
    for (uint32_t i = threadIdx.x; i < kHistBins; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        uint32_t d = get(i);
        if ((d >> 8) == hb) atomicAdd(&hist[d & 0xFFu], 1u);
    }
    __syncthreads();
    const uint32_t need = want - below;
    uint32_t v = threadIdx.x < kHistBins ? hist[threadIdx.x] : 0u;
    uint32_t total;
    uint32_t ex = block_excl_scan_u32(v, scratch, &total);
    uint32_t cand = (threadIdx.x < kHistBins && ex < need && ex + v >= need) ? threadIdx.x : kNone;
    uint32_t lb = block_min_u32(cand, scratch);
    return (hb << 8) | lb;
}

// ---------------------------------------------------------------- upload-time layout kernels

// Entry-major codes from FastScan blocks: entry i of cell c lives in block fs_off[c] + i/32, lane
// i%32; nibble j is byte [(j/2)*32 + (j%2)*16 + lane%16], low half for lanes < 16
// (src/quantize.rs:238-265).
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

// The other home of every entry (two homes per slot).
__global__ void entry_alt_kernel(const uint32_t* __restrict__ mem_off, const uint32_t* __restrict__ members,
                                 const uint32_t* __restrict__ slot_cells, uint32_t M, uint32_t* __restrict__ alt) {
    uint32_t c = blockIdx.x;
    if (c >= M) return;
    uint32_t e0 = mem_off[c], len = mem_off[c + 1] - e0;
    for (uint32_t i = threadIdx.x; i < len; i += blockDim.x) {
        uint32_t s = members[e0 + i];
        uint32_t h0 = slot_cells[2ull * s], h1 = slot_cells[2ull * s + 1];
        uint32_t o = h0 == c ? h1 : h0;
        alt[e0 + i] = o == kNone ? kNoAlt : o;
    }
}

// Row-major -> chain-major (see Chain). One block per row.
template <class T>
__global__ void to_chain_kernel(const T* __restrict__ src, uint64_t rows, uint32_t d, Chain C, T* __restrict__ dst) {
    for (uint64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const T* s = src + r * d;
        T* o = dst + r * C.stride;
        for (uint32_t i = threadIdx.x; i < C.stride; i += blockDim.x) {
            T v = T(0);
            if (i < 8 * C.Tp) {
                uint32_t l = i / C.Tp, t = i % C.Tp;
                if (t < C.T) v = s[8 * t + l];
            } else {
                uint32_t k = i - 8 * C.Tp;
                if (k < C.tail) v = s[8 * C.T + k];
            }
            o[i] = v;
        }
    }
}

// Test entry point: nibble sums of entry-major codes (32 per block) against per-block tables.
template <int NW>
__global__ void entry_sums_kernel(const uint32_t* __restrict__ codes, const uint8_t* __restrict__ luts,
                                  uint32_t n_entries, uint16_t* __restrict__ out) {
    extern __shared__ uint8_t smem[];
    constexpr uint32_t TB = NW * 256;
    uint32_t b = blockIdx.x;
    for (uint32_t i = threadIdx.x; i < TB; i += blockDim.x) smem[i] = luts[static_cast<uint64_t>(b) * TB + i];
    __syncthreads();
    uint32_t e = b * 32 + threadIdx.x;
    if (threadIdx.x < 32 && e < n_entries) {
        Code<NW> c;
        c.load(codes + static_cast<uint64_t>(e) * (2 * NW));
        uint32_t s[1];
        lut_sums<NW, 1>(c, smem, s);
        out[e] = static_cast<uint16_t>(s[0]);
    }
}

// Zero the per-call counters: control block, cell counts, candidate counts.
__global__ void reset_kernel(Work Wk, uint32_t M, uint32_t nq) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x, stride = gridDim.x * blockDim.x;
    if (i < sizeof(Ctl) / 4) reinterpret_cast<uint32_t*>(Wk.ctl)[i] = 0;
    for (uint32_t j = i; j <= M; j += stride) Wk.cell_cnt[j] = 0;
    for (uint32_t j = i; j < nq; j += stride) Wk.cand_cnt[j] = 0;
}

// ---------------------------------------------------------------- prep + route (one WG per query)

template <int NW>
__global__ void __launch_bounds__(kRouteThreads)
prep_route_kernel(DevArena A, Work Wk, KParams K, const float* __restrict__ queries, uint32_t mode) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t qi = blockIdx.x;
    if (qi >= K.nq) return;
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    const uint32_t d = A.d, P = A.P, M = A.M, npos = A.npos;
    constexpr uint32_t W = NW;
    const uint32_t d4 = (d + 3) & ~3u;
    float* x = reinterpret_cast<float*>(smem);
    float* cqs = x + P;
    float* cqp = cqs + d4;
    uint16_t* hs = reinterpret_cast<uint16_t*>(cqp + d4);
    uint64_t* keys = reinterpret_cast<uint64_t*>(hs + ((M + 7) & ~7u));
    float* mins = reinterpret_cast<float*>(keys + K.sort_cap);
    uint32_t* hist = reinterpret_cast<uint32_t*>(mins + ((npos + 3) & ~3u));
    const uint32_t nbins = W * 64 + 1;
    uint32_t* scratch = hist + ((nbins + 3) & ~3u);
    __shared__ float s_cqbase;
    __shared__ uint32_t s_cut, s_nsl;
    __shared__ uint64_t s_qw[16];

    const float* q = queries + static_cast<uint64_t>(qi) * d;
    const bool sq8 = A.cent_sq8 != nullptr;
    // ---- load: query, and the SQ8 rescore operands cqs = q*step, q*min (src/index.rs:1934-1942)
    for (uint32_t i = tid; i < P; i += nt) {
        float v = i < d ? q[i] : 0.0f;
        x[i] = v;
        if (i < d) {
            cqs[i] = sq8 ? v * A.csq_step[i] : v;
            cqp[i] = sq8 ? v * A.csq_min[i] : 0.0f;
        }
    }
    // ---- rotation: 2 x (sign flip, FWHT, x 1/sqrt(P)), src/quantize.rs:152-163
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
    // ---- 1-bit code: bit i = x[i] < 0 (src/quantize.rs:57-67)
    uint64_t* qb_out = Wk.qbits + static_cast<uint64_t>(qi) * W;
    for (uint32_t base = 0; base < W * 64; base += nt) {
        uint32_t i = base + tid;
        bool neg = i < W * 64 && x[i] < 0.0f;
        uint64_t m = __ballot(neg);
        if (lane_id() == 0 && i < W * 64) {
            qb_out[i >> 6] = m;
            s_qw[i >> 6] = m;
        }
    }
    // ---- FastScan table (src/quantize.rs:279-313): position j uses x[4j .. 4j+3]
    float lo = INFINITY, hi = -INFINITY;
    float raw[16];
    const bool own = tid < npos;
    if (own) {
        float xs[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) xs[t] = x[4 * tid + t];
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
    const float range = fmaxf(block_max_f32(own ? hi - lo : 0.0f, reinterpret_cast<float*>(scratch)), 0.0f);
    const float delta = fmaxf(range / 255.0f, 1e-12f);
    if (own) {
        uint32_t pk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            float qv = fminf(fmaxf(roundf((raw[e] - lo) / delta), 0.0f), 255.0f);
            pk[e >> 2] |= static_cast<uint32_t>(qv) << (8 * (e & 3));
        }
        reinterpret_cast<uint4*>(Wk.lut + static_cast<uint64_t>(qi) * npos * 16)[tid] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
    __syncthreads();
    if (mode == 2) {  // query_prep test entry point
        if (tid == 0) {
            Wk.bias[qi] = seq_sum_lds(mins, npos, -0.0f);  // Rust's f32 Sum folds from -0.0
            Wk.delta[qi] = delta;
        }
        return;
    }
    // ---- wave 0 lane 0: the two sequential sums (bias, cqbase) while the other waves run the
    // Hamming pass; everything else: Hamming against every centroid code + live histogram
    for (uint32_t i = tid; i < nbins; i += nt) hist[i] = 0;
    __syncthreads();
    if (tid == 0) {
        Wk.bias[qi] = seq_sum_lds(mins, npos, -0.0f);
        Wk.delta[qi] = delta;
        s_cqbase = sq8 ? seq_sum_lds(cqp, d, 0.0f) : 0.0f;
    }
    {
        uint64_t qw[W];
#pragma unroll
        for (int w = 0; w < (int)W; ++w) qw[w] = s_qw[w];
        const uint32_t h0 = nt > 64 ? 64u : 0u;  // wave 0 is busy with the sums
        for (uint32_t c = tid - h0; tid >= h0 && c < M; c += 2 * (nt - h0)) {
            const uint32_t c2 = c + (nt - h0);
            uint64_t a[W], b[W];
#pragma unroll
            for (int w = 0; w < (int)W; ++w) a[w] = A.cent_bits[static_cast<uint64_t>(c) * W + w];
            const bool two = c2 < M;
            if (two) {
#pragma unroll
                for (int w = 0; w < (int)W; ++w) b[w] = A.cent_bits[static_cast<uint64_t>(c2) * W + w];
            }
            const uint8_t l1 = A.live[c];
            const uint8_t l2 = two ? A.live[c2] : 0;
            uint32_t h1 = 0, h2 = 0;
#pragma unroll
            for (int w = 0; w < (int)W; ++w) h1 += __popcll(qw[w] ^ a[w]);
            hs[c] = l1 ? static_cast<uint16_t>(h1) : 0xFFFFu;
            if (l1) atomicAdd(&hist[h1], 1u);
            if (two) {
#pragma unroll
                for (int w = 0; w < (int)W; ++w) h2 += __popcll(qw[w] ^ b[w]);
                hs[c2] = l2 ? static_cast<uint16_t>(h2) : 0xFFFFu;
                if (l2) atomicAdd(&hist[h2], 1u);
            }
        }
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
    // ---- shortlist: live cells with h <= cut, ascending id (dead cells hold 0xFFFF)
    {
        uint32_t per = (M + nt - 1) / nt, c0 = tid * per, c1 = min(c0 + per, M), cnt = 0;
        for (uint32_t c = c0; c < c1; ++c) cnt += hs[c] <= cut;
        uint32_t total;
        uint32_t pos = block_excl_scan_u32(cnt, scratch, &total);
        if (tid == 0) s_nsl = total;
        if (total <= K.sort_cap)
            for (uint32_t c = c0; c < c1; ++c)
                if (hs[c] <= cut) keys[pos++] = c;
    }
    __syncthreads();
    const uint32_t nsl = s_nsl;
    uint32_t* chosen = Wk.chosen + static_cast<uint64_t>(qi) * K.nprobe;
    float* cscore = Wk.cscore + static_cast<uint64_t>(qi) * K.nprobe;
    if (nsl > K.sort_cap) {
        if (tid == 0) {
            atomicAdd(&Wk.ctl->err_shortlist, 1u);
            atomicMax(&Wk.ctl->max_shortlist, nsl);
            Wk.nchosen[qi] = 0;
        }
        return;
    }
    // ---- exact rescore, 8 lanes per cell in the reference's FMA order (:777-800)
    const float cqbase = sq8 ? s_cqbase : 0.0f;
    {
        const uint32_t l = tid & 7, grp = tid >> 3, ngrp = nt >> 3;
        const uint32_t rounds = (nsl + ngrp - 1) / ngrp;
        for (uint32_t rr = 0; rr < rounds; ++rr) {
            const uint32_t i = rr * ngrp + grp;
            const uint32_t c = i < nsl ? static_cast<uint32_t>(keys[i]) : static_cast<uint32_t>(keys[0]);
            float s;
            if (sq8)
                s = dot_cm_u8(A.cent_sq8 + static_cast<uint64_t>(c) * A.cu.stride, A.cu, l,
                              [&](uint32_t j) { return cqs[j]; }) + cqbase;
            else
                s = dot_cm_f32(A.cents + static_cast<uint64_t>(c) * A.cf.stride, A.cf, l,
                               [&](uint32_t j) { return cqs[j]; });
            __syncthreads();  // every read of keys[] in this round precedes the writes
            if (i < nsl && l == 0) keys[i] = desc_score_key(s, c);
        }
    }
    __syncthreads();
    // ---- probe list: ascending keys = (score desc, cell asc)
    const uint32_t cap = min(K.nprobe, nsl);
    if (nsl <= 256) {
        wave0_sort_prefix(keys, nsl, keys, nsl);
    } else {
        uint32_t n2 = 1;
        while (n2 < nsl) n2 <<= 1;
        for (uint32_t i = nsl + tid; i < n2; i += nt) keys[i] = kKeyMax;
        bitonic_sort_u64(keys, n2);
    }
    __syncthreads();
    for (uint32_t i = tid; i < K.nprobe; i += nt) {
        bool ok = i < cap;
        chosen[i] = ok ? static_cast<uint32_t>(keys[i]) : kNone;
        cscore[i] = ok ? key_score(keys[i]) : __uint_as_float(0x7fc00000u);
    }
    // ---- nucleus over the capped list (:1960-1973); tc >= 1 keeps all cap cells
    if (tid == 0) {
        uint32_t nch = cap;
        if (K.use_nucleus && cap > 0) {
            const float max_s = key_score(keys[0]);
            float z = -0.0f;
            for (uint32_t i = 0; i < cap; ++i) z += exp_f((key_score(keys[i]) - max_s) * K.beta);
            float cum = 0.0f;
            bool near = false;
            for (uint32_t i = 0; i < cap; ++i) {
                cum += exp_f((key_score(keys[i]) - max_s) * K.beta) / (z + 1e-9f);
                if (fabsf(cum - K.tc) <= K.nucleus_band) near = true;
                if (cum >= K.tc) {
                    nch = i + 1;
                    break;
                }
            }
            if (near) Wk.flag_route[atomicAdd(&Wk.ctl->nflag_route, 1u)] = qi;
        }
        Wk.nchosen[qi] = nch;
    }
}

// ---------------------------------------------------------------- seed (one WG per query)

// All canonical members of the first 8 probed cells are scored at once (src/index.rs:2150-2154);
// tau is their exact target-th smallest d (:2155-2160) and only d <= tau is kept; then the
// adaptive cut (:2166-2188) and the per-cell probe counts for the inversion.
template <int NW>
__global__ void __launch_bounds__(kSeedThreads)
seed_kernel(DevArena A, Work Wk, KParams K) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t qi = blockIdx.x;
    if (qi >= K.nq) return;
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    constexpr uint32_t TB = NW * 256;
    uint8_t* table = smem;
    uint32_t* probed = reinterpret_cast<uint32_t*>(smem + TB);
    uint32_t* sbuf = probed + ((A.MW + 3) & ~3u);              // seed_cap: d << 16 | item (item < 65536)
    uint32_t* hist = sbuf + ((K.seed_cap + 3) & ~3u);
    uint32_t* scratch = hist + kHistBins;
    float* fsc = reinterpret_cast<float*>(scratch + 32);       // nt floats
    __shared__ uint32_t s_off[kSeedCells + 1], s_cell[kSeedCells], s_cnt, s_keep;

    const uint32_t nch = Wk.nchosen[qi];
    const uint32_t* chosen = Wk.chosen + static_cast<uint64_t>(qi) * K.nprobe;
    const float* cscore = Wk.cscore + static_cast<uint64_t>(qi) * K.nprobe;
    const uint32_t ns = min(kSeedCells, nch);
    {
        const uint32_t* lut = reinterpret_cast<const uint32_t*>(Wk.lut + static_cast<uint64_t>(qi) * TB);
        for (uint32_t i = tid; i < TB / 4; i += nt) reinterpret_cast<uint32_t*>(table)[i] = lut[i];
    }
    for (uint32_t i = tid; i < A.MW; i += nt) probed[i] = 0;
    if (tid == 0) {
        s_cnt = 0;
        s_keep = 0;
        uint32_t o = 0;
        for (uint32_t s = 0; s < ns; ++s) {
            uint32_t c = chosen[s];
            s_cell[s] = c;
            s_off[s] = o;
            o += A.mem_off[c + 1] - A.mem_off[c];
        }
        s_off[ns] = o;
    }
    __syncthreads();
    for (uint32_t i = tid; i < nch; i += nt) atomicOr(&probed[chosen[i] >> 5], 1u << (chosen[i] & 31));
    __syncthreads();
    {
        uint32_t* gprobed = Wk.probed + static_cast<uint64_t>(qi) * A.MW;
        for (uint32_t i = tid; i < A.MW; i += nt) gprobed[i] = probed[i];
    }
    const uint32_t total = s_off[ns];
    if (total > K.seed_cap) {  // cannot happen for an arena whose largest cell fits (checked at upload)
        if (tid == 0) atomicAdd(&Wk.ctl->err_seed, 1u);
        return;
    }
    // ---- score every seed member, all cells at once
    for (uint32_t base = 0; base < total; base += nt) {
        const uint32_t it = base + tid;
        bool pass = false;
        uint32_t dv = 0;
        if (it < total) {
            uint32_t s = 0;
#pragma unroll
            for (uint32_t k = 1; k < kSeedCells; ++k) s += (k < ns && it >= s_off[k]);
            const uint32_t c = s_cell[s];
            const uint64_t e = static_cast<uint64_t>(A.mem_off[c]) + (it - s_off[s]);
            Code<NW> code;
            code.load(A.codes + e * (2 * NW));
            const uint32_t slot = A.members[e];
            pass = canonical(A, e, slot, c, probed);
            uint32_t sm[1];
            lut_sums<NW, 1>(code, table, sm);
            dv = A.maxk - sm[0];
        }
        uint64_t m = __ballot(pass);
        uint32_t wb = 0;
        if (lane_id() == 0 && m) wb = atomicAdd(&s_cnt, static_cast<uint32_t>(__popcll(m)));
        wb = __shfl(wb, 0, kWave);
        if (pass) sbuf[wb + lanes_below(m)] = (dv << 16) | it;
    }
    __syncthreads();
    const uint32_t cnt = s_cnt;
    // ---- tau = target-th smallest seed d; keep d <= tau (src/index.rs:2155-2160)
    uint32_t tau = A.maxk;
    if (cnt >= K.target) tau = select_kth(cnt, K.target, [&](uint32_t i) { return sbuf[i] >> 16; }, hist, scratch);
    uint2* seed = Wk.seed + static_cast<uint64_t>(qi) * K.seed_cap;
    for (uint32_t base = 0; base < cnt; base += nt) {
        const uint32_t i = base + tid;
        uint32_t v = i < cnt ? sbuf[i] : 0u;
        const bool keep = i < cnt && (v >> 16) <= tau;
        uint64_t m = __ballot(keep);
        uint32_t wb = 0;
        if (lane_id() == 0 && m) wb = atomicAdd(&s_keep, static_cast<uint32_t>(__popcll(m)));
        wb = __shfl(wb, 0, kWave);
        if (keep) {
            const uint32_t it = v & 0xFFFFu;
            uint32_t s = 0;
#pragma unroll
            for (uint32_t k = 1; k < kSeedCells; ++k) s += (k < ns && it >= s_off[k]);
            const uint32_t slot = A.members[A.mem_off[s_cell[s]] + (it - s_off[s])];
            seed[wb + lanes_below(m)] = make_uint2(v >> 16, slot);
        }
    }
    // ---- adaptive cut: b_i = cos(max(acos(clamp(cs_i)) - r_c, 0)), suffix max, first i >= ns
    // with suffix_i < thr - margin
    uint32_t rest_end = nch;
    if (K.adaptive && cnt >= K.target && ns < nch) {
        const float est = Wk.delta[qi] * static_cast<float>(A.maxk - tau) + Wk.bias[qi];
        const float thr = fminf(fmaxf(est / K.norm, -1.0f), 1.0f);
        const float T = thr - K.at_margin;
        const uint32_t m = nch - ns, per = (m + nt - 1) / nt;
        const uint32_t i0 = ns + tid * per, i1 = min(i0 + per, nch);
        float run_max = -INFINITY;
        for (uint32_t i = i1; i-- > i0;)
            run_max = fmaxf(run_max, cos_f(fmaxf(acos_f(fminf(fmaxf(cscore[i], -1.0f), 1.0f)) - A.r_bound[chosen[i]], 0.0f)));
        // inclusive suffix max of the run maxima (Hillis-Steele over the block, from the right)
        fsc[tid] = run_max;
        __syncthreads();
        for (uint32_t off = 1; off < nt; off <<= 1) {
            float o = tid + off < nt ? fsc[tid + off] : -INFINITY;
            __syncthreads();
            fsc[tid] = fmaxf(fsc[tid], o);
            __syncthreads();
        }
        float later = tid + 1 < nt ? fsc[tid + 1] : -INFINITY;
        uint32_t first = kNone;
        bool near = false;
        float sfx = later;
        for (uint32_t i = i1; i-- > i0;) {
            sfx = fmaxf(sfx, cos_f(fmaxf(acos_f(fminf(fmaxf(cscore[i], -1.0f), 1.0f)) - A.r_bound[chosen[i]], 0.0f)));
            if (sfx < T) first = i;
            if (fabsf(sfx - T) <= K.prune_band) near = true;
        }
        const uint32_t fe = block_min_u32(first, scratch);
        const uint32_t any_near = block_sum_u32(near ? 1u : 0u, scratch);
        if (fe != kNone) rest_end = fe;
        if (tid == 0 && any_near) Wk.flag_prune[atomicAdd(&Wk.ctl->nflag_prune, 1u)] = qi;
    }
    // ---- probe counts for the inversion, and this query's work counters
    uint32_t sb = 0, rb = 0;
    for (uint32_t i = tid; i < rest_end; i += nt) {
        const uint32_t c = chosen[i];
        const uint32_t nb = (A.mem_off[c + 1] - A.mem_off[c] + 31) / 32;
        if (i < ns) {
            sb += nb;
        } else {
            rb += nb;
            atomicAdd(&Wk.cell_cnt[c], 1u);
        }
    }
    sb = block_sum_u32(sb, scratch);
    rb = block_sum_u32(rb, scratch);
    if (tid == 0) {
        Wk.seed_cnt[qi] = s_keep;
        Wk.tau[qi] = tau;
        Wk.rest_end[qi] = rest_end;
        Wk.qstat[3ull * qi] = sb;
        Wk.qstat[3ull * qi + 1] = rb;
        Wk.qstat[3ull * qi + 2] = rest_end > ns ? rest_end - ns : 0u;
    }
}

// ---------------------------------------------------------------- inversion: cell -> queries

// Probe counts alone (used when a host fix changes a cut after the seed stage ran).
__global__ void invert_count_kernel(Work Wk, KParams K) {
    uint32_t qi = blockIdx.x;
    if (qi >= K.nq) return;
    uint32_t ns = min(kSeedCells, Wk.nchosen[qi]), re = Wk.rest_end[qi];
    const uint32_t* chosen = Wk.chosen + static_cast<uint64_t>(qi) * K.nprobe;
    for (uint32_t i = ns + threadIdx.x; i < re; i += blockDim.x) atomicAdd(&Wk.cell_cnt[chosen[i]], 1u);
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

// One workgroup per cell (the CPU loop this replaces is src/index.rs:2231-2275). Lanes own
// members; each lane's code is loaded once per pass while groups of kG probing queries stream
// through the LDS table; survivors d <= tau of canonical members are appended per query.
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
        const uint64_t e = static_cast<uint64_t>(e0) + (have ? i : 0u);  // past the end: member 0, no output
        Code<NW> code;
        code.load(A.codes + e * (2 * NW));
        const uint32_t slot = A.members[e];
        const uint32_t alt = A.ma == 2 ? A.entry_alt[e] : kNoAlt;
        for (uint32_t g0 = 0; g0 < nqc; g0 += kG) {
            const uint32_t ng = min(kG, nqc - g0);
            __syncthreads();
            if (tid < kG) {
                uint32_t qq = tid < ng ? Wk.qof[q0 + g0 + tid] : kNone;
                s_q[tid] = qq;
                s_t[tid] = qq != kNone ? Wk.tau[qq] : 0u;
            }
            // interleave the group's tables: table[x*4 + g] = lut_g[x] (4x4 byte transpose)
            for (uint32_t x4 = tid; x4 < TB / 4; x4 += nt) {
                uint32_t v[kG];
#pragma unroll
                for (uint32_t g = 0; g < kG; ++g) {
                    uint32_t qq = g < ng ? Wk.qof[q0 + g0 + g] : kNone;
                    v[g] = qq != kNone ? reinterpret_cast<const uint32_t*>(Wk.lut + static_cast<uint64_t>(qq) * TB)[x4] : 0u;
                }
                uint32_t lo01 = __builtin_amdgcn_perm(v[1], v[0], 0x05010400u);
                uint32_t hi01 = __builtin_amdgcn_perm(v[1], v[0], 0x07030602u);
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
                    if (dv <= s_t[g]) {
                        const uint32_t* probed = Wk.probed + static_cast<uint64_t>(qq) * A.MW;
                        if (A.ma == 2)
                            pass = !(alt < c && ((probed[alt >> 5] >> (alt & 31)) & 1u));
                        else
                            pass = canonical(A, e, slot, c, probed);
                    }
                }
                uint64_t m = __ballot(pass);
                if (m) {
                    uint32_t wb = 0;
                    if (lane_id() == 0) wb = atomicAdd(&Wk.cand_cnt[qq], static_cast<uint32_t>(__popcll(m)));
                    wb = __shfl(wb, 0, kWave);
                    uint32_t pos = wb + lanes_below(m);
                    if (pass && pos < K.cand_cap) Wk.cand[static_cast<uint64_t>(qq) * K.cand_cap + pos] = make_uint2(dv, slot);
                }
            }
        }
    }
}

// ---------------------------------------------------------------- finish (one WG per query)

// Exact tie-inclusive cut at k*rerank_factor over the seed and scan candidates
// (src/index.rs:2281-2293), exact rerank (rerank_exact, :1309-1378), top-k by (score desc, slot asc).
__global__ void __launch_bounds__(kFinishThreads)
finish_kernel(DevArena A, Work Wk, KParams K, const float* __restrict__ queries, uint32_t* __restrict__ out_slots,
              float* __restrict__ out_scores) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t qi = blockIdx.x;
    if (qi >= K.nq) return;
    const uint32_t tid = threadIdx.x, nt = blockDim.x, d = A.d;
    uint32_t* hist = reinterpret_cast<uint32_t*>(smem);
    uint32_t* scratch = hist + kHistBins;
    float* qs = reinterpret_cast<float*>(scratch + 32);
    uint64_t* keys = reinterpret_cast<uint64_t*>(qs + ((d + 3) & ~3u));  // kFinishLdsCap
    __shared__ uint32_t s_n;
    __shared__ float s_base;

    const uint32_t ns_cnt = Wk.seed_cnt[qi];
    const uint32_t cc = Wk.cand_cnt[qi];
    const uint32_t nc = min(cc, K.cand_cap);
    const uint2* seed = Wk.seed + static_cast<uint64_t>(qi) * K.seed_cap;
    const uint2* cand = Wk.cand + static_cast<uint64_t>(qi) * K.cand_cap;
    const uint32_t total = ns_cnt + nc;
    const float* q = queries + static_cast<uint64_t>(qi) * d;
    const bool sq8 = A.rerank_mode == MAIVS_RERANK_SQ8;
    for (uint32_t j = tid; j < d; j += nt) qs[j] = sq8 ? q[j] * A.sq_step[j] : q[j];
    if (tid == 0) s_n = 0;
    // ---- G = target-th smallest d; with fewer than target candidates every one is kept
    uint32_t cutv = A.maxk;
    if (total >= K.target)
        cutv = select_kth(total, K.target, [&](uint32_t i) { return i < ns_cnt ? seed[i].x : cand[i - ns_cnt].x; },
                          hist, scratch);
    if (sq8 && tid == 0) {
        float b = 0.0f;
        for (uint32_t j = 0; j < d; ++j) b += q[j] * A.sq_min[j];
        s_base = b;
    }
    __syncthreads();
    // ---- compact the survivors into fin[] (global, read back by the debug entry point)
    uint2* fin = Wk.fin + static_cast<uint64_t>(qi) * K.fin_cap;
    for (uint32_t base = 0; base < total; base += nt) {
        const uint32_t i = base + tid;
        uint2 e = make_uint2(0, 0);
        bool pass = false;
        if (i < total) {
            e = i < ns_cnt ? seed[i] : cand[i - ns_cnt];
            pass = e.x <= cutv;
        }
        uint64_t m = __ballot(pass);
        uint32_t wb = 0;
        if (lane_id() == 0 && m) wb = atomicAdd(&s_n, static_cast<uint32_t>(__popcll(m)));
        wb = __shfl(wb, 0, kWave);
        if (pass) fin[wb + lanes_below(m)] = e;
    }
    __syncthreads();
    const uint32_t n = s_n;
    // ---- exact rerank, 8 lanes per row
    const bool in_lds = n <= kFinishLdsCap;
    uint64_t* kk = in_lds ? keys : (Wk.keys + static_cast<uint64_t>(qi) * K.key_cap);
    {
        const uint32_t l = tid & 7, grp = tid >> 3, ngrp = nt >> 3;
        const uint32_t rounds = (n + ngrp - 1) / ngrp;
        const float base = sq8 ? s_base : 0.0f;
        for (uint32_t rr = 0; rr < rounds; ++rr) {
            const uint32_t i = rr * ngrp + grp;
            const uint32_t slot = i < n ? fin[i].y : fin[0].y;
            float s;
            if (sq8)
                s = base + dot_cm_u8(A.sq8 + static_cast<uint64_t>(slot) * A.cu.stride, A.cu, l,
                                     [&](uint32_t j) { return qs[j]; });
            else
                s = dot_cm_f32(A.vecs + static_cast<uint64_t>(slot) * A.cf.stride, A.cf, l,
                               [&](uint32_t j) { return qs[j]; });
            if (i < n && l == 0) kk[i] = desc_score_key(s, slot);
        }
    }
    __syncthreads();
    const uint32_t kout = min(K.k, n);
    if (n <= 256) {
        wave0_sort_prefix(kk, n, kk, kout);
    } else {
        // n <= kFinishLdsCap (a power of two) keeps n2 in LDS; larger lists live in the global key buffer
        uint32_t n2 = 1;
        while (n2 < n) n2 <<= 1;
        for (uint32_t i = n + tid; i < n2; i += nt) kk[i] = kKeyMax;
        bitonic_sort_u64(kk, n2);
    }
    __syncthreads();
    for (uint32_t i = tid; i < K.k; i += nt) {
        const bool ok = i < kout;
        out_slots[static_cast<uint64_t>(qi) * K.k + i] = ok ? static_cast<uint32_t>(kk[i]) : kNone;
        out_scores[static_cast<uint64_t>(qi) * K.k + i] = ok ? key_score(kk[i]) : -INFINITY;
    }
    if (tid == 0) {
        Wk.cut[qi] = cutv;
        Wk.ncand[qi] = n;
        if (cc > K.cand_cap) atomicMax(&Wk.ctl->max_cand, cc);
    }
}

// Work counters of the last batch (on demand, one workgroup).
__global__ void counters_kernel(Work Wk, uint32_t nq) {
    __shared__ uint32_t scratch[32];
    unsigned long long v[5] = {0, 0, 0, 0, 0};
    for (uint32_t i = threadIdx.x; i < nq; i += blockDim.x) {
        v[0] += Wk.qstat[3ull * i];
        v[1] += Wk.qstat[3ull * i + 1];
        v[2] += Wk.qstat[3ull * i + 2];
        v[3] += Wk.cand_cnt[i];
        v[4] += Wk.ncand[i];
    }
    for (int k = 0; k < 5; ++k) {
        // per-thread partials are < 2^32 for any batch the buffers can hold
        uint32_t s = block_sum_u32(static_cast<uint32_t>(v[k]), scratch);
        if (threadIdx.x == 0) (&Wk.ctl->seed_blocks)[k] = s;
    }
}

}  // namespace maivs_dev
