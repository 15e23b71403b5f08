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
#include "types.h"
#include "wave_tree.h"

namespace maivs_dev {

// ---------------------------------------------------------------- small pieces

// f32 acos / cos / exp evaluated in f64 and rounded once. glibc's acosf / cosf / expf (what the
// reference's f32::acos / cos / exp call) are not correctly rounded, so a decision that lands
// within a small band of its threshold is flagged and re-evaluated on the host with libm.
__device__ __forceinline__ float acos_f(float x) { return static_cast<float>(acos(static_cast<double>(x))); }
__device__ __forceinline__ float cos_f(float x) { return static_cast<float>(cos(static_cast<double>(x))); }
__device__ __forceinline__ float exp_f(float x) { return static_cast<float>(exp(static_cast<double>(x))); }

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
    float s = acc + xor_lanes<4>(acc);
    float s2 = xor_lanes<2>(s);
    float u = s + s2;
    float r = u + xor_lanes<1>(u);
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
    float s = acc + xor_lanes<4>(acc);
    float s2 = xor_lanes<2>(s);
    float u = s + s2;
    float r = u + xor_lanes<1>(u);
    const uint8_t* tp = row + 8 * C.Tp;
    for (uint32_t i = 0; i < C.tail; ++i) r += q(8 * C.T + i) * static_cast<float>(tp[i]);
    return r;
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
                // keep both running sums in order every 8 lookups (no re-association into trees
                // that hold every looked-up word live)
                if ((t & 7) == 7) asm volatile("" : "+v"(S), "+v"(T));
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

// Hamming distance of a member's code to the query's code words (qd: the query's 2 * NW dwords).
template <int NW>
__device__ __forceinline__ uint32_t code_hamming(const Code<NW>& c, const uint32_t (&qd)[2 * NW]) {
    if constexpr (NW == 1) {
        return __popc(c.v[0].x ^ qd[0]) + __popc(c.v[0].y ^ qd[1]);
    } else {
        uint32_t h = 0;
#pragma unroll
        for (int k = 0; k < Code<NW>::NCH; ++k)
            h += __popc(c.v[k].x ^ qd[4 * k]) + __popc(c.v[k].y ^ qd[4 * k + 1]) + __popc(c.v[k].z ^ qd[4 * k + 2]) +
                 __popc(c.v[k].w ^ qd[4 * k + 3]);
        return h;
    }
}

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

// One member's nibble sums against an 8-query interleaved FastScan table in LDS (table byte
// x*8 + g = query g's entry x, x = position*16 + value). kWide: one 8-byte lookup serves queries
// 0-7; otherwise a 4-byte lookup serves queries 0-3 (items of at most 4 queries). Each half
// accumulates as in lut_sums: whole words S and the odd bytes T as u16 lanes, un-mixed at the end.
template <int NW, bool kWide>
__device__ __forceinline__ void lut_chunk8(uint32_t dw0, uint32_t dw1, uint32_t dw2, uint32_t dw3, int npos,
                                           const uint8_t* tk, uint32_t& S0, uint32_t& T0, uint32_t& S1,
                                           uint32_t& T1) {
#pragma unroll
    for (int t = 0; t < 32; ++t) {
        if (t < npos) {
            const uint32_t dw = t < 8 ? dw0 : t < 16 ? dw1 : t < 24 ? dw2 : dw3;
            const uint32_t nib = (dw >> (4 * (t & 7))) & 0xFu;
            if constexpr (kWide) {
                const uint2 e = reinterpret_cast<const uint2*>(tk)[t * 16 + nib];
                S0 += e.x;
                T0 += __builtin_amdgcn_perm(0u, e.x, 0x0c030c01u);
                S1 += e.y;
                T1 += __builtin_amdgcn_perm(0u, e.y, 0x0c030c01u);
                if ((t & 3) == 3) asm volatile("" : "+v"(S0), "+v"(T0), "+v"(S1), "+v"(T1));
            } else {
                const uint32_t e = reinterpret_cast<const uint32_t*>(tk)[2 * (t * 16 + nib)];
                S0 += e;
                T0 += __builtin_amdgcn_perm(0u, e, 0x0c030c01u);
                if ((t & 7) == 7) asm volatile("" : "+v"(S0), "+v"(T0));
            }
        }
    }
}

template <int NW, bool kWide>
__device__ __forceinline__ void lut_sums8(const Code<NW>& c, const uint8_t* table, uint32_t (&sum)[8]) {
    uint32_t S0 = 0, T0 = 0, S1 = 0, T1 = 0;
    if constexpr (NW == 1) {
        lut_chunk8<NW, kWide>(c.v[0].x, c.v[0].y, 0u, 0u, 16, table, S0, T0, S1, T1);
    } else {
        uint4 v[Code<NW>::NCH];
#pragma unroll
        for (int k = 0; k < Code<NW>::NCH; ++k) v[k] = c.v[k];
#pragma unroll 1
        for (int k = 0; k < Code<NW>::NCH; ++k) {
            lut_chunk8<NW, kWide>(v[0].x, v[0].y, v[0].z, v[0].w, 32, table + static_cast<uint32_t>(k) * 32 * 16 * 8,
                                  S0, T0, S1, T1);
#pragma unroll
            for (int r = 0; r + 1 < Code<NW>::NCH; ++r) v[r] = v[r + 1];  // rotate: chunk k+1 to the front
        }
    }
    auto unmix = [](uint32_t S, uint32_t T, uint32_t* out) {
        const uint32_t b1 = T & 0xFFFFu, b3 = T >> 16;
        const uint32_t r = S - (b1 << 8) - (b3 << 24);
        out[0] = r & 0xFFFFu;
        out[1] = b1;
        out[2] = r >> 16;
        out[3] = b3;
    };
    unmix(S0, T0, sum);
    if constexpr (kWide)
        unmix(S1, T1, sum + 4);
    else
        sum[4] = sum[5] = sum[6] = sum[7] = 0;
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

// f(get(i)) for i in [0, n), each thread taking i = tid, tid + nt, ...: eight values are loaded
// before any is used, so a long list in global memory has eight loads per thread in flight.
template <class Get, class F>
__device__ __forceinline__ void for_each_value8(uint32_t n, Get get, F f) {
    constexpr uint32_t U = 8;
    for (uint32_t base = threadIdx.x; base < n; base += U * blockDim.x) {
        uint32_t v[U];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t i = base + u * blockDim.x;
            v[u] = i < n ? get(i) : 0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < U; ++u)
            if (base + u * blockDim.x < n) f(v[u]);
    }
}

// Exact `want`-th smallest (1-based) of n values d < 65536 from get(i). Two 256-bin LDS histogram
// passes; every thread returns the value. Block-uniform call.
template <class Get>
__device__ uint32_t select_kth(uint32_t n, uint32_t want, Get get, uint32_t* hist, uint32_t* scratch) {
    for (uint32_t i = threadIdx.x; i < kHistBins; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    for_each_value8(n, get, [&](uint32_t d) { atomicAdd(&hist[d >> 8], 1u); });
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
    for_each_value8(n, get, [&](uint32_t d) {
        if ((d >> 8) == hb) atomicAdd(&hist[d & 0xFFu], 1u);
    });
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

// The tag of every entry's slot (for the filter test inside the scans).
__global__ void entry_tag_kernel(const uint32_t* __restrict__ members, const uint32_t* __restrict__ tags, uint64_t E,
                                 uint32_t* __restrict__ out) {
    for (uint64_t e = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; e < E;
         e += static_cast<uint64_t>(gridDim.x) * blockDim.x)
        out[e] = tags[members[e]];
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

// Zero the per-call counters: control block, cell counts, candidate counts, the epilogue's count.
__global__ void reset_kernel(Work Wk, uint32_t M, uint32_t nq) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x, stride = gridDim.x * blockDim.x;
    if (i < sizeof(Ctl) / 4) reinterpret_cast<uint32_t*>(Wk.ctl)[i] = 0;
    if (i == 0) *Wk.done = 0;
    for (uint32_t j = i; j <= M; j += stride) Wk.cell_cnt[j] = 0;
    for (uint32_t j = i; j < nq; j += stride) Wk.cand_cnt[j] = 0;
}

// Entry-major codes of an index without FastScan blocks: entry e gets its slot's code words.
__global__ void gather_codes_kernel(const uint64_t* __restrict__ slot_codes, const uint32_t* __restrict__ members,
                                    uint64_t E, uint32_t W, uint64_t* __restrict__ codes) {
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < E * W;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t e = i / W, w = i - e * W;
        codes[i] = slot_codes[static_cast<uint64_t>(members[e]) * W + w];
    }
}

// Padded results (no cell probed): no slot, score -inf (src/index.rs:3353-3361).
__global__ void pad_kernel(uint32_t* __restrict__ slots, float* __restrict__ scores, uint64_t n) {
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        slots[i] = kNone;
        scores[i] = -INFINITY;
    }
}

// ---------------------------------------------------------------- prep + Hamming (one wave per query)

// Rotation and sign code of one query, by one wave (src/quantize.rs:57-67,152-163;
// src/index.rs:1934-1942), with the rescore operands. Lane l holds rotated
// coordinates [l*EPL, (l+1)*EPL) in registers: FWHT levels below EPL run inside the lane, the
// others across lanes (partner l ^ (h / EPL)), in the reference's ascending level order, so every
// butterfly sees the reference's operands. `xs` is the wave's LDS region (x[P] | mins[npos4] |
// cqp[d4] | rqp[d4]): it receives the rotated query and the summands q * csq_min (and, for an SQ8
// rerank store, q * sq_min) that prep_wave_tables adds up; `qw` receives the code words. cqs_lds
// (or null): an LDS copy of the rescore operand cqs (d floats, 16-byte aligned).
template <int EPL>
__device__ __forceinline__ void prep_wave_codes(const DevArena& A, const Work& Wk, const float* __restrict__ queries,
                                                uint32_t qi, uint32_t lane, float* xs, uint64_t* qw,
                                                float* cqs_lds = nullptr) {
    const uint32_t P = A.P, d = A.d, npos = A.npos;
    const uint32_t np4 = (npos + 3) & ~3u;
    float* mins = xs + P;
    float* cqp = mins + np4;
    float* rqp = cqp + ((d + 3) & ~3u);
    const float* q = queries + static_cast<uint64_t>(qi) * d;
    const bool sq8 = A.cent_sq8 != nullptr;
    const bool rsq8 = A.rerank_mode == MAIVS_RERANK_SQ8;
    const uint32_t base = lane * EPL;
    float x[EPL], sg[2][EPL];
    // whole float4s where the lane's coordinates are all inside the query (the common case)
    const bool vec = EPL >= 4 && (d & 3u) == 0 && base + EPL <= d;
    if (vec) {
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
            const float4 v = *reinterpret_cast<const float4*>(q + base + e);
            x[e] = v.x;
            x[e + 1] = v.y;
            x[e + 2] = v.z;
            x[e + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) x[e] = base + e < d ? q[base + e] : 0.0f;
    }
    // signs, steps and mins are 16-byte aligned device arrays; base is a multiple of EPL
    auto ld4 = [](const float* p, float* o) {
        const float4 v = *reinterpret_cast<const float4*>(p);
        o[0] = v.x;
        o[1] = v.y;
        o[2] = v.z;
        o[3] = v.w;
    };
    if constexpr (EPL >= 4) {
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
            ld4(A.rot_signs + base + e, &sg[0][e]);
            ld4(A.rot_signs + P + base + e, &sg[1][e]);
        }
    } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            sg[0][e] = A.rot_signs[base + e];
            sg[1][e] = A.rot_signs[P + base + e];
        }
    }
    float* cqs_out = Wk.cqs + static_cast<uint64_t>(qi) * d;
    if (vec) {
        // rescore operands: cqs = q * step and q * min, each rounded once (src/index.rs:1937-1941)
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
            float st[4] = {1.f, 1.f, 1.f, 1.f}, mn[4] = {0.f, 0.f, 0.f, 0.f};
            if (sq8) {
                ld4(A.csq_step + base + e, st);
                ld4(A.csq_min + base + e, mn);
            }
            float4 o, m;
            o.x = sq8 ? x[e] * st[0] : x[e];
            o.y = sq8 ? x[e + 1] * st[1] : x[e + 1];
            o.z = sq8 ? x[e + 2] * st[2] : x[e + 2];
            o.w = sq8 ? x[e + 3] * st[3] : x[e + 3];
            m.x = sq8 ? x[e] * mn[0] : 0.0f;
            m.y = sq8 ? x[e + 1] * mn[1] : 0.0f;
            m.z = sq8 ? x[e + 2] * mn[2] : 0.0f;
            m.w = sq8 ? x[e + 3] * mn[3] : 0.0f;
            *reinterpret_cast<float4*>(cqs_out + base + e) = o;
            if (cqs_lds) *reinterpret_cast<float4*>(cqs_lds + base + e) = o;
            *reinterpret_cast<float4*>(cqp + base + e) = m;
        }
    } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const uint32_t i = base + e;
            if (i < d) {
                const float v = x[e];
                const float o = sq8 ? v * A.csq_step[i] : v;
                cqs_out[i] = o;
                if (cqs_lds) cqs_lds[i] = o;
                cqp[i] = sq8 ? v * A.csq_min[i] : 0.0f;
            }
        }
    }
    if (rsq8) {
        // (the loads unconditional, past d from the last coordinate, so they are in flight together)
        float mn[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) mn[e] = A.sq_min[min(base + e, d - 1)];
#pragma unroll
        for (int e = 0; e < EPL; ++e)
            if (base + e < d) rqp[base + e] = x[e] * mn[e];
    }
    for (int r = 0; r < 2; ++r) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) x[e] *= sg[r][e];
#pragma unroll
        for (int h = 1; h < EPL; h <<= 1) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                if ((e & h) == 0) {
                    const float u = x[e], v = x[e + h];
                    x[e] = u + v;
                    x[e + h] = u - v;
                }
            }
        }
        auto across = [&](auto mc) {
            constexpr int m = decltype(mc)::value;
            const bool upper = (lane & m) != 0;
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const float v = xor_lanes<m>(x[e]);
                x[e] = upper ? v - x[e] : x[e] + v;
            }
        };
        across(std::integral_constant<int, 1>{});
        across(std::integral_constant<int, 2>{});
        across(std::integral_constant<int, 4>{});
        across(std::integral_constant<int, 8>{});
        across(std::integral_constant<int, 16>{});
        across(std::integral_constant<int, 32>{});
#pragma unroll
        for (int e = 0; e < EPL; ++e) x[e] *= A.fht_scale;
    }
#pragma unroll
    for (int e = 0; e < EPL; ++e) xs[base + e] = x[e];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- 1-bit code over the first 64*W coordinates: bit i = x[i] < 0
    {
        uint64_t mine = 0;
        for (uint32_t w = 0; w < A.W; ++w) {
            const uint64_t m = __ballot(xs[64 * w + lane] < 0.0f);
            if (lane == w) mine = m;
        }
        if (lane < A.W) {
            Wk.qbits[static_cast<uint64_t>(qi) * A.W + lane] = mine;
            qw[lane] = mine;
        }
    }
    (void)mins;
}

// s + src[0] + ... + src[n - 1] added in index order by one lane, from LDS (16-byte aligned): 32
// floats at a time in two alternating buffers, each chunk's reads in flight while the one before
// is added.
__device__ __forceinline__ float seq_sum_lds(const float* src, uint32_t n, float s) {
    const float4* src4 = reinterpret_cast<const float4*>(src);
    const uint32_t nfull = n / 32;
    float4 ba[8], bb[8];
    auto fetch = [&](float4 (&buf)[8], uint32_t c) {
#pragma unroll
        for (int j = 0; j < 8; ++j) buf[j] = src4[8 * c + j];
    };
    auto add = [&](const float4 (&buf)[8]) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            s += buf[j].x;
            s += buf[j].y;
            s += buf[j].z;
            s += buf[j].w;
        }
    };
    if (nfull > 0) fetch(ba, 0);
    for (uint32_t c = 0; c < nfull; c += 2) {
        if (c + 1 < nfull) fetch(bb, c + 1);
        add(ba);
        if (c + 1 >= nfull) break;
        if (c + 2 < nfull) fetch(ba, c + 2);
        add(bb);
    }
    for (uint32_t i = nfull * 32; i < n; ++i) s += src[i];
    return s;
}

// The FastScan table and the sequential sums of one query, by one wave, from prep_wave_codes'
// LDS region (src/quantize.rs:279-313; src/index.rs:1326-1330,1934-1942).
__device__ __forceinline__ void prep_wave_tables(const DevArena& A, const Work& Wk, uint32_t qi, uint32_t lane,
                                                 float* xs, uint8_t* lds_table = nullptr) {
    const uint32_t P = A.P, d = A.d, npos = A.npos;
    const uint32_t np4 = (npos + 3) & ~3u;
    float* mins = xs + P;
    float* cqp = mins + np4;
    float* rqp = cqp + ((d + 3) & ~3u);
    const bool sq8 = A.cent_sq8 != nullptr;
    const bool rsq8 = A.rerank_mode == MAIVS_RERANK_SQ8;
    // ---- FastScan table: position j from x[4j .. 4j+3], 16 sums accumulated from 0 in order t = 0..3
    auto raw_of = [&](const float4& v, int e) {
        float s = 0.0f;
        s += (e & 1) ? -v.x : v.x;
        s += (e & 2) ? -v.y : v.y;
        s += (e & 4) ? -v.z : v.z;
        s += (e & 8) ? -v.w : v.w;
        return s;
    };
    float range = 0.0f;
    for (uint32_t j = lane; j < npos; j += kWave) {
        const float4 v = reinterpret_cast<const float4*>(xs)[j];
        float lo = INFINITY, hi = -INFINITY;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float s = raw_of(v, e);
            lo = fminf(lo, s);
            hi = fmaxf(hi, s);
        }
        mins[j] = lo;
        range = fmaxf(range, hi - lo);
    }
    range = wave_max_f32(range);
    const float delta = fmaxf(range / 255.0f, 1e-12f);
    uint4* lut = reinterpret_cast<uint4*>(Wk.lut + static_cast<uint64_t>(qi) * npos * 16);
    for (uint32_t j = lane; j < npos; j += kWave) {
        const float4 v = reinterpret_cast<const float4*>(xs)[j];
        const float lo = mins[j];
        uint32_t pk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float qv = fminf(fmaxf(roundf((raw_of(v, e) - lo) / delta), 0.0f), 255.0f);
            pk[e >> 2] |= static_cast<uint32_t>(qv) << (8 * (e & 3));
        }
        lut[j] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        if (lds_table) reinterpret_cast<uint4*>(lds_table)[j] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- sequential sums in index order: lane 0 the table bias (Rust's f32 Sum folds from -0.0),
    // lane 1 the rescore base sum(q * csq_min) from 0.0, lane 2 the SQ8 rerank base
    // sum(q * sq_min) from 0.0
    if (lane < 3) {
        const uint32_t n = lane == 0 ? npos : lane == 1 ? (sq8 ? d : 0u) : (rsq8 ? d : 0u);
        const float* src = lane == 0 ? mins : lane == 1 ? cqp : rqp;
        const float s = seq_sum_lds(src, n, lane == 0 ? -0.0f : 0.0f);
        if (lane == 0) {
            Wk.bias[qi] = s;
            Wk.delta[qi] = delta;
        } else if (lane == 1) {
            Wk.cqbase[qi] = s;
        } else {
            Wk.rbase[qi] = s;
        }
    }
}

// Rotation, sign code, FastScan table and sums of one query by one wave (prep_wave_codes, then
// prep_wave_tables once the wave's LDS writes are visible to it).
template <int EPL>
__device__ __forceinline__ void prep_wave(const DevArena& A, const Work& Wk, const float* __restrict__ queries,
                                          uint32_t qi, uint32_t lane, float* xs, uint64_t* qw) {
    prep_wave_codes<EPL>(A, Wk, queries, qi, lane, xs, qw);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    prep_wave_tables(A, Wk, qi, lane, xs);
}

// kPrepWaves queries per workgroup, one wave each (prep_wave). Flag kPrepReset also clears the
// per-call counters (control block, probe counts, candidate counts).
// LDS: codes[kPrepWaves * 16] u64 | per wave x[P] | mins[npos4] | cqp[d4] | rqp[d4].
template <int EPL>
__global__ void __launch_bounds__(kPrepWaves * kWave)
prep_kernel(DevArena A, Work Wk, KParams K, const float* __restrict__ queries, uint32_t flags) {
    extern __shared__ __align__(16) uint8_t smem[];
    if (flags & kPrepReset) {
        const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x, stride = gridDim.x * blockDim.x;
        if (i < sizeof(Ctl) / 4) reinterpret_cast<uint32_t*>(Wk.ctl)[i] = 0;
        if (i == 0) *Wk.done = 0;
        for (uint32_t j = i; j <= A.M; j += stride) Wk.cell_cnt[j] = 0;
        for (uint32_t j = i; j < K.nq; j += stride) Wk.cand_cnt[j] = 0;
    }
    const uint32_t lane = lane_id(), wv = threadIdx.x / kWave;
    const uint32_t qi = blockIdx.x * kPrepWaves + wv;
    uint64_t* qbl = reinterpret_cast<uint64_t*>(smem);
    if (qi < K.nq) prep_wave<EPL>(A, Wk, queries, qi, lane, reinterpret_cast<float*>(qbl + kPrepWaves * 16) +
                                  wv * (A.P + ((A.npos + 3) & ~3u) + 2 * ((A.d + 3) & ~3u)), qbl + wv * 16);
}


// ---------------------------------------------------------------- route (one WG per query)

// The query's Hamming row (src/index.rs:1896-1915): h = popcount(q ^ c) over the code words for
// every cell, into hd (LDS, up to kHdLdsCells cells; else the query's row of Wk.hs) with the
// padding up to Mp holding 0xFFFF, and the histogram of the cells' h. Dead cells are counted too:
// dead_fixup takes them out afterwards (there are few or none). Run by threads t = 0 .. nt-1
// (nt a multiple of 64) of the workgroup. L lanes share a cell code, a 16-byte chunk each
// (NW = 1: one lane, the whole 8-byte code), so that one load instruction reads a contiguous run
// of codes; the partial counts meet by lane exchange. Rounds of U codes per lane are double
// buffered: the next round's loads are in flight while this round is counted. The loop bounds are
// uniform: every lane takes part in the exchanges. The query's code comes from q_lds (LDS) or else
// from Wk.qbits; before reading it the threads call wait() (the caller's barrier after which the
// code and the cleared histogram are ready), with the first round's code loads already in flight.
struct NoWait {
    __device__ void operator()() const {}
};
template <int NW, class Wait = NoWait>
__device__ __forceinline__ void hamming_row(const DevArena& A, const Work& Wk, uint32_t qi, uint32_t* hist,
                                            uint16_t* hd_lds, uint32_t t, uint32_t nt,
                                            const uint64_t* q_lds = nullptr, Wait wait = Wait{}) {
    const uint32_t M = A.M, Mp = A.Mp;
    auto run = [&](auto* out) {
        constexpr uint32_t L = NW >= 2 ? NW / 2 : 1;
        constexpr uint32_t U = 8;
        const uint32_t sub = t % L, cpr = nt / L, cl = t / L, step = U * cpr;
        uint64_t q0 = 0, q1 = 0;  // the query's code words of this lane, read after wait()
        // (32-bit byte offsets from the codes' base, M * NW * 8 < 2^32: one offset register per load.
        // A lane's cells of a round are stepped one from the last, each step behind an empty asm
        // statement, so the compiler keeps no per-u offsets live across the loop.)
        const char* cb = reinterpret_cast<const char*>(A.cent_bits);
        auto load = [&](uint32_t base, uint64_t (&w0)[U], uint64_t (&w1)[U]) {
            uint32_t c = base + cl;
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                if (u) {
                    c += cpr;
                    asm volatile("" : "+v"(c));
                }
                const uint32_t off = (c < M ? c : 0u) * (NW * 8u) + (NW >= 2 ? sub * 16u : 0u);
                if constexpr (NW == 1) {
                    w0[u] = *reinterpret_cast<const uint64_t*>(cb + off);
                    w1[u] = 0ull;
                } else {
                    const uint4 v = *reinterpret_cast<const uint4*>(cb + off);
                    w0[u] = (static_cast<uint64_t>(v.y) << 32) | v.x;
                    w1[u] = (static_cast<uint64_t>(v.w) << 32) | v.z;
                }
            }
        };
        auto count = [&](uint32_t base, const uint64_t (&w0)[U], const uint64_t (&w1)[U]) {
            uint32_t c = base + cl;
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                if (u) {
                    c += cpr;
                    asm volatile("" : "+v"(c));
                }
                uint32_t h = __popcll(q0 ^ w0[u]) + (NW >= 2 ? __popcll(q1 ^ w1[u]) : 0u);
                if constexpr (L >= 2) h += static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(h), 0xB1, 0xF, 0xF, true));
                if constexpr (L >= 4) h += static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(h), 0x4E, 0xF, 0xF, true));
                if constexpr (L >= 8) h += __shfl_xor(h, 4, kWave);
                if (sub == 0 && c < Mp) {
                    out[c] = c < M ? static_cast<uint16_t>(h) : static_cast<uint16_t>(0xFFFFu);
                    if (c < M) atomicAdd(&hist[h], 1u);
                }
            }
        };
        uint64_t a0[U], a1[U], b0[U], b1[U];
        load(0, a0, a1);
        wait();
        const uint64_t* qg = q_lds ? q_lds : Wk.qbits + static_cast<uint64_t>(qi) * NW;
        q0 = qg[NW >= 2 ? 2 * sub : 0];
        q1 = NW >= 2 ? qg[2 * sub + 1] : 0ull;
        // (the loads are unconditional, cells past M read cell 0's code and are not counted: with no
        // branch around them the compiler's wait counts let a round's loads stay in flight while the
        // round before it is counted)
        for (uint32_t base = 0; base < Mp; base += 2 * step) {
            load(base + step, b0, b1);
            count(base, a0, a1);
            if (base + step >= Mp) break;
            load(base + 2 * step, a0, a1);
            count(base + step, b0, b1);
        }
    };
    if (Mp <= kHdLdsCells)
        run(hd_lds);
    else
        run(Wk.hs + static_cast<uint64_t>(qi) * Mp);
}

// Takes the dead cells (no members) out of hamming_row's histogram and row: h = 0xFFFF. The row
// is in LDS up to kHdLdsCells cells unless global_row (the rows a Hamming-rows kernel wrote).
__device__ __forceinline__ void dead_fixup(const DevArena& A, const Work& Wk, uint32_t qi, uint32_t* hist,
                                           uint16_t* hd_lds, uint32_t t, uint32_t nt, bool global_row = false) {
    uint16_t* hd = !global_row && A.Mp <= kHdLdsCells ? hd_lds : Wk.hs + static_cast<uint64_t>(qi) * A.Mp;
    for (uint32_t i = t; i < A.n_dead; i += nt) {
        const uint32_t c = A.dead[i];
        atomicSub(&hist[hd[c]], 1u);
        hd[c] = static_cast<uint16_t>(0xFFFFu);
    }
}

// kFront: the caller (front_kernel) already cleared the histogram, staged cqs and ran hamming_row,
// and K.tree_list and K.flat_route are 0. kRowsReady: hamming_kernel already wrote the query's row of Wk.hs (more
// cells than the LDS row holds); the histogram is built from it. Callers that hold them on chip
// pass (else null): cqs_src, the query's cqs in LDS; tl_lds and n_tl, the tree's leaf list in LDS
// and its length; aux, nt floats of LDS that carry each shortlisted cell's r_bound through the
// sort (loaded beside its centroid row at the rescore).
template <class Get>
__device__ uint32_t select_kth_u32(uint32_t n, uint32_t want, Get get, uint32_t* hist, uint32_t* scratch);

template <int NW, bool kFront = false, bool kRowsReady = false>
__device__ __forceinline__ void route_phase(const DevArena& A, const Work& Wk, const KParams& K, uint32_t qi,
                                            const float* cqs_src = nullptr, const uint32_t* tl_lds = nullptr,
                                            uint32_t n_tl = 0, float* aux = nullptr) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    const uint32_t d = A.d, M = A.M, Mp = A.Mp;
    const uint32_t d4 = (d + 3) & ~3u, np4 = min((K.nprobe + 3) & ~3u, K.sort_cap);
    const uint32_t nbins = NW * 64 + 1;
    float* cqs = reinterpret_cast<float*>(smem);
    float* ex = cqs + d4;
    uint64_t* keys = reinterpret_cast<uint64_t*>(ex + np4);
    uint32_t* hist = reinterpret_cast<uint32_t*>(keys + K.sort_cap);
    uint32_t* scratch = hist + ((nbins + 3) & ~3u);
    __shared__ uint32_t s_cut;

    if constexpr (!kFront) {
        for (uint32_t i = tid; i < nbins; i += nt) hist[i] = 0;
        for (uint32_t i = tid; i < d; i += nt) cqs[i] = cqs_src ? cqs_src[i] : Wk.cqs[static_cast<uint64_t>(qi) * d + i];
        __syncthreads();
    }
    uint32_t nsl = 0;
    if (!kFront && K.tree_list && tl_lds && A.n_dead == 0) {
        // the centroid tree's leaves, every one live (route_query, src/index.rs:1193-1204)
        for (uint32_t i = tid; i < min(n_tl, K.sort_cap); i += nt) keys[i] = tl_lds[i];
        nsl = n_tl;
    } else if (!kFront && K.tree_list) {
        // the centroid tree's leaves, live cells only (route_query, src/index.rs:1193-1204)
        const uint32_t* tl = tl_lds ? tl_lds : Wk.tlist + static_cast<uint64_t>(qi) * K.tcap;
        const uint32_t nt_list = tl_lds ? n_tl : Wk.tcount[qi];
        for (uint32_t r0 = 0; r0 < nt_list; r0 += nt) {
            const uint32_t i = r0 + tid;
            const uint32_t c = i < nt_list ? tl[i] : 0u;
            // (an index without dead cells has every cell live: no member-range loads)
            const bool live = i < nt_list && A.mem_off[c + 1] > A.mem_off[c];
            uint32_t tot;
            const uint32_t pos = nsl + block_excl_scan_u32(live ? 1u : 0u, scratch, &tot);
            if (live && pos < K.sort_cap) keys[pos] = c;
            nsl += tot;
        }
    } else if (!kFront && K.flat_route) {
        // every live cell, ascending id (route_query without a tree or two-stage routing,
        // src/index.rs:1260-1269)
        for (uint32_t r0 = 0; r0 < M; r0 += nt) {
            const uint32_t c = r0 + tid;
            const bool live = c < M && A.mem_off[c + 1] > A.mem_off[c];
            uint32_t tot;
            const uint32_t pos = nsl + block_excl_scan_u32(live ? 1u : 0u, scratch, &tot);
            if (live && pos < K.sort_cap) keys[pos] = c;
            nsl += tot;
        }
    } else {
    if constexpr (kRowsReady) {
        // the row in 16-byte chunks (Mp is a multiple of 8), four per thread in flight
        const uint4* row = reinterpret_cast<const uint4*>(Wk.hs + static_cast<uint64_t>(qi) * Mp);
        const uint32_t nch8 = Mp / 8;
        for (uint32_t c0 = tid; c0 < nch8; c0 += 4 * nt) {
            uint4 v[4];
#pragma unroll
            for (uint32_t u = 0; u < 4; ++u) {
                const uint32_t ch = c0 + u * nt;
                v[u] = ch < nch8 ? row[ch] : make_uint4(0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu);
            }
#pragma unroll
            for (uint32_t u = 0; u < 4; ++u) {
                const uint32_t w4[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
                for (uint32_t k = 0; k < 8; ++k) {
                    const uint32_t h = (k & 1) ? (w4[k >> 1] >> 16) : (w4[k >> 1] & 0xFFFFu);
                    if (h != 0xFFFFu) atomicAdd(&hist[h], 1u);
                }
            }
        }
        __syncthreads();
    } else if constexpr (!kFront) {
        hamming_row<NW>(A, Wk, qi, hist, reinterpret_cast<uint16_t*>(scratch + 16), tid, nt);
        __syncthreads();
    }
    if (A.n_dead) {
        dead_fixup(A, Wk, qi, hist, reinterpret_cast<uint16_t*>(scratch + 16), tid, nt, kRowsReady);
        __syncthreads();
    }
    // cut = smallest t whose cumulative live count reaches want_c (wave 0: a run of bins per lane,
    // a wave scan, and the one lane whose run crosses want_c)
    if (tid < kWave) {
        const uint32_t lane = tid, per = (nbins + kWave - 1) / kWave, b0 = lane * per, b1 = min(b0 + per, nbins);
        uint32_t loc = 0;
        for (uint32_t i = b0; i < b1; ++i) loc += hist[i];
        uint32_t x = wave_incl_scan_u32(loc);
        uint32_t cand = kNone, cum = x - loc;
        if (cum < K.want_c && x >= K.want_c) {
            for (uint32_t i = b0; i < b1; ++i) {
                cum += hist[i];
                if (cum >= K.want_c) {
                    cand = i;
                    break;
                }
            }
        }
        const uint64_t m = __ballot(cand != kNone);
        const uint32_t cut = m ? __shfl(cand, __ffsll(static_cast<long long>(m)) - 1, kWave) : NW * 64;
        if (lane == 0) s_cut = cut;
    }
    __syncthreads();
    const uint32_t cut = s_cut;
    // ---- shortlist: live cells with h <= cut, ascending id (dead cells and padding hold 0xFFFF)
    auto shortlist = [&](const auto* hd) {
        const uint4* hrow = reinterpret_cast<const uint4*>(hd);
        const uint32_t nch8 = Mp / 8;
        auto h_at = [](const uint4& v, int k) -> uint32_t {
            const uint32_t w = k < 2 ? v.x : k < 4 ? v.y : k < 6 ? v.z : v.w;
            return (k & 1) ? (w >> 16) : (w & 0xFFFFu);
        };
        // each thread a run of consecutive chunks of 8 cells, so one block scan orders them all;
        // the chunks four at a time, their loads in flight together
        const uint32_t per = (nch8 + nt - 1) / nt, c0 = min(tid * per, nch8), c1 = min(c0 + per, nch8);
        auto chunks4 = [&](uint32_t ch, uint4 (&v)[4]) {
#pragma unroll
            for (uint32_t u = 0; u < 4; ++u) v[u] = ch + u < c1 ? hrow[ch + u] : make_uint4(0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu);
        };
        uint32_t cnt = 0;
        for (uint32_t ch = c0; ch < c1; ch += 4) {
            uint4 v[4];
            chunks4(ch, v);
#pragma unroll
            for (uint32_t u = 0; u < 4; ++u)
#pragma unroll
                for (int k = 0; k < 8; ++k) cnt += h_at(v[u], k) <= cut;
        }
        uint32_t tot;
        uint32_t pos = block_excl_scan_u32(cnt, scratch, &tot);
        if (tot <= K.sort_cap) {
            for (uint32_t ch = c0; ch < c1; ch += 4) {
                uint4 v[4];
                chunks4(ch, v);
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u)
#pragma unroll
                    for (int k = 0; k < 8; ++k)
                        if (h_at(v[u], k) <= cut) keys[pos++] = (ch + u) * 8 + k;
            }
        }
        nsl = tot;
    };
    if (!kRowsReady && Mp <= kHdLdsCells)
        shortlist(reinterpret_cast<const uint16_t*>(scratch + 16));
    else
        shortlist(Wk.hs + static_cast<uint64_t>(qi) * Mp);
    }
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
    __syncthreads();
    // ---- exact rescore, 8 lanes per cell in the reference's FMA order (:777-800)
    const bool sq8 = A.cent_sq8 != nullptr;
    const float cqbase = sq8 ? Wk.cqbase[qi] : 0.0f;
    // (the adaptive stop's bound of a probed cell needs its r_bound: with aux, loaded at the
    // rescore and carried through the rank sort)
    const bool carry = aux != nullptr && K.adaptive && nsl <= nt;
    {
        const uint32_t l = tid & 7, grp = tid >> 3, ngrp = nt >> 3;
        const uint32_t rounds = (nsl + ngrp - 1) / ngrp;
        for (uint32_t rr = 0; rr < rounds; ++rr) {
            const uint32_t i = rr * ngrp + grp;
            const uint32_t c = i < nsl ? static_cast<uint32_t>(keys[i]) : static_cast<uint32_t>(keys[0]);
            const float rb = carry && l == 0 ? A.r_bound[c] : 0.0f;
            float s;
            if (sq8)
                s = dot_cm_u8(A.cent_sq8 + static_cast<uint64_t>(c) * A.cu.stride, A.cu, l,
                              [&](uint32_t j) { return cqs[j]; }) + cqbase;
            else
                s = dot_cm_f32(A.cents + static_cast<uint64_t>(c) * A.cf.stride, A.cf, l,
                               [&](uint32_t j) { return cqs[j]; });
            __syncthreads();  // every read of keys[] in this round precedes the writes
            if (i < nsl && l == 0) {
                const uint64_t key = desc_score_key(s, c);
                keys[i] = key;
                if (carry) aux[i] = rb;
            }
        }
    }
    __syncthreads();
    // ---- probe list: ascending keys = (score desc, cell asc)
    const uint32_t cap = min(K.nprobe, nsl);
    if (nsl <= nt) {
        // keys are unique: each one's rank among the nsl places it (read all, then write)
        uint64_t mine = 0;
        uint32_t r = 0;
        float mb = 0.0f;
        if (tid < nsl) {
            mine = keys[tid];
            if (carry) mb = aux[tid];
#pragma unroll 8
            for (uint32_t j = 0; j < nsl; ++j) r += keys[j] < mine;
        }
        __syncthreads();
        if (tid < nsl) {
            keys[r] = mine;
            if (carry) aux[r] = mb;
        }
    } else {
        uint32_t n2 = 1;
        while (n2 < nsl) n2 <<= 1;
        uint32_t m = nsl;  // keys that go to the sort
        if (nbins >= kHistBins && K.nprobe <= 2 * nt && n2 > 2 * nt) {
            // only keys[0 .. nprobe) are used: the nprobe-th smallest key's high word (the
            // score), then the keys up to it compacted to the front in order (every write lands
            // at or before an element already read), and only those sorted
            const uint32_t hv = select_kth_u32(nsl, K.nprobe, [&](uint32_t i) { return static_cast<uint32_t>(keys[i] >> 32); },
                                               hist, scratch);
            uint32_t base = 0;
            for (uint32_t r = 0; r < nsl; r += nt) {
                const uint32_t i = r + tid;
                const uint64_t key = i < nsl ? keys[i] : kKeyMax;
                const bool take = i < nsl && static_cast<uint32_t>(key >> 32) <= hv;
                uint32_t tot;
                // the scan's barriers follow every read of this round, so the writes below are safe
                const uint32_t off = block_excl_scan_u32(take ? 1u : 0u, scratch, &tot);
                if (take) keys[base + off] = key;
                base += tot;
                __syncthreads();
            }
            m = base;
            n2 = 1;
            while (n2 < m) n2 <<= 1;
        }
        for (uint32_t i = m + tid; i < n2; i += nt) keys[i] = kKeyMax;
        bitonic_sort_u64(keys, n2);
    }
    __syncthreads();
    for (uint32_t i = tid; i < K.nprobe; i += nt) {
        const bool ok = i < cap;
        const uint32_t c = ok ? static_cast<uint32_t>(keys[i]) : kNone;
        const float s = ok ? key_score(keys[i]) : __uint_as_float(0x7fc00000u);
        chosen[i] = c;
        cscore[i] = s;
        // the adaptive stop's bound of a probed cell (src/index.rs:1484-1485, 2178-2179)
        if (K.adaptive && ok && i >= K.bnd_from)
            Wk.bnd[static_cast<uint64_t>(qi) * K.nprobe + i] =
                cos_f(fmaxf(acos_f(fminf(fmaxf(s, -1.0f), 1.0f)) - (carry ? aux[i] : A.r_bound[c]), 0.0f));
    }
    // ---- nucleus over the capped list (:1960-1973); tc >= 1 keeps all cap cells
    uint32_t nch = cap;
    if (K.use_nucleus && cap > 0) {
        const float max_s = key_score(keys[0]);
        for (uint32_t i = tid; i < cap; i += nt) ex[i] = exp_f((key_score(keys[i]) - max_s) * K.beta);
        __syncthreads();
        if (tid == 0) {
            float z = -0.0f;
            for (uint32_t i = 0; i < cap; ++i) z += ex[i];
            float cum = 0.0f;
            bool near = false;
            for (uint32_t i = 0; i < cap; ++i) {
                cum += ex[i] / (z + 1e-9f);
                if (fabsf(cum - K.tc) <= K.nucleus_band) near = true;
                if (cum >= K.tc) {
                    nch = i + 1;
                    break;
                }
            }
            if (near) Wk.flag_route[atomicAdd(&Wk.ctl->nflag_route, 1u)] = qi;
        }
    }
    if (tid == 0) Wk.nchosen[qi] = nch;
}

template <int NW>
__global__ void __launch_bounds__(kRouteThreads)
route_kernel(DevArena A, Work Wk, KParams K) {
    if (blockIdx.x < K.nq) route_phase<NW>(A, Wk, K, blockIdx.x);
}

// ---------------------------------------------------------------- seed (one WG per query)

// One member's nibble sums against a single query's FastScan table at LDS offset 0: the
// position offsets are immediates of the LDS reads, so each lookup costs one bit-field
// extract and half an add.
template <int NW>
__device__ __forceinline__ uint32_t lut_sum1(const Code<NW>& c, const uint8_t* __restrict__ table) {
    uint32_t S = 0;
#pragma unroll
    for (int k = 0; k < Code<NW>::NCH; ++k) {
        const uint32_t dw[4] = {c.v[k].x, c.v[k].y, c.v[k].z, c.v[k].w};
        constexpr int npos = NW == 1 ? 16 : 32;
#pragma unroll
        for (int t = 0; t < npos; ++t) {
            const uint32_t nib = (dw[t >> 3] >> (4 * (t & 7))) & 0xFu;
            S += table[(k * 32 + t) * 16 + nib];
            // keep the running sum in order per 16 lookups: without this the compiler re-associates
            // all 16*NW terms into one tree and holds every looked-up byte live at once
            if ((t & 15) == 15) asm volatile("" : "+v"(S));
        }
    }
    return S;
}

// The same sum from a pair table in LDS: entry p*256 + (a | b << 4) = lut[2p][a] + lut[2p+1][b]
// (u16; every sum stays below 65536), looked up by code byte p, which holds nibbles 2p (low) and
// 2p + 1 (high). Half the lookups of lut_sum1; it wins where one workgroup has the CU's LDS to itself.
template <int NW>
__device__ __forceinline__ uint32_t lut_sum_pair(const Code<NW>& c, const uint16_t* __restrict__ pair) {
    uint32_t S = 0;
#pragma unroll
    for (int k = 0; k < Code<NW>::NCH; ++k) {
        const uint32_t dw[4] = {c.v[k].x, c.v[k].y, c.v[k].z, c.v[k].w};
        constexpr int nbytes = NW == 1 ? 8 : 16;
#pragma unroll
        for (int t = 0; t < nbytes; ++t) {
            const uint32_t byte = (dw[t >> 2] >> (8 * (t & 3))) & 0xFFu;
            S += pair[(k * 16 + t) * 256 + byte];
            if ((t & 15) == 15) asm volatile("" : "+v"(S));
        }
    }
    return S;
}

// All canonical members of the first SEED_CELLS probed cells are scored
// (src/index.rs:2150-2154); tau is their exact target-th smallest d (:2155-2160) and only
// d <= tau is kept; then the adaptive cut (:2166-2188) from the route's bounds, and the per-cell
// probe counts for the inversion.
// LDS: static table[TB] at offset 0; dynamic probed[MW4] | coarse[256] | fine[256] | misc[64] |
// sbuf[seed_cap4] u16 (d by item index).
// The seed stage's FastScan table in static LDS: the kernel's largest static LDS variable, at
// address 0, so the table lookups need no base add.
template <int NW>
__device__ __forceinline__ uint8_t* seed_table() {
    __shared__ __align__(16) uint8_t table[NW * 256];
    return table;
}

// kTableReady: the caller already wrote the query's table into seed_table<NW>().
template <int NW, bool kTableReady = false>
__device__ __forceinline__ void seed_phase(const DevArena& A, const Work& Wk, const KParams& K, uint32_t qi) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t tid = threadIdx.x, nt = blockDim.x, lane = lane_id();
    constexpr uint32_t TB = NW * 256;
    constexpr uint32_t kOff = 0, kCell = 9, kE0 = 17, kCnt = 25, kKeep = 26, kTau = 27, kRe = 28, kHb = 29, kBelow = 30;
    // the first rest cells (ranks ns .. ns + nr_max - 1): member offsets, cells and first entries
    constexpr uint32_t kROff = 32, kRCell = 41, kRE0 = 49;
    uint8_t* const table = seed_table<NW>();
    uint32_t* probed = reinterpret_cast<uint32_t*>(smem);
    uint32_t* coarse = probed + ((A.MW + 3) & ~3u);
    uint32_t* fine = coarse + 256;
    uint32_t* misc = fine + 256;
    uint16_t* sbuf = reinterpret_cast<uint16_t*>(misc + 64);

    const uint32_t nch = Wk.nchosen[qi];
    const uint32_t* chosen = Wk.chosen + static_cast<uint64_t>(qi) * K.nprobe;
    const uint32_t ns = min(kSeedCells, nch);
    const uint32_t nr_max = nch > ns ? min(nch - ns, K.front_rest) : 0u;
    if constexpr (!kTableReady) {
        const uint4* src = reinterpret_cast<const uint4*>(Wk.lut + static_cast<uint64_t>(qi) * TB);
        for (uint32_t i = tid; i < TB / 16; i += nt) reinterpret_cast<uint4*>(table)[i] = src[i];
    }
    for (uint32_t i = tid; i < A.MW; i += nt) probed[i] = 0;
    for (uint32_t i = tid; i < 512; i += nt) coarse[i] = 0;  // coarse and fine
    if (tid < kWave) {
        // the seed cells, and with the same loads the rest cells that the seed stage may scan
        uint32_t c = 0, e0 = 0, len = 0;
        if (tid < ns + nr_max) {
            c = chosen[tid];
            e0 = A.mem_off[c];
            len = A.mem_off[c + 1] - e0;
        }
        const bool rest = tid >= ns && tid < ns + nr_max;
        const uint32_t x = wave_incl_scan_u32(tid < ns ? len : 0u);
        const uint32_t xr = wave_incl_scan_u32(rest ? len : 0u);
        if (tid < ns) {
            misc[kOff + tid + 1] = x;
            misc[kCell + tid] = c;
            misc[kE0 + tid] = e0;
        }
        if (rest) {
            misc[kROff + tid - ns + 1] = xr;
            misc[kRCell + tid - ns] = c;
            misc[kRE0 + tid - ns] = e0;
        }
        if (tid == 0) {
            misc[kOff] = 0;
            misc[kROff] = 0;
            misc[kCnt] = 0;
            misc[kKeep] = 0;
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < nch; i += nt) atomicOr(&probed[chosen[i] >> 5], 1u << (chosen[i] & 31));
    __syncthreads();
    {
        uint32_t* gp = Wk.probed + static_cast<uint64_t>(qi) * A.MW;
        for (uint32_t i = tid; i < A.MW; i += nt) gp[i] = probed[i];
    }
    const uint32_t total = misc[kOff + ns];
    if (total > K.seed_cap) {  // cannot happen: seed_cap bounds the SEED_CELLS largest cells
        if (tid == 0) atomicAdd(&Wk.ctl->err_seed, 1u);
        return;
    }
    // seed-cell boundaries in scalar registers: a member's cell is the number of boundaries at or
    // below its item index
    uint32_t offv[kSeedCells];
#pragma unroll
    for (uint32_t k = 1; k < kSeedCells; ++k)
        offv[k] = k < ns ? __builtin_amdgcn_readfirstlane(misc[kOff + k]) : 0xFFFFFFFFu;
    auto seed_cell = [&](uint32_t it) {
        uint32_t s = 0;
#pragma unroll
        for (uint32_t k = 1; k < kSeedCells; ++k) s += it >= offv[k];
        return s;
    };
    // ---- score every seed member, all cells at once; coarse histogram of d >> 8 on the fly.
    // sbuf[item] = d, or kNoD for a member another probed home scores (or the filter drops).
    // Each thread scores two members per round while the next round's two codes are in flight.
    uint32_t npass = 0;
    if (total > 0) {
        const bool filt = K.filter != 0;
        struct Mem {
            Code<NW> code;
            uint64_t e;
            uint32_t c, alt, tag;
        };
        auto fetch = [&](uint32_t it, Mem& m) {
            const uint32_t j = min(it, total - 1);
            const uint32_t s = seed_cell(j);
            m.c = misc[kCell + s];
            m.e = static_cast<uint64_t>(misc[kE0 + s]) + (j - misc[kOff + s]);
            m.code.load(A.codes + m.e * (2 * NW));
            m.alt = A.ma == 2 ? A.entry_alt[m.e] : kNoAlt;
            m.tag = filt ? A.entry_tag[m.e] : 0u;
        };
        auto score = [&](const Mem& m, uint32_t it) {
            bool pass;
            if (A.ma == 2)
                pass = !(m.alt < m.c && ((probed[m.alt >> 5] >> (m.alt & 31)) & 1u));
            else
                pass = canonical(A, m.e, A.ma > 2 ? A.members[m.e] : 0u, m.c, probed);
            if (filt) pass = pass && m.tag >= K.tag_lo && m.tag <= K.tag_hi;
            const uint32_t dv = A.maxk - lut_sum1<NW>(m.code, table);
            if (pass) {
                atomicAdd(&coarse[dv >> 8], 1u);
                ++npass;
            }
            sbuf[it] = static_cast<uint16_t>(pass ? dv : kNoD);
        };
        Mem a, b;
        fetch(tid, a);
        fetch(tid + nt, b);
        for (uint32_t r = 0; r < total; r += 2 * nt) {
            const bool more = r + 2 * nt < total;
            Mem na, nb;
            if (more) {
                fetch(r + 2 * nt + tid, na);
                fetch(r + 3 * nt + tid, nb);
            }
            if (r + tid < total) score(a, r + tid);
            if (r + nt + tid < total) score(b, r + nt + tid);
            if (more) {
                a = na;
                b = nb;
            }
        }
    }
    {
        const uint32_t ws = wave_sum_u32(npass);
        if (lane == 0 && ws) atomicAdd(&misc[kCnt], ws);
    }
    __syncthreads();
    const uint32_t cnt = misc[kCnt];
    // ---- each thread's first two members of the first rest cells, loaded now so that their
    // latency passes under tau, the keep and the adaptive cut. Which of the cells are scanned
    // depends on those (ranks [ns, r_in) below): members past them are loaded but not kept.
    const bool filt = K.filter != 0;
    struct RMem {
        Code<NW> code;
        uint64_t e;
        uint32_t c, alt, tag, slot;
    };
    // member it (< tot) of the rest cells whose offsets are roff (roff[k] = offset of cell k)
    auto rfetch = [&](uint32_t it, uint32_t tot, const uint32_t (&roff)[kFrontRestMax], RMem& m) {
        const uint32_t j = min(it, tot - 1);
        uint32_t s = 0;
#pragma unroll
        for (uint32_t k = 1; k < kFrontRestMax; ++k) s += j >= roff[k];
        m.c = misc[kRCell + s];
        m.e = static_cast<uint64_t>(misc[kRE0 + s]) + (j - misc[kROff + s]);
        m.code.load(A.codes + m.e * (2 * NW));
        m.alt = A.ma == 2 ? A.entry_alt[m.e] : kNoAlt;
        m.tag = filt ? A.entry_tag[m.e] : 0u;
        m.slot = A.members[m.e];
    };
    auto rest_offsets = [&](uint32_t nr, uint32_t (&roff)[kFrontRestMax]) {
#pragma unroll
        for (uint32_t k = 1; k < kFrontRestMax; ++k)
            roff[k] = k < nr ? __builtin_amdgcn_readfirstlane(misc[kROff + k]) : 0xFFFFFFFFu;
    };
    const uint32_t rtot_max = misc[kROff + nr_max];
    RMem ra, rb;
    if (rtot_max > 0) {
        uint32_t roff[kFrontRestMax];
        rest_offsets(nr_max, roff);
        rfetch(tid, rtot_max, roff, ra);
        rfetch(tid + nt, rtot_max, roff, rb);
    }
    // ---- tau = target-th smallest seed d (two 256-bin passes, scanned by wave 0)
    uint32_t tau = A.maxk;
    if (cnt >= K.target) {
        auto find_bin = [&](const uint32_t* h, uint32_t want, uint32_t* bin, uint32_t* below) {
            uint32_t v[4], s4 = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[k] = h[4 * lane + k];
                s4 += v[k];
            }
            uint32_t x = wave_incl_scan_u32(s4);
            uint32_t cum = x - s4;
            if (cum < want && x >= want) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (cum + v[k] >= want) {
                        *bin = 4 * lane + k;
                        *below = cum;
                        break;
                    }
                    cum += v[k];
                }
            }
        };
        if (tid < kWave) find_bin(coarse, K.target, &misc[kHb], &misc[kBelow]);
        __syncthreads();
        const uint32_t hb = misc[kHb], need = K.target - misc[kBelow];
        for (uint32_t i = tid; i < total; i += nt) {
            const uint32_t dd = sbuf[i];
            if (dd != kNoD && (dd >> 8) == hb) atomicAdd(&fine[dd & 0xFFu], 1u);
        }
        __syncthreads();
        if (tid < kWave) find_bin(fine, need, &misc[kTau], &misc[kBelow]);
        __syncthreads();
        tau = (hb << 8) | misc[kTau];
    }
    // ---- keep d <= tau, with the member's slot (kNoD exceeds every tau: tau <= maxk < kNoD);
    // four rounds at a time, so that their slot loads are in flight together
    uint2* seed = Wk.seed + static_cast<uint64_t>(qi) * K.seed_cap;
    for (uint32_t b = 0; b < total; b += 4 * nt) {
        uint32_t v[4], slot[4];
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t i = b + u * nt + tid;
            v[u] = i < total ? sbuf[i] : kNoD;
            slot[u] = 0;
            if (v[u] <= tau) {
                const uint32_t sc = seed_cell(i);
                slot[u] = A.members[misc[kE0 + sc] + (i - misc[kOff + sc])];
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const bool keep = v[u] <= tau;
            const uint64_t m = __ballot(keep);
            uint32_t wb = 0;
            if (lane == 0 && m) wb = atomicAdd(&misc[kKeep], static_cast<uint32_t>(__popcll(m)));
            wb = __shfl(wb, 0, kWave);
            if (keep) seed[wb + lanes_below(m)] = make_uint2(v[u], slot[u]);
        }
    }
    __syncthreads();  // every wave's kept count is in misc[kKeep]
    // ---- the scans' running cut starts at tau, its histogram with the scored seed members
    if (K.run_thr == 1) {
        uint32_t* dh = Wk.dhist + static_cast<uint64_t>(qi) * kThrBins;
        for (uint32_t i = tid; i < kThrBins; i += nt) dh[i] = coarse[i];
        if (tid == 0) {
            Wk.thr[qi] = tau;
            Wk.thr_at[qi] = 0;
        }
    }
    // ---- adaptive cut: suffix maxima of the route's bounds, first i >= ns below thr - margin
    uint32_t rest_end = nch;
    if (K.adaptive && cnt >= K.target && ns < nch) {
        if (tid < kWave) {
            const float est = Wk.delta[qi] * static_cast<float>(A.maxk - tau) + Wk.bias[qi];
            const float thr = fminf(fmaxf(est / K.norm, -1.0f), 1.0f);
            const float T = thr - K.at_margin;
            const float* bnd = Wk.bnd + static_cast<uint64_t>(qi) * K.nprobe;
            float carry = -INFINITY;
            uint32_t firstb = kNone;
            bool near = false;
            for (int32_t hi = static_cast<int32_t>(nch); hi > static_cast<int32_t>(ns); hi -= kWave) {
                const int32_t lo = max(hi - kWave, static_cast<int32_t>(ns));
                const int32_t i = lo + static_cast<int32_t>(lane);
                const bool valid = i < hi;
                float x = valid ? bnd[i] : -INFINITY;
#pragma unroll
                for (int o = 1; o < kWave; o <<= 1) {
                    const float y = __shfl_down(x, o, kWave);
                    if (lane + o < static_cast<uint32_t>(kWave)) x = fmaxf(x, y);
                }
                x = fmaxf(x, carry);
                carry = __shfl(x, 0, kWave);
                const uint64_t below = __ballot(valid && x < T);
                if (below) firstb = static_cast<uint32_t>(lo) + static_cast<uint32_t>(__ffsll(static_cast<long long>(below)) - 1);
                if (__ballot(valid && fabsf(x - T) <= K.prune_band)) near = true;
            }
            if (lane == 0) {
                misc[kRe] = firstb != kNone ? firstb : nch;
                if (near) Wk.flag_prune[atomicAdd(&Wk.ctl->nflag_prune, 1u)] = qi;
            }
        }
        __syncthreads();
        rest_end = misc[kRe];
    }
    // ---- the first rest cells, ranks [ns, r_in), scanned here and query-major (the cell-major
    // scan takes the others): their canonical members with d <= tau become the query's first
    // candidates, as the cell-major scan would emit them (src/index.rs:2231-2275)
    const uint32_t r_in = min(rest_end, ns + K.front_rest);
    if (r_in > ns) {
        const uint32_t nr = r_in - ns;  // <= nr_max
        if (tid == 0) misc[kCnt] = 0;
        __syncthreads();
        const uint32_t rtotal = misc[kROff + nr];
        uint32_t roff[kFrontRestMax];
        rest_offsets(nr, roff);
        if (rtotal > 0) {
            // (the members below rtotal are the same under nr_max's offsets as under nr's)
            auto fetch = [&](uint32_t it, RMem& m) { rfetch(it, rtotal, roff, m); };
            auto keep = [&](const RMem& m, bool have, uint32_t& dv) {
                dv = A.maxk - lut_sum1<NW>(m.code, table);
                if (!have || dv > tau) return false;
                bool pass;
                if (A.ma == 2)
                    pass = !(m.alt < m.c && ((probed[m.alt >> 5] >> (m.alt & 31)) & 1u));
                else
                    pass = canonical(A, m.e, m.slot, m.c, probed);
                return pass && (!filt || (m.tag >= K.tag_lo && m.tag <= K.tag_hi));
            };
            uint2* cand = Wk.cand + static_cast<uint64_t>(qi) * K.cand_cap;
            RMem a = ra, b = rb;
            for (uint32_t r = 0; r < rtotal; r += 2 * nt) {
                const bool more = r + 2 * nt < rtotal;
                RMem na, nb;
                if (more) {
                    fetch(r + 2 * nt + tid, na);
                    fetch(r + 3 * nt + tid, nb);
                }
                uint32_t da, db;
                const bool pa = keep(a, r + tid < rtotal, da);
                const bool pb = keep(b, r + nt + tid < rtotal, db);
                const uint64_t ma = __ballot(pa), mb = __ballot(pb);
                if (ma | mb) {
                    uint32_t wb = 0;
                    if (lane == 0) wb = atomicAdd(&misc[kCnt], static_cast<uint32_t>(__popcll(ma) + __popcll(mb)));
                    wb = __shfl(wb, 0, kWave);
                    const uint32_t posa = wb + lanes_below(ma), posb = wb + static_cast<uint32_t>(__popcll(ma)) + lanes_below(mb);
                    if (pa && posa < K.cand_cap) cand[posa] = make_uint2(da, a.slot);
                    if (pb && posb < K.cand_cap) cand[posb] = make_uint2(db, b.slot);
                }
                if (more) {
                    a = na;
                    b = nb;
                }
            }
        }
        __syncthreads();
        // the query's count so far (the counters were cleared; the cell-major scan adds to it later)
        if (tid == 0) Wk.cand_cnt[qi] = misc[kCnt];
    }
    // ---- the query into each other rest cell's bucket (bucket mode), else probe counts for the
    // counting-sort inversion. Every kItemQ-th query of a cell opens a lookup work item for those
    // bucket entries, or, when the pass uses the matrix-core scan, every kBucketQ-th one a work
    // item of kBucketQ entries; the openings take one list-counter atomic per wave.
    const uint32_t per_item = K.mma_min ? kBucketQ : kItemQ;
    uint32_t* const list = K.mma_min ? Wk.active : Wk.active8;
    uint32_t* const list_n = K.mma_min ? &Wk.ctl->n_active : &Wk.ctl->n_active8;
    for (uint32_t i0 = r_in; i0 < rest_end; i0 += nt) {
        const uint32_t i = i0 + tid;
        bool opens = false;
        uint32_t c = 0, slot = 0;
        if (i < rest_end) {
            c = chosen[i];
            slot = atomicAdd(&Wk.cell_cnt[c], 1u);
            if (K.bucket_cap) {
                opens = slot % per_item == 0 && slot < K.bucket_cap;
                if (slot < K.bucket_cap)
                    Wk.qbuck[static_cast<uint64_t>(c) * K.bucket_cap + slot] = qi;
                else
                    atomicOr(&Wk.ctl->bucket_overflow, 1u);
            }
        }
        if (K.bucket_cap) {
            const uint64_t bm = __ballot(opens);
            if (bm) {
                uint32_t wb = 0;
                if (lane_id() == 0) wb = atomicAdd(list_n, static_cast<uint32_t>(__popcll(bm)));
                wb = __shfl(wb, 0, kWave);
                if (opens) list[wb + lanes_below(bm)] = c * kItemGroups + slot / per_item;
            }
        }
    }
    if (tid == 0) {
        Wk.seed_cnt[qi] = misc[kKeep];
        Wk.tau[qi] = tau;
        Wk.rest_end[qi] = rest_end;
    }
}

template <int NW>
__global__ void __launch_bounds__(kSeedThreads, 4)
seed_kernel(DevArena A, Work Wk, KParams K) {
    if (blockIdx.x < K.nq) seed_phase<NW>(A, Wk, K, blockIdx.x);
}

// Route and seed of one query in one workgroup (the seed reads the probe list the route just
// wrote; LDS is reused: the route's regions are dead once the list is written).
template <int NW, bool kRowsReady = false>
__global__ void __launch_bounds__(kSeedThreads)
route_seed_kernel(DevArena A, Work Wk, KParams K) {
    if (blockIdx.x >= K.nq) return;
    route_phase<NW, false, kRowsReady>(A, Wk, K, blockIdx.x);
    __syncthreads();
    seed_phase<NW>(A, Wk, K, blockIdx.x);
}

// Hamming rows of a tile of kHamQ queries against kHamC cells (src/index.rs:1896-1915), for
// indexes with more cells than a route keeps in LDS: one cell per thread, its code in registers,
// the tile's query codes in LDS, so each code is loaded once per kHamQ queries. Dead cells get
// their distance too (the route's dead_fixup takes them out); the padding up to Mp gets 0xFFFF.
template <int NW>
__global__ void __launch_bounds__(kHamC)
hamming_kernel(DevArena A, Work Wk, uint32_t nq) {
    __shared__ uint64_t qb[kHamQ][NW];
    const uint32_t q0 = blockIdx.x * kHamQ, c = blockIdx.y * kHamC + threadIdx.x;
    const uint32_t nqt = min(kHamQ, nq - q0);
    for (uint32_t i = threadIdx.x; i < kHamQ * NW; i += kHamC)
        qb[i / NW][i % NW] = i / NW < nqt ? Wk.qbits[static_cast<uint64_t>(q0 + i / NW) * NW + i % NW] : 0ull;
    uint64_t cw[NW];
    const uint64_t* src = A.cent_bits + static_cast<uint64_t>(c < A.M ? c : 0u) * NW;
#pragma unroll
    for (int w = 0; w < NW; ++w) cw[w] = src[w];
    __syncthreads();
    if (c >= A.Mp) return;
    for (uint32_t j = 0; j < nqt; ++j) {
        uint32_t h = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) h += __popcll(qb[j][w] ^ cw[w]);
        Wk.hs[static_cast<uint64_t>(q0 + j) * A.Mp + c] = c < A.M ? static_cast<uint16_t>(h) : static_cast<uint16_t>(0xFFFFu);
    }
}

// The same rows on the matrix cores: h = popc(q) + popc(c) - 2 (q . c), the code bits taken as
// int8 0/1 values in v_mfma_i32_32x32x32_i8 steps of 32 bits (the i32 sums are exact). A workgroup
// takes kHamMmaQ queries, 32 per wave, whose bits each wave expands into registers once, and
// kHamMmaC cells, 32 at a time: the 256 threads expand a tile's codes into LDS in the operand
// layout (double-buffered, so one barrier per tile), and each wave multiplies it with its queries.
// Operands of step s (bits 32s .. 32s + 31): lane l holds the 16 bits 32s + 16(l/32) .. + 15 of row
// (query) or column (cell) l % 32, one byte each; result register r of lane l is query
// 8(r/4) + 4(l/32) + r%4, cell l % 32.
typedef int mma_v4 __attribute__((ext_vector_type(4)));
typedef int mma_v16 __attribute__((ext_vector_type(16)));
constexpr uint32_t kHamMmaQ = 128, kHamMmaC = 256;

// bits b0..b3 of x to bytes 0..3 (the four shifted copies of x do not overlap, so no carries)
__device__ __forceinline__ uint32_t spread4(uint32_t x) { return ((x & 0xFu) * 0x00204081u) & 0x01010101u; }

__device__ __forceinline__ mma_v4 spread16(uint32_t b) {
    const mma_v4 v = {static_cast<int>(spread4(b)), static_cast<int>(spread4(b >> 4)), static_cast<int>(spread4(b >> 8)),
                      static_cast<int>(spread4(b >> 12))};
    return v;
}

template <int NW>
__global__ void __launch_bounds__(256) hamming_mma_kernel(DevArena A, Work Wk, uint32_t nq) {
    constexpr uint32_t S = 2 * NW;                         // 32-bit steps
    constexpr uint32_t PPT = (S * kWave + 255) / 256;      // operand pieces per thread per tile
    __shared__ mma_v4 bx[2][S][kWave];
    __shared__ uint32_t pcs[kHamMmaC];
    const uint32_t tid = threadIdx.x, lane = lane_id(), w = tid / kWave, g = lane >> 5, j = lane & 31;
    const uint32_t q0 = blockIdx.x * kHamMmaQ + w * 32, cb = blockIdx.y * kHamMmaC;
    const uint32_t ntile = (min(kHamMmaC, A.Mp > cb ? A.Mp - cb : 0u) + 31) / 32;
    if (ntile == 0) return;  // uniform over the workgroup
    // the block's cells' popcounts, one cell per thread
    {
        const uint32_t c = cb + tid;
        uint32_t pc = 0;
        if (c < A.M) {
#pragma unroll
            for (int k = 0; k < NW; ++k) pc += __popcll(A.cent_bits[static_cast<uint64_t>(c) * NW + k]);
        }
        pcs[tid] = pc;
    }
    // this wave's queries: lane (j, g) holds query q0 + j's bits 32s + 16g .. + 15 for every step
    mma_v4 a[S];
    uint32_t pq;
    {
        uint64_t qw[NW];
        const bool in = q0 + j < nq;
#pragma unroll
        for (int k = 0; k < NW; ++k) qw[k] = in ? Wk.qbits[static_cast<uint64_t>(q0 + j) * NW + k] : 0ull;
        pq = 0;
#pragma unroll
        for (int k = 0; k < NW; ++k) pq += __popcll(qw[k]);
#pragma unroll
        for (uint32_t s = 0; s < S; ++s)
            a[s] = spread16(static_cast<uint32_t>(qw[s / 2] >> (32 * (s & 1) + 16 * g)) & 0xFFFFu);
    }
    uint32_t prow[16];  // popc of the query of each result register
#pragma unroll
    for (uint32_t r = 0; r < 16; ++r) prow[r] = __shfl(pq, 8 * (r / 4) + 4 * g + (r % 4), kWave);
    // a tile's S * 64 operand pieces (step s, half gg, cell jj): their code words, then their bytes
    uint64_t raw[PPT];
    auto fetch = [&](uint32_t c0) {
#pragma unroll
        for (uint32_t k = 0; k < PPT; ++k) {
            const uint32_t u = tid + 256 * k, jj = u & 31, s = u >> 6, c = c0 + jj;
            raw[k] = u < S * kWave && c < A.M ? A.cent_bits[static_cast<uint64_t>(c) * NW + s / 2] : 0ull;
        }
    };
    auto store = [&](uint32_t buf) {
#pragma unroll
        for (uint32_t k = 0; k < PPT; ++k) {
            const uint32_t u = tid + 256 * k, jj = u & 31, gg = (u >> 5) & 1, s = u >> 6;
            if (u < S * kWave)
                bx[buf][s][gg * 32 + jj] = spread16(static_cast<uint32_t>(raw[k] >> (32 * (s & 1) + 16 * gg)) & 0xFFFFu);
        }
    };
    fetch(cb);
    store(0);
    for (uint32_t t = 0; t < ntile; ++t) {
        const uint32_t buf = t & 1, c0 = cb + 32 * t;
        __syncthreads();  // tile t is in bx[buf]; every wave is done with tile t - 1's buffer
        if (t + 1 < ntile) fetch(c0 + 32);
        // two independent accumulation chains over the steps
        mma_v16 acc0 = {}, acc1 = {};
#pragma unroll
        for (uint32_t s = 0; s < S; s += 2) {
            acc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s], bx[buf][s][lane], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s + 1], bx[buf][s + 1][lane], acc1, 0, 0, 0);
        }
        if (t + 1 < ntile) store(buf ^ 1);
        const uint32_t c = c0 + j, pc = pcs[32 * t + j];
        if (c < A.Mp) {
#pragma unroll
            for (uint32_t r = 0; r < 16; ++r) {
                const uint32_t q = q0 + 8 * (r / 4) + 4 * g + (r % 4);
                if (q < nq)
                    Wk.hs[static_cast<uint64_t>(q) * A.Mp + c] =
                        c < A.M ? static_cast<uint16_t>(prow[r] + pc - 2u * static_cast<uint32_t>(acc0[r] + acc1[r]))
                                : static_cast<uint16_t>(0xFFFFu);
            }
        }
    }
}

// Prep, route and seed of one query in one workgroup, for codes over the whole padded dimension
// (n_words * 64 == dim_pad, so prep's coordinates per lane equal NW). Wave 0 computes the query's
// rotation, code and rescore operand (prep_wave_codes, the operand straight into the route's LDS)
// while the other waves clear the route's histogram and load their first cell codes; then wave 0
// builds the FastScan table and sums (prep_wave_tables) while the others compute the Hamming row
// from the code in LDS; then every wave routes and seeds the query. LDS: the route's regions
// (route_phase's layout) | the prep region (codes[16] u64 | x[P] | mins | cqp | rqp); the seed
// phase reuses all of it.
template <int NW>
__global__ void __launch_bounds__(kSeedThreads, NW >= 16 ? 3 : 4)
front_kernel(DevArena A, Work Wk, KParams K, const float* __restrict__ queries) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t qi = blockIdx.x;
    if (qi >= K.nq) return;
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    const uint32_t d = A.d, d4 = (d + 3) & ~3u, np4 = min((K.nprobe + 3) & ~3u, K.sort_cap);
    const uint32_t nbins = NW * 64 + 1;
    float* cqs = reinterpret_cast<float*>(smem);
    uint32_t* hist = reinterpret_cast<uint32_t*>(reinterpret_cast<uint64_t*>(cqs + d4 + np4) + K.sort_cap);
    uint32_t* scratch = hist + ((nbins + 3) & ~3u);
    uint8_t* prep = smem + route_lds_bytes(d, NW, A.Mp, K.sort_cap, K.nprobe);
    float* xs = reinterpret_cast<float*>(prep + 16 * 8);
    // (waves 1-3 clear the histogram and put their first Hamming loads in flight before the barrier
    // that waits for the code; the rescore operand goes straight to the route's LDS)
    if (tid < kWave) {
        prep_wave_codes<NW>(A, Wk, queries, qi, lane_id(), xs, reinterpret_cast<uint64_t*>(prep), cqs);
        __syncthreads();
        prep_wave_tables(A, Wk, qi, lane_id(), xs, seed_table<NW>());
    } else {
        for (uint32_t i = tid - kWave; i < nbins; i += nt - kWave) hist[i] = 0;
        hamming_row<NW>(A, Wk, qi, hist, reinterpret_cast<uint16_t*>(scratch + 16), tid - kWave, nt - kWave,
                        reinterpret_cast<const uint64_t*>(prep), [] { __syncthreads(); });
    }
    __syncthreads();
    // (the rotated query x[P] is free once the table is built: it carries the route's bounds)
    route_phase<NW, true>(A, Wk, K, qi, nullptr, nullptr, 0, A.P >= nt ? xs : nullptr);
    __syncthreads();
    seed_phase<NW, true>(A, Wk, K, qi);
}

// ---------------------------------------------------------------- inversion: cell -> queries

// Probe counts alone (used when a host fix changes a cut after the seed stage ran).
__global__ void invert_count_kernel(Work Wk, KParams K) {
    uint32_t qi = blockIdx.x;
    if (qi >= K.nq) return;
    uint32_t ns = min(kSeedCells, Wk.nchosen[qi]), re = Wk.rest_end[qi];
    const uint32_t r0 = min(re, ns + K.front_rest);  // the seed stage scanned ranks [ns, r0)
    const uint32_t* chosen = Wk.chosen + static_cast<uint64_t>(qi) * K.nprobe;
    for (uint32_t i = r0 + threadIdx.x; i < re; i += blockDim.x) atomicAdd(&Wk.cell_cnt[chosen[i]], 1u);
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
    const uint32_t r0 = min(re, ns + K.front_rest);  // the seed stage scanned ranks [ns, r0)
    const uint32_t* chosen = Wk.chosen + static_cast<uint64_t>(qi) * K.nprobe;
    for (uint32_t i = r0 + threadIdx.x; i < re; i += blockDim.x) {
        uint32_t c = chosen[i];
        uint32_t pos = atomicAdd(&Wk.cell_cur[c], 1u);
        Wk.qof[pos] = qi;
    }
}

// ---------------------------------------------------------------- the cell-major scan


// Lowers query q's running cut to the upper edge of the d >> 8 bin holding the target-th smallest
// counted entry (one thread). Counts it reads may lag atomics still in flight; fewer counts give
// a higher edge, never one below the final cut.
__device__ __forceinline__ void thr_lower(const Work& Wk, const KParams& K, uint32_t q) {
    const uint4* h = reinterpret_cast<const uint4*>(Wk.dhist + static_cast<uint64_t>(q) * kThrBins);
    uint32_t cum = 0;
#pragma unroll 1
    for (uint32_t i = 0; i < kThrBins / 4; ++i) {
        const uint4 v = h[i];
        const uint32_t s4 = v.x + v.y + v.z + v.w;
        if (cum + s4 >= K.target) {
            const uint32_t b = 4 * i + (cum + v.x >= K.target ? 0u : cum + v.x + v.y >= K.target ? 1u
                                                                  : cum + v.x + v.y + v.z >= K.target ? 2u : 3u);
            atomicMin(&Wk.thr[q], b * 256 + 255);
            return;
        }
        cum += s4;
    }
}

// A query's cut for a work item of the scans (K.run_thr: tau, or the running cut), read when the
// item starts. With K.run_thr 1, the cut is first lowered from the histogram when the query has
// appended kThrEvery candidates since its last update (the item start, not the append, does it:
// there the scans hold no tables or codes in registers).
__device__ __forceinline__ uint32_t scan_cut(const Work& Wk, const KParams& K, uint32_t q, bool update = true) {
    if (!K.run_thr) return Wk.tau[q];
    if (K.run_thr == 1 && update) {
        const uint32_t c = Wk.cand_cnt[q];
        if (c >= Wk.thr_at[q] + kThrEvery) {
            Wk.thr_at[q] = c;
            thr_lower(Wk, K, q);
        }
    }
    return Wk.thr[q];
}

// One workgroup per cell (the CPU loop this replaces is src/index.rs:2231-2275). Lanes own
// members; each lane's code is loaded once per pass while groups of kG probing queries stream
// through the LDS table; survivors d <= tau of canonical members are appended per query.
// One work item: the members of cell c (entries [e0, e0 + len)) against the nqi <= kItemQ queries
// in s_q / s_t (LDS, already visible), kG per interleaved table. The member data of the first
// chunk is loaded before the tables are built so both latencies overlap.
template <int NW>
__device__ __forceinline__ void scan_item(const DevArena& A, const Work& Wk, const KParams& K, uint32_t c, uint32_t e0,
                                          uint32_t len, uint32_t nqi, uint8_t* table, const uint32_t* s_q,
                                          const uint32_t* s_t) {
    constexpr uint32_t TB = NW * 256;
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    const bool wide = nqi > 4;
    struct Member {
        Code<NW> code;
        uint32_t slot, alt;
        bool kept;
    };
    auto load_member = [&](uint32_t ebase, Member& m) {
        const uint32_t i = ebase + tid;
        const bool have = i < len;
        const uint64_t e = static_cast<uint64_t>(e0) + (have ? i : 0u);  // past the end: member 0, no output
        m.code.load(A.codes + e * (2 * NW));
        m.slot = A.members[e];
        m.alt = A.ma == 2 ? A.entry_alt[e] : kNoAlt;
        m.kept = have;
        if (K.filter) {
            const uint32_t tg = A.entry_tag[e];
            m.kept = m.kept && tg >= K.tag_lo && tg <= K.tag_hi;
        }
    };
    Member m;
    load_member(0, m);
    // interleave the item's tables: table[x*8 + g] = lut_g[x]. Per table dword x4 of the queries,
    // two 4x4 byte transposes (queries 0-3 and 4-7) give the 8-byte entries of x = 4*x4 .. 4*x4+3;
    // every word the thread needs is loaded before the first transpose (one round trip). Items of
    // at most 4 queries fill only the low half of each entry, the part their lookups read.
    {
        constexpr uint32_t X4 = (TB / 4 + kScanThreads - 1) / kScanThreads;
        auto transpose = [](const uint32_t* w, uint32_t (&o)[4]) {
            const uint32_t lo01 = __builtin_amdgcn_perm(w[1], w[0], 0x05010400u);
            const uint32_t hi01 = __builtin_amdgcn_perm(w[1], w[0], 0x07030602u);
            const uint32_t lo23 = __builtin_amdgcn_perm(w[3], w[2], 0x05010400u);
            const uint32_t hi23 = __builtin_amdgcn_perm(w[3], w[2], 0x07030602u);
            o[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
            o[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
            o[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
            o[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
        };
        uint32_t v[X4][kItemQ];
#pragma unroll
        for (uint32_t xi = 0; xi < X4; ++xi)
#pragma unroll
            for (uint32_t g = 0; g < kItemQ; ++g) {
                const uint32_t x4 = tid + xi * nt, qq = s_q[g];
                v[xi][g] = x4 < TB / 4 && qq != kNone && (g < 4 || wide)
                               ? reinterpret_cast<const uint32_t*>(Wk.lut + static_cast<uint64_t>(qq) * TB)[x4]
                               : 0u;
            }
#pragma unroll
        for (uint32_t xi = 0; xi < X4; ++xi) {
            const uint32_t x4 = tid + xi * nt;
            if (x4 >= TB / 4) continue;
            uint32_t lo[4], hi[4];
            transpose(v[xi], lo);
            transpose(v[xi] + 4, hi);
            uint4* dst = reinterpret_cast<uint4*>(table + static_cast<size_t>(x4) * 32);
            dst[0] = make_uint4(lo[0], hi[0], lo[1], hi[1]);
            dst[1] = make_uint4(lo[2], hi[2], lo[3], hi[3]);
        }
    }
    __syncthreads();
    const uint32_t lane = lane_id();
    for (uint32_t ebase = 0; ebase < len; ebase += nt) {
        if (ebase) load_member(ebase, m);
        const uint64_t e = static_cast<uint64_t>(e0) + min(ebase + tid, len - 1);
        uint32_t sums[8];
        if (wide)
            lut_sums8<NW, true>(m.code, table, sums);
        else
            lut_sums8<NW, false>(m.code, table, sums);
        // survivors, four queries at a time
        for (uint32_t h = 0; h < (wide ? 2u : 1u); ++h) {
            bool pass[kG];
            uint32_t dv[kG];
            uint64_t bm[kG];
            // the members under a query's cut-off (few), then their exactly-once tests: with two
            // homes every query's probed-bitset word is loaded before any is used
            bool under[kG];
            uint32_t pw[kG];
#pragma unroll
            for (uint32_t g = 0; g < kG; ++g) {
                const uint32_t qq = s_q[h * kG + g];
                dv[g] = A.maxk - (h ? sums[4 + g] : sums[g]);
                under[g] = m.kept && qq != kNone && dv[g] <= s_t[h * kG + g];
                pw[g] = 0;
                if (A.ma == 2 && under[g] && m.alt < c)
                    pw[g] = Wk.probed[static_cast<uint64_t>(qq) * A.MW + (m.alt >> 5)];
            }
#pragma unroll
            for (uint32_t g = 0; g < kG; ++g) {
                pass[g] = false;
                if (under[g]) {
                    if (A.ma == 2)
                        pass[g] = !(m.alt < c && ((pw[g] >> (m.alt & 31)) & 1u));
                    else
                        pass[g] = canonical(A, e, m.slot, c, Wk.probed + static_cast<uint64_t>(s_q[h * kG + g]) * A.MW);
                }
                bm[g] = __ballot(pass[g]);
            }
            // one atomic round for the four queries: lane g reserves query g's slots
            if ((bm[0] | bm[1] | bm[2] | bm[3]) == 0) continue;
            uint32_t mine = 0;
#pragma unroll
            for (uint32_t g = 0; g < kG; ++g)
                if (lane == g) mine = static_cast<uint32_t>(__popcll(bm[g]));
            uint32_t wb = 0;
            if (lane < kG && mine) wb = atomicAdd(&Wk.cand_cnt[s_q[h * kG + lane]], mine);
#pragma unroll
            for (uint32_t g = 0; g < kG; ++g) {
                const uint32_t base = __shfl(wb, static_cast<int>(g), kWave);
                const uint32_t pos = base + lanes_below(bm[g]);
                const uint32_t qq = s_q[h * kG + g];
                if (pass[g] && pos < K.cand_cap)
                    Wk.cand[static_cast<uint64_t>(qq) * K.cand_cap + pos] = make_uint2(dv[g], m.slot);
                if (pass[g] && K.run_thr == 1) atomicAdd(&Wk.dhist[static_cast<uint64_t>(qq) * kThrBins + (dv[g] >> 8)], 1u);
            }

        }
    }
    __syncthreads();  // the table and s_q / s_t are reused by the next item
}

// The cell-major scan (src/index.rs:2231-2275). Bucket mode: each work item is one cell and up
// to kBucketQ queries of its bucket, so a popular cell's items run in parallel workgroups; the grid
// strides over the items, and items of at least K.mma_min queries are left to cell_mma_kernel.
// Counting-sort mode: workgroup c scans cell c for all its queries. Either way the lookups run
// kItemQ queries at a time.
template <int NW>
__global__ void __launch_bounds__(kScanThreads, NW >= 16 ? 4 : 7)
cell_scan_kernel(DevArena A, Work Wk, KParams K) {
    constexpr uint32_t TB = NW * 256;
    __shared__ __align__(16) uint8_t table[kItemQ * TB];
    __shared__ uint32_t s_q[kItemQ], s_t[kItemQ];
    const uint32_t tid = threadIdx.x;
    if (K.bucket_cap) {
        if (!K.mma_min) {
            // every work item of kItemQ queries, grid-stride
            const uint32_t items = Wk.ctl->n_active8;
            for (uint32_t b = blockIdx.x; b < items; b += gridDim.x) {
                const uint32_t it = Wk.active8[b];
                const uint32_t c = it / kItemGroups, g0 = (it % kItemGroups) * kItemQ;
                // the cell's range, its bucket count and the item's bucket entries, in one round:
                // g0 + kItemQ <= bucket_cap (both multiples of kItemQ), so the entry reads stay in the bucket
                const uint32_t e0 = A.mem_off[c], e1 = A.mem_off[c + 1];
                const uint32_t cnt = min(Wk.cell_cnt[c], K.bucket_cap);
                const uint32_t qv = tid < kItemQ ? Wk.qbuck[static_cast<uint64_t>(c) * K.bucket_cap + g0 + tid] : kNone;
                const uint32_t nqi = min(kItemQ, cnt - g0);
                if (tid < kItemQ) {
                    const bool ok = tid < nqi;
                    s_q[tid] = ok ? qv : kNone;
                    s_t[tid] = ok ? scan_cut(Wk, K, qv) : 0u;
                }
                __syncthreads();
                scan_item<NW>(A, Wk, K, c, e0, e1 - e0, nqi, table, s_q, s_t);
            }
            return;
        }
        // with the matrix-core scan: the kItemQ groups of the work items it leaves (fewer than
        // K.mma_min queries), grid-stride over (item, group); the groups of one item run in
        // parallel workgroups. A workgroup screens its next kScanThreads of them in one round of
        // loads and keeps those it scans (groups past the item's count and items left to the
        // matrix-core scan drop out), so a skipped group costs no round trip of its own.
        constexpr uint32_t kSub = kBucketQ / kItemQ;
        __shared__ uint32_t s_list[kScanThreads], s_nl;
        const uint32_t n = Wk.ctl->n_active * kSub, lane = lane_id();
        for (uint32_t base = blockIdx.x; base < n; base += gridDim.x * kScanThreads) {
            const uint32_t v = base + tid * gridDim.x;
            bool keep = false;
            if (v < n) {
                const uint32_t it = Wk.active[v / kSub], s0 = (v % kSub) * kItemQ;
                const uint32_t c = it / kItemGroups, g0 = (it % kItemGroups) * kBucketQ;
                const uint32_t nb = min(kBucketQ, min(Wk.cell_cnt[c], K.bucket_cap) - g0);
                keep = s0 < nb && !(K.mma_min && nb >= K.mma_min);
            }
            if (tid == 0) s_nl = 0;
            __syncthreads();
            const uint64_t bm = __ballot(keep);
            uint32_t wb = 0;
            if (lane == 0 && bm) wb = atomicAdd(&s_nl, static_cast<uint32_t>(__popcll(bm)));
            wb = __shfl(wb, 0, kWave);
            if (keep) s_list[wb + lanes_below(bm)] = v;
            __syncthreads();
            const uint32_t nl = s_nl;
            for (uint32_t k = 0; k < nl; ++k) {
                const uint32_t vk = s_list[k];
                const uint32_t it = Wk.active[vk / kSub], s0 = (vk % kSub) * kItemQ;
                const uint32_t c = it / kItemGroups, g0 = (it % kItemGroups) * kBucketQ;
                // the cell's range, its bucket count and the group's bucket entries, in one round:
                // g0 + kBucketQ <= bucket_cap (both multiples of kBucketQ), so the entry reads stay in the bucket
                const uint32_t e0 = A.mem_off[c], e1 = A.mem_off[c + 1];
                const uint32_t cnt = min(Wk.cell_cnt[c], K.bucket_cap);
                const uint32_t qv = tid < kItemQ ? Wk.qbuck[static_cast<uint64_t>(c) * K.bucket_cap + g0 + s0 + tid] : kNone;
                const uint32_t nqi = min(kItemQ, min(kBucketQ, cnt - g0) - s0);
                if (tid < kItemQ) {
                    const bool ok = tid < nqi;
                    s_q[tid] = ok ? qv : kNone;
                    s_t[tid] = ok ? scan_cut(Wk, K, qv) : 0u;
                }
                __syncthreads();
                scan_item<NW>(A, Wk, K, c, e0, e1 - e0, nqi, table, s_q, s_t);
            }
            __syncthreads();  // s_list / s_nl are rewritten by the next batch
        }
    } else {
        const uint32_t c = blockIdx.x;
        if (c >= A.M) return;
        const uint32_t q0 = Wk.cell_off[c], nqc = Wk.cell_off[c + 1] - q0;
        const uint32_t e0 = A.mem_off[c], len = A.mem_off[c + 1] - e0;
        if (len == 0) return;
        for (uint32_t g0 = 0; g0 < nqc; g0 += kItemQ) {
            const uint32_t nqi = min(kItemQ, nqc - g0);
            if (tid < kItemQ) {
                const bool ok = tid < nqi;
                const uint32_t qv = ok ? Wk.qof[q0 + g0 + tid] : kNone;
                s_q[tid] = qv;
                s_t[tid] = ok ? scan_cut(Wk, K, qv) : 0u;
            }
            __syncthreads();
            scan_item<NW>(A, Wk, K, c, e0, len, nqi, table, s_q, s_t);
        }
    }
}

// ---------------------------------------------------------------- cell-major scan, matrix cores


// The cell-major scan of bucket work items with many queries (at least K.mma_min of kBucketQ) on
// the matrix cores. A member's FastScan sum is an integer dot product,
//   sum_p lut_p[n_p] = sum_p onehot(n_p) . (lut_p - 128) + 128 * npos,
// with onehot(n) the 16 bytes whose byte n is 1, so v_mfma_i32_32x32x32_i8 over K = 16 * npos
// gives exactly the integers of the table lookups (|partial sums| <= 128 * npos). Operands of
// one 32x32x32 step (two positions): A row i = member i of a 32-member tile, B column j = query j
// of the item; lanes i + 32g and j + 32g hold the 16 values of position 2s + g. Result register r
// of lane l is member 8(r/4) + 4(l/32) + r%4, query l%32.
// The four waves split K: wave w takes positions [w, w+1) * npos/4 and holds that quarter of the
// item's 32 tables in registers for the whole item; per tile the partial sums meet in LDS and wave
// w finishes members 8w .. 8w+7 for every query. Members with d <= tau go to an LDS queue that is
// settled (keep!, exactly-once, one append per query) at the item's end, or earlier when it could
// not take another tile, so these global round trips are paid per item, not per tile.
constexpr uint32_t kMmaQueue = kBucketQ * 32;  // one tile's worst case of (member, d | query << 16)
constexpr uint32_t kXcds = 8;                  // MI355X: workgroup b runs on XCD b % 8

// The matrix-core scan's work items in cell order: cell c's items c * kItemGroups + g for
// g < ceil(min(count_c, bucket_cap) / kBucketQ), the same set the seed stage opened in arrival
// order. One workgroup: a block scan of the cells' item counts, then each thread writes its cells'.
__global__ void __launch_bounds__(1024) order_items_kernel(Work Wk, KParams K, uint32_t M) {
    __shared__ uint32_t scratch[32];
    const uint32_t t = threadIdx.x, nt = blockDim.x;
    const uint32_t per = (M + nt - 1) / nt, c0 = min(t * per, M), c1 = min(c0 + per, M);
    uint32_t loc = 0;
    for (uint32_t c = c0; c < c1; ++c) loc += (min(Wk.cell_cnt[c], K.bucket_cap) + kBucketQ - 1) / kBucketQ;
    uint32_t tot;
    uint32_t pos = block_excl_scan_u32(loc, scratch, &tot);
    for (uint32_t c = c0; c < c1; ++c) {
        const uint32_t n = (min(Wk.cell_cnt[c], K.bucket_cap) + kBucketQ - 1) / kBucketQ;
        for (uint32_t g = 0; g < n; ++g) Wk.active_cs[pos++] = c * kItemGroups + g;
    }
}

template <int NW>
__global__ void __launch_bounds__(kScanThreads, NW >= 16 ? 2 : 4)
cell_mma_kernel(DevArena A, Work Wk, KParams K) {
    constexpr uint32_t TB = NW * 256;               // table bytes per query, 16 per position
    constexpr uint32_t NPOS = NW * 16;
    constexpr uint32_t SPW = NPOS / 8;              // 32x32x32 steps per wave, two positions each
    constexpr uint32_t CDW = NW >= 2 ? NW / 2 : 1;  // code dwords one wave reads per member
    constexpr uint32_t PER = kMmaQueue / kScanThreads;
    __shared__ uint32_t red[4][16][kWave];          // partial sums of one tile, by wave
    __shared__ uint2 queue[kMmaQueue];
    __shared__ uint32_t s_q[kBucketQ], s_cnt[kBucketQ], s_base[kBucketQ], s_tot[4];
    const uint32_t tid = threadIdx.x, lane = lane_id(), w = tid / kWave;
    const uint32_t g = lane >> 5, j = lane & 31;
    const uint32_t dw_lo = (w * SPW) >> 2;          // first code dword of this wave's positions
    if (tid < kBucketQ) s_cnt[tid] = 0;
    // keep!, exactly-once and the appends of the n queued survivors of cell c; every thread calls
    // it after a barrier that follows the last queue write, and it ends with a barrier
    auto settle = [&](uint32_t n, uint32_t c, uint32_t e0) {
        uint32_t slot[PER], dq[PER], off[PER];
#pragma unroll
        for (uint32_t k = 0; k < PER; ++k) {
            const uint32_t i = tid + k * kScanThreads;
            bool ok = i < n;
            const uint2 qe = ok ? queue[i] : make_uint2(0u, 0u);
            const uint64_t e = static_cast<uint64_t>(e0) + qe.x;
            dq[k] = qe.y;
            slot[k] = ok ? A.members[e] : 0u;
            if (K.filter && ok) {
                const uint32_t tg = A.entry_tag[e];
                ok = tg >= K.tag_lo && tg <= K.tag_hi;
            }
            off[k] = !ok ? kNone : A.ma == 2 ? A.entry_alt[e] : qe.x;  // the other home, or the member
        }
#pragma unroll
        for (uint32_t k = 0; k < PER; ++k) {
            if (off[k] == kNone) continue;
            const uint32_t qv = s_q[dq[k] >> 16];
            bool ok;
            if (A.ma == 2) {
                const uint32_t alt = off[k];
                ok = !(alt < c && ((Wk.probed[static_cast<uint64_t>(qv) * A.MW + (alt >> 5)] >> (alt & 31)) & 1u));
            } else {
                ok = canonical(A, static_cast<uint64_t>(e0) + off[k], slot[k], c, Wk.probed + static_cast<uint64_t>(qv) * A.MW);
            }
            off[k] = ok ? atomicAdd(&s_cnt[dq[k] >> 16], 1u) : kNone;  // rank within the query's appends
        }
        __syncthreads();
        if (tid < kBucketQ) {
            const uint32_t m = s_cnt[tid];
            const uint32_t b = m ? atomicAdd(&Wk.cand_cnt[s_q[tid]], m) : 0u;
            s_base[tid] = b;
            s_cnt[tid] = 0;
        }
        __syncthreads();
#pragma unroll
        for (uint32_t k = 0; k < PER; ++k) {
            if (off[k] == kNone) continue;
            const uint32_t jj = dq[k] >> 16, pos = s_base[jj] + off[k];
            const uint32_t dd = dq[k] & 0xFFFFu;
            if (pos < K.cand_cap) Wk.cand[static_cast<uint64_t>(s_q[jj]) * K.cand_cap + pos] = make_uint2(dd, slot[k]);
            if (K.run_thr == 1) atomicAdd(&Wk.dhist[static_cast<uint64_t>(s_q[jj]) * kThrBins + (dd >> 8)], 1u);
        }
        __syncthreads();
    };
    const uint32_t items = Wk.ctl->n_active;
    // With K.xcd_order the items come in cell order and each XCD takes a contiguous chunk of them:
    // the items one XCD runs together are then neighbouring cells, whose probing queries overlap, so
    // their tables and codes are reused from that XCD's L2. Else the grid strides over the
    // arrival-order list.
    const uint32_t* list = K.xcd_order ? Wk.active_cs : Wk.active;
    uint32_t lo = 0, hi = items, first = blockIdx.x, step = gridDim.x;
    if (K.xcd_order && gridDim.x >= kXcds) {
        const uint32_t x = blockIdx.x % kXcds;
        lo = static_cast<uint32_t>(static_cast<uint64_t>(items) * x / kXcds);
        hi = static_cast<uint32_t>(static_cast<uint64_t>(items) * (x + 1) / kXcds);
        first = lo + blockIdx.x / kXcds;
        step = (gridDim.x - x + kXcds - 1) / kXcds;  // the workgroups on this XCD
    }
    uint32_t itn = first < hi ? list[first] : 0u;  // the next item's id, one item ahead
    for (uint32_t b = first; b < hi; b += step) {
        const uint32_t it = itn;
        if (b + step < hi) itn = list[b + step];
        const uint32_t c = it / kItemGroups, g0 = (it % kItemGroups) * kBucketQ;
        const uint32_t cnt = min(Wk.cell_cnt[c], K.bucket_cap);
        const uint32_t nqi = min(kBucketQ, cnt - g0);
        if (nqi < K.mma_min) continue;
        const uint32_t e0 = A.mem_off[c], len = A.mem_off[c + 1] - e0;
        // every wave reads the item's bucket entries itself (lane j: query j), so its table loads
        // follow the bucket read directly; wave 0 also publishes them for the settle
        const uint32_t qj = j < nqi ? Wk.qbuck[static_cast<uint64_t>(c) * K.bucket_cap + g0 + j] : kNone;
        // B operands: this wave's quarter of query j's table, 128 subtracted from every byte. The
        // loads are unconditional (an empty column j reads query 0's table; its sums are never
        // kept), so all SPW of them are in flight together instead of one round trip each.
        mma_v4 bq[SPW];
        {
            const uint4* lut = reinterpret_cast<const uint4*>(Wk.lut + static_cast<uint64_t>(qj != kNone ? qj : 0u) * TB);
            uint4 v[SPW];
#pragma unroll
            for (uint32_t s = 0; s < SPW; ++s) v[s] = lut[2 * (w * SPW + s) + g];
#pragma unroll
            for (uint32_t s = 0; s < SPW; ++s)
                bq[s] = mma_v4{static_cast<int>(v[s].x ^ 0x80808080u), static_cast<int>(v[s].y ^ 0x80808080u),
                               static_cast<int>(v[s].z ^ 0x80808080u), static_cast<int>(v[s].w ^ 0x80808080u)};
        }
        // this wave's code dwords of member t*32 + j (member 0's past the cell's end: the sums of
        // those rows are never kept, and no select waits for the load)
        auto load_codes = [&](uint32_t t, uint32_t (&dw)[CDW]) {
            const uint32_t mi = t * 32 + j;
            const uint32_t* src = A.codes + static_cast<uint64_t>(e0 + (mi < len ? mi : 0u)) * (2 * NW) + dw_lo;
            if constexpr (CDW % 4 == 0) {
#pragma unroll
                for (uint32_t k = 0; k < CDW; k += 4) {
                    const uint4 v = reinterpret_cast<const uint4*>(src)[k / 4];
                    dw[k] = v.x;
                    dw[k + 1] = v.y;
                    dw[k + 2] = v.z;
                    dw[k + 3] = v.w;
                }
            } else {
#pragma unroll
                for (uint32_t k = 0; k < CDW; ++k) dw[k] = src[k];
            }
        };
        const uint32_t ntile = (len + 31) / 32;
        // three code buffers in turn, each loaded two tiles ahead (unconditionally: past the cell's
        // end the loads read member 0), so a tile waits only for its own codes: with the roles
        // rotating in code rather than by register copies, the wait counts stay exact
        uint32_t ca[CDW], cb[CDW], cc[CDW];
        load_codes(0, ca);
        load_codes(1, cb);
        // the query's cut after the tables' and codes' loads: its reads wait for those in flight
        // (the counter is in order) rather than putting a round trip between them
        const uint32_t tj = qj != kNone ? scan_cut(Wk, K, qj, w == 0) : 0u;  // wave 0 lowers the cuts
        if (tid < kBucketQ) s_q[tid] = qj;
        uint32_t n = 0;  // queued survivors (the same in every thread)
        auto tile = [&](uint32_t t, const uint32_t (&cd)[CDW]) {
            // nibble * 8 of each of this lane's positions, one per byte
            uint32_t cw8[CDW];
#pragma unroll
            for (uint32_t k = 0; k < CDW; ++k) cw8[k] = ((cd[k] >> (4 * g)) & 0x0F0F0F0Fu) << 3;
            mma_v16 acc = {};
#pragma unroll
            for (uint32_t s = 0; s < SPW; ++s) {
                const uint32_t sub = NW >= 2 ? (s & 3) : ((w * SPW + s) & 3);
                const uint32_t ld = NW >= 2 ? (s >> 2) : 0u;
                const uint32_t n8 = (cw8[ld] >> (8 * sub)) & 0xFFu;  // 8 * nibble
                const uint32_t hb = n8 >> 6;                          // nibble >= 8
                const uint64_t lo = static_cast<uint64_t>(hb ^ 1u) << (n8 & 63u);
                const uint64_t hi = static_cast<uint64_t>(hb) << (n8 & 63u);
                const mma_v4 a = {static_cast<int>(static_cast<uint32_t>(lo)), static_cast<int>(static_cast<uint32_t>(lo >> 32)),
                                  static_cast<int>(static_cast<uint32_t>(hi)), static_cast<int>(static_cast<uint32_t>(hi >> 32))};
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq[s], acc, 0, 0, 0);
            }
            __syncthreads();  // the previous tile's partial sums and survivor counts are read
#pragma unroll
            for (uint32_t r = 0; r < 16; ++r) red[w][r][lane] = static_cast<uint32_t>(acc[r]);
            __syncthreads();
            // registers 4w .. 4w+3 of every wave: members 8w + 4g + rr of the tile, query j
            uint64_t bm[4];
            uint32_t dv[4], total = 0;
#pragma unroll
            for (uint32_t rr = 0; rr < 4; ++rr) {
                const uint32_t r = 4 * w + rr;
                const uint32_t tot = red[0][r][lane] + red[1][r][lane] + red[2][r][lane] + red[3][r][lane] + 128u * NPOS;
                const uint32_t mi = t * 32 + 8 * w + 4 * g + rr;
                dv[rr] = A.maxk - tot;
                bm[rr] = __ballot(mi < len && qj != kNone && dv[rr] <= tj);
                total += static_cast<uint32_t>(__popcll(bm[rr]));
            }
            if (lane == 0) s_tot[w] = total;
            __syncthreads();
            const uint32_t t0 = s_tot[0], t1 = s_tot[1], t2 = s_tot[2], t3 = s_tot[3];
            if (n + t0 + t1 + t2 + t3 > kMmaQueue) {
                settle(n, c, e0);
                n = 0;
            }
            if (total) {
                uint32_t base = n + (w > 0 ? t0 : 0u) + (w > 1 ? t1 : 0u) + (w > 2 ? t2 : 0u);
#pragma unroll
                for (uint32_t rr = 0; rr < 4; ++rr) {
                    if ((bm[rr] >> lane) & 1u)
                        queue[base + lanes_below(bm[rr])] = make_uint2(t * 32 + 8 * w + 4 * g + rr, dv[rr] | (j << 16));
                    base += static_cast<uint32_t>(__popcll(bm[rr]));
                }
            }
            n += t0 + t1 + t2 + t3;
        };
        for (uint32_t t = 0; t < ntile; t += 3) {
            load_codes(t + 2, cc);
            tile(t, ca);
            if (t + 1 >= ntile) break;
            load_codes(t + 3, ca);
            tile(t + 1, cb);
            if (t + 2 >= ntile) break;
            load_codes(t + 4, cb);
            tile(t + 2, cc);
        }
        __syncthreads();  // the last tile's queue entries are written
        if (n) settle(n, c, e0);
        else __syncthreads();  // s_q is rewritten by the next item
    }
}

// ---------------------------------------------------------------- finish (one WG per query)

// Exact `want`-th smallest (1-based) of the n <= 64 * KPL values v (below 2^BITS, or below
// 0xFFFFFFFF for BITS = 32) held by one wave, lane-major (value r*64 + lane in v[r]; invalid ones
// are 0xFFFFFFFF, never counted: they never match a prefix whose current bit is 0), with want at
// most the number of valid values: a most-significant-bit-first radix select with ballots, no LDS
// and no barriers. Every lane returns the value.
template <int KPL, int BITS = 16>
__device__ __forceinline__ uint32_t wave_select_kth(const uint32_t (&v)[KPL], uint32_t want) {
    uint32_t prefix = 0;
#pragma unroll 1
    for (int b = BITS - 1; b >= 0; --b) {
        const uint32_t hi = prefix >> b;  // the candidate prefix with bit b = 0
        uint32_t cnt0 = 0;
#pragma unroll
        for (int r = 0; r < KPL; ++r) cnt0 += __popcll(__ballot((v[r] >> b) == hi));
        if (cnt0 < want) {
            want -= cnt0;
            prefix |= 1u << b;
        }
    }
    return prefix;
}

// The k best of n unique keys kk (ascending key: descending score, then ascending slot) into query
// qi's output row, padded with kNone / -inf. Block-wide; a list longer than the block is sorted
// in place (kk has room for n rounded up to a power of two).
__device__ __forceinline__ void write_topk(uint64_t* kk, uint32_t n, const KParams& K, uint32_t qi,
                                           uint32_t* __restrict__ out_slots, float* __restrict__ out_scores) {
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    const uint32_t kout = min(K.k, n);
    if (n <= nt) {
        // the rank of each (unique) key among the n places it directly in the output
        if (tid < n) {
            const uint64_t mine = kk[tid];
            uint32_t r = 0;
#pragma unroll 8
            for (uint32_t j = 0; j < n; ++j) r += kk[j] < mine;
            if (r < kout) {
                out_slots[static_cast<uint64_t>(qi) * K.k + r] = static_cast<uint32_t>(mine);
                out_scores[static_cast<uint64_t>(qi) * K.k + r] = key_score(mine);
            }
        }
        for (uint32_t i = kout + tid; i < K.k; i += nt) {
            out_slots[static_cast<uint64_t>(qi) * K.k + i] = kNone;
            out_scores[static_cast<uint64_t>(qi) * K.k + i] = -INFINITY;
        }
    } else {
        // an LDS list has n <= kFinishLdsCap (a power of two), so n2 fits; longer lists sort in
        // the global key buffer
        uint32_t n2 = 1;
        while (n2 < n) n2 <<= 1;
        for (uint32_t i = n + tid; i < n2; i += nt) kk[i] = kKeyMax;
        bitonic_sort_u64(kk, n2);
        for (uint32_t i = tid; i < K.k; i += nt) {
            const bool ok = i < kout;
            out_slots[static_cast<uint64_t>(qi) * K.k + i] = ok ? static_cast<uint32_t>(kk[i]) : kNone;
            out_scores[static_cast<uint64_t>(qi) * K.k + i] = ok ? key_score(kk[i]) : -INFINITY;
        }
    }
}

// Exact tie-inclusive cut at k*rerank_factor over the seed and scan candidates
// (src/index.rs:2281-2293), exact rerank (rerank_exact, :1309-1378), top-k by (score desc, slot asc).
// Up to kFinishLdsCap candidates are staged in LDS once; the cut G is then a one-wave radix
// select, and the top k of up to 256 reranked keys come from their ranks (keys are unique).
// LDS: hist[256] | scratch[32] | qs[d4] | ent[kFinishLdsCap] (d, slot) | keys[kFinishLdsCap] u64.
__device__ __forceinline__ uint32_t finish_phase(const DevArena& A, const Work& Wk, const KParams& K,
                                                 const float* __restrict__ queries, uint32_t* __restrict__ out_slots,
                                                 float* __restrict__ out_scores, uint32_t qi) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t tid = threadIdx.x, nt = blockDim.x, d = A.d, lane = lane_id();
    uint32_t* hist = reinterpret_cast<uint32_t*>(smem);
    uint32_t* scratch = hist + kHistBins;
    float* qs = reinterpret_cast<float*>(scratch + 32);
    uint2* ent = reinterpret_cast<uint2*>(qs + ((d + 3) & ~3u));
    uint64_t* keys = reinterpret_cast<uint64_t*>(ent + kFinishLdsCap);
    __shared__ uint32_t s_n, s_g;

    const uint32_t ns_cnt = Wk.seed_cnt[qi];
    const uint32_t cc = Wk.cand_cnt[qi];
    const uint32_t nc = min(cc, K.cand_cap);
    if (tid == 0) Wk.cand_n[qi] = cc;
    const uint2* seed = Wk.seed + static_cast<uint64_t>(qi) * K.seed_cap;
    const uint2* cand = Wk.cand + static_cast<uint64_t>(qi) * K.cand_cap;
    const uint32_t total = ns_cnt + nc;
    const float* q = queries + static_cast<uint64_t>(qi) * d;
    const bool sq8 = A.rerank_mode == MAIVS_RERANK_SQ8;
    const bool staged = total <= kFinishLdsCap;
    for (uint32_t j = tid; j < d; j += nt) qs[j] = sq8 ? q[j] * A.sq_step[j] : q[j];
    if (staged)
        for (uint32_t i = tid; i < total; i += nt) ent[i] = i < ns_cnt ? seed[i] : cand[i - ns_cnt];
    if (tid == 0) {
        s_n = 0;
        s_g = A.maxk;
    }
    __syncthreads();
    auto entry = [&](uint32_t i) -> uint2 { return staged ? ent[i] : (i < ns_cnt ? seed[i] : cand[i - ns_cnt]); };
    // ---- G = target-th smallest d; with fewer than target candidates every one is kept
    uint32_t cutv = A.maxk;
    if (total >= K.target) {
        if (total <= 64 * 16) {
            if (tid < kWave) {
                auto run = [&](auto kpl_tag) {
                    constexpr int KPL = decltype(kpl_tag)::value;
                    uint32_t v[KPL];
#pragma unroll
                    for (int r = 0; r < KPL; ++r) {
                        const uint32_t i = static_cast<uint32_t>(r) * 64 + lane;
                        v[r] = i < total ? ent[i].x : 0xFFFFFFFFu;
                    }
                    const uint32_t g = wave_select_kth<KPL>(v, K.target);
                    if (lane == 0) s_g = g;
                };
                if (total <= 64 * 4)
                    run(std::integral_constant<int, 4>{});
                else
                    run(std::integral_constant<int, 16>{});
            }
            __syncthreads();
            cutv = s_g;
        } else {
            cutv = select_kth(total, K.target, [&](uint32_t i) { return entry(i).x; }, hist, scratch);
        }
    }
    // ---- compaction, rerank and top-k over the key list `kk`: written once for each address space
    // (an LDS list for up to kFinishLdsCap candidates, else the global key buffer) so that every
    // access compiles to LDS or global instructions rather than generic ones
    uint2* fin = Wk.fin + static_cast<uint64_t>(qi) * K.fin_cap;
    auto tail = [&](uint64_t* kk) -> uint32_t {
        // compact the survivors into fin[] (global, read back by the debug entry point); their
        // slots go into the key list. Four rounds' entries are loaded before the first is used.
        constexpr uint32_t U = 4;
        for (uint32_t base = 0; base < total; base += U * nt) {
            uint2 e[U];
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const uint32_t i = base + u * nt + tid;
                e[u] = i < total ? entry(i) : make_uint2(0, 0);
            }
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const bool pass = base + u * nt + tid < total && e[u].x <= cutv;
                const uint64_t m = __ballot(pass);
                uint32_t wb = 0;
                if (lane == 0 && m) wb = atomicAdd(&s_n, static_cast<uint32_t>(__popcll(m)));
                wb = __shfl(wb, 0, kWave);
                if (pass) {
                    const uint32_t pos = wb + lanes_below(m);
                    fin[pos] = e[u];
                    kk[pos] = e[u].y;
                }
            }
        }
        __syncthreads();
        const uint32_t n = s_n;
        // exact rerank, 8 lanes per row
        {
            const uint32_t l = tid & 7, grp = tid >> 3, ngrp = nt >> 3;
            const uint32_t rounds = (n + ngrp - 1) / ngrp;
            const float base = sq8 ? Wk.rbase[qi] : 0.0f;
            auto slot_of = [&](uint32_t rr) {
                const uint32_t i = rr * ngrp + grp;
                return static_cast<uint32_t>(kk[i < n ? i : 0]);
            };
            auto qf = [&](uint32_t j) { return qs[j]; };
            for (uint32_t rr = 0; rr < rounds; ++rr) {
                const uint32_t i = rr * ngrp + grp;
                const uint32_t slot = slot_of(rr);
                float sc;
                if (sq8)
                    sc = base + dot_cm_u8(A.sq8 + static_cast<uint64_t>(slot) * A.cu.stride, A.cu, l, qf);
                else
                    sc = dot_cm_f32(A.vecs + static_cast<uint64_t>(slot) * A.cf.stride, A.cf, l, qf);
                if (i < n && l == 0) kk[i] = desc_score_key(sc, slot);
            }
        }
        __syncthreads();
        write_topk(kk, n, K, qi, out_slots, out_scores);
        return n;
    };
    const uint32_t n = total <= kFinishLdsCap ? tail(keys) : tail(Wk.keys + static_cast<uint64_t>(qi) * K.key_cap);
    if (tid == 0) {
        Wk.cut[qi] = cutv;
        Wk.ncand[qi] = n;
    }
    return cc;  // the candidate count, past the buffer when it overflowed
}

// The end of a pass, in its last kernel: the workgroup that finishes last copies the control block
// to its pinned host mirror and clears the per-call counters (control block, probe counts,
// candidate counts, its own count) for the next pass, so a pass needs no clearing kernel and no
// copy of its own. The control block is only ever changed by device-scope atomics; this kernel's
// one update (max_cand, when `over` is non-zero) returns before the workgroup counts itself in,
// by a data dependency rather than a device-wide fence (a fence would write back the L2 of every
// workgroup's XCD). The last workgroup reads the block with device-scope atomic loads. Other
// workgroups' candidate-count reads are done before they count themselves in, so clearing those
// counts is safe; the clears reach the next kernel at the kernel boundary.
__device__ __forceinline__ void pass_epilogue(const Work& Wk, uint32_t M, uint32_t nq, uint32_t over) {
    __shared__ uint32_t s_last;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t prev = over ? atomicMax(&Wk.ctl->max_cand, over) : 0u, zero;
        asm volatile("v_mov_b32 %0, 0" : "=v"(zero) : "v"(prev));
        s_last = atomicAdd(Wk.done + zero, 1u) == gridDim.x - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    const uint32_t t = threadIdx.x, nt = blockDim.x;
    constexpr uint32_t kWords = sizeof(Ctl) / 4;
    static_assert(kWords <= kFinishThreads, "one control word per thread");
    uint32_t* c = reinterpret_cast<uint32_t*>(Wk.ctl);
    if (t < kWords) {
        reinterpret_cast<uint32_t*>(Wk.h_ctl)[t] = __hip_atomic_load(c + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        c[t] = 0;
    }
    for (uint32_t j = t; j <= M; j += nt) Wk.cell_cnt[j] = 0;
    for (uint32_t j = t; j < nq; j += nt) Wk.cand_cnt[j] = 0;
    if (t == 0) *Wk.done = 0;
}

// NT threads per query: kFinishThreads, or kFinishWideThreads for small batches (one round of
// rerank gathers for the usual candidate lists instead of several dependent ones).
template <uint32_t NT>
__global__ void __launch_bounds__(NT, 1024 / NT)
finish_kernel(DevArena A, Work Wk, KParams K, const float* __restrict__ queries, uint32_t* __restrict__ out_slots,
              float* __restrict__ out_scores) {
    uint32_t cc = 0;
    if (blockIdx.x < K.nq) cc = finish_phase(A, Wk, K, queries, out_slots, out_scores, blockIdx.x);
    pass_epilogue(Wk, A.M, K.nq, cc > K.cand_cap ? cc : 0u);
}

// The per-query path's finish for small batches whose candidate lists the scan already cut to the
// target (the FastScan branch): every candidate is kept (finish_phase's cut keeps them all), so
// the exact rerank is spread over workgroups of kRerankRows rows, one per CU, and pq_topk_kernel
// orders each query's keys. Workgroup (g, qi) reranks candidates [g * kRerankRows, ...) of query
// qi, 8 lanes per row with the finish's dots, into Wk.keys. LDS: qs[d4].
constexpr uint32_t kRerankRows = 8;

__global__ void __launch_bounds__(kRerankRows * 8)
pq_rerank_kernel(DevArena A, Work Wk, KParams K, const float* __restrict__ queries) {
    extern __shared__ __align__(16) float qsm[];
    const uint32_t g = blockIdx.x, qi = blockIdx.y;
    if (qi >= K.nq) return;
    const uint32_t n = min(Wk.cand_cnt[qi], K.cand_cap), i0 = g * kRerankRows;
    if (i0 >= n) return;  // uniform over the workgroup
    const uint32_t tid = threadIdx.x, l = tid & 7, i = i0 + (tid >> 3);
    const bool sq8 = A.rerank_mode == MAIVS_RERANK_SQ8;
    const uint32_t slot = Wk.cand[static_cast<uint64_t>(qi) * K.cand_cap + (i < n ? i : i0)].y;
    const float* q = queries + static_cast<uint64_t>(qi) * A.d;
    for (uint32_t j = tid; j < A.d; j += blockDim.x) qsm[j] = sq8 ? q[j] * A.sq_step[j] : q[j];
    __syncthreads();
    auto qf = [&](uint32_t j) { return qsm[j]; };
    float sc;
    if (sq8)
        sc = Wk.rbase[qi] + dot_cm_u8(A.sq8 + static_cast<uint64_t>(slot) * A.cu.stride, A.cu, l, qf);
    else
        sc = dot_cm_f32(A.vecs + static_cast<uint64_t>(slot) * A.cf.stride, A.cf, l, qf);
    if (i < n && l == 0) Wk.keys[static_cast<uint64_t>(qi) * K.key_cap + i] = desc_score_key(sc, slot);
}

// The end of that finish: one workgroup per query orders its reranked keys into the output
// (write_topk), records the list, cut and count as finish_phase does (every candidate kept: the
// cut is the largest d when the list reaches the target, else maxk), then the pass epilogue.
// LDS: keys[kFinishLdsCap] u64 | scratch[32].
__global__ void __launch_bounds__(kFinishThreads)
pq_topk_kernel(DevArena A, Work Wk, KParams K, uint32_t* __restrict__ out_slots, float* __restrict__ out_scores) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint64_t* lk = reinterpret_cast<uint64_t*>(smem);
    uint32_t* scratch = reinterpret_cast<uint32_t*>(lk + kFinishLdsCap);
    uint32_t cc = 0;
    if (blockIdx.x < K.nq) {
        const uint32_t qi = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
        cc = Wk.cand_cnt[qi];
        const uint32_t n = min(cc, K.cand_cap);
        if (tid == 0) Wk.cand_n[qi] = cc;
        const uint2* cand = Wk.cand + static_cast<uint64_t>(qi) * K.cand_cap;
        uint2* fin = Wk.fin + static_cast<uint64_t>(qi) * K.fin_cap;
        uint64_t* gk = Wk.keys + static_cast<uint64_t>(qi) * K.key_cap;
        const bool staged = n <= kFinishLdsCap;
        uint32_t dmax = 0;
        for (uint32_t i = tid; i < n; i += nt) {
            const uint2 e = cand[i];
            fin[i] = e;
            dmax = max(dmax, e.x);
            if (staged) lk[i] = gk[i];
        }
        dmax = block_max_u32(dmax, scratch);  // ends with a barrier: the staged keys are visible
        if (staged)
            write_topk(lk, n, K, qi, out_slots, out_scores);
        else
            write_topk(gk, n, K, qi, out_slots, out_scores);
        if (tid == 0) {
            Wk.cut[qi] = n >= K.target ? dmax : A.maxk;
            Wk.ncand[qi] = n;
        }
    }
    pass_epilogue(Wk, A.M, K.nq, cc > K.cand_cap ? cc : 0u);
}

// Work counters of the last batch (on demand, one workgroup), from the routed lists: seed and
// scan blocks (32-vector FastScan blocks per (query, cell) pair), scan pairs, survivors, reranked
// rows.
__global__ void counters_kernel(DevArena A, Work Wk, KParams K) {
    __shared__ uint32_t scratch[32];
    unsigned long long v[5] = {0, 0, 0, 0, 0};
    for (uint32_t q = threadIdx.x; q < K.nq; q += blockDim.x) {
        const uint32_t* ch = Wk.chosen + static_cast<uint64_t>(q) * K.nprobe;
        // rest_end lies in [ns, nch] after a batched pass; clamp anyway so that no value can index
        // past the probe list, and skip unused (kNone) entries
        const uint32_t nch = min(Wk.nchosen[q], K.nprobe), ns = min(kSeedCells, nch);
        const uint32_t re = min(max(Wk.rest_end[q], ns), nch);
        for (uint32_t i = 0; i < re; ++i) {
            const uint32_t c = ch[i];
            if (c >= A.M) continue;
            const uint32_t nb = (A.mem_off[c + 1] - A.mem_off[c] + 31) / 32;
            v[i < ns ? 0 : 1] += nb;
        }
        v[2] += re > ns ? re - ns : 0u;
        v[3] += Wk.cand_n[q];
        v[4] += Wk.ncand[q];
    }
    for (int k = 0; k < 5; ++k) {
        // per-thread partials are < 2^32 for any batch the buffers can hold
        uint32_t s = block_sum_u32(static_cast<uint32_t>(v[k]), scratch);
        if (threadIdx.x == 0) (&Wk.ctl->seed_blocks)[k] = s;
    }
}

// ================================================================ the per-query path

// The reference's per-query search (search_one, src/index.rs:1381-1864, routed by route_query,
// :1168-1305): each query on its own, its probed cells scanned in probe order.

// Routing through the centroid tree (route_query's tree branch, src/index.rs:1185-1206): one wave
// per query descends the tree on the query's 1-bit code (prep) and lists up to want_c leaf cells,
// best first by Hamming, for route_phase to rescore. An empty descent lists nothing (the query
// then probes no cell, as in the reference).
constexpr uint32_t kPqTreeWaves = 4;

__host__ __device__ inline uint32_t pq_tree_lds_words(uint32_t W, uint32_t cap) {
    return 2 * W + ((W * 64 + 1 + 3) & ~3u) + (cap + 1) + (cap + 2) + cap + kTreeHCache / 2;
}

__global__ void __launch_bounds__(kPqTreeWaves * kWave)
pq_tree_kernel(DevArena A, Work Wk, KParams K, TreeDev T, const uint32_t* __restrict__ beams, uint32_t cap,
               uint32_t lds_per_wave) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t lane = lane_id(), wv = threadIdx.x / kWave;
    const uint32_t qi = blockIdx.x * kPqTreeWaves + wv;
    if (qi >= K.nq) return;  // wave-uniform; the kernel has no workgroup barrier
    uint64_t* qb = reinterpret_cast<uint64_t*>(smem + static_cast<size_t>(wv) * lds_per_wave);
    uint32_t* hist = reinterpret_cast<uint32_t*>(qb + A.W);
    uint32_t* rbase = hist + ((A.W * 64 + 1 + 3) & ~3u);
    uint32_t* rpre = rbase + cap + 1;
    uint32_t* knodes = rpre + cap + 2;
    uint16_t* hcache = reinterpret_cast<uint16_t*>(knodes + cap);
    for (uint32_t w = lane; w < A.W; w += kWave) qb[w] = Wk.qbits[static_cast<uint64_t>(qi) * A.W + w];
    wave_sync();
    const uint32_t n = tree_descent(T, beams, K.want_c, qb, A.W, hist, rbase, rpre, knodes,
                                    Wk.tlist + static_cast<uint64_t>(qi) * K.tcap, hcache, kTreeHCache);
    if (lane == 0) Wk.tcount[qi] = n;
}

// The same descent by a whole workgroup per query (block_tree_descent): the frontier's code loads
// and the selections spread over kPqTreeBlock threads instead of one wave. The top level's codes
// are staged in LDS while the query's code is read, when they fit in kTreeTopWords words.
// LDS: qb[W] u64 | hist[W*64 + 1 (4)] | rbase[cap + 1] | rpre[cap + 2] | knodes[cap] | scratch[32] |
// hcache[kTreeHCache] u16 | fr[kTreeHCache] | fid[kTreeHCache] | top[top_words] (8-byte aligned).
constexpr uint32_t kPqTreeBlock = 256;
constexpr uint32_t kTreeTopWords = 8192;  // 32 KB of top-level codes at most

__host__ __device__ inline uint32_t pq_tree_block_lds_words(uint32_t W, uint32_t cap, uint32_t top_words) {
    return ((pq_tree_lds_words(W, cap) + 32 + 2 * kTreeHCache + 1) & ~1u) + top_words;
}

__global__ void __launch_bounds__(kPqTreeBlock)
pq_tree_block_kernel(DevArena A, Work Wk, KParams K, TreeDev T, const uint32_t* __restrict__ beams, uint32_t cap,
                     uint32_t top_words) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t qi = blockIdx.x;
    if (qi >= K.nq) return;  // uniform over the workgroup
    uint64_t* qb = reinterpret_cast<uint64_t*>(smem);
    uint32_t* hist = reinterpret_cast<uint32_t*>(qb + A.W);
    uint32_t* rbase = hist + ((A.W * 64 + 1 + 3) & ~3u);
    uint32_t* rpre = rbase + cap + 1;
    uint32_t* knodes = rpre + cap + 2;
    uint32_t* scratch = knodes + cap;
    uint16_t* hcache = reinterpret_cast<uint16_t*>(scratch + 32);
    uint32_t* fr = scratch + 32 + kTreeHCache / 2;
    uint32_t* fid = fr + kTreeHCache;
    uint64_t* top = reinterpret_cast<uint64_t*>(reinterpret_cast<uint32_t*>(smem) +
                                                pq_tree_block_lds_words(A.W, cap, 0));
    for (uint32_t w = threadIdx.x; w < A.W; w += blockDim.x) qb[w] = Wk.qbits[static_cast<uint64_t>(qi) * A.W + w];
    if (top_words) {
        const uint64_t* src = T.lv_codes + static_cast<uint64_t>(T.lv_off[0]) * A.W;
        for (uint32_t i = threadIdx.x; i < top_words / 2; i += blockDim.x) top[i] = src[i];
    }
    __syncthreads();
    const uint32_t n = block_tree_descent(T, beams, K.want_c, qb, A.W, hist, rbase, rpre, knodes,
                                          Wk.tlist + static_cast<uint64_t>(qi) * K.tcap, hcache, kTreeHCache, scratch,
                                          fr, fid, kTreeHCache, top_words ? top : nullptr);
    if (threadIdx.x == 0) Wk.tcount[qi] = n;
}

// LDS of pq_front_kernel's routing workgroup after its prep region (u32 words from there): the
// tree descent's regions as pq_tree_block_kernel has them (fr, fid and top 16-byte aligned).
struct PqFrontLds {
    uint32_t hist, rbase, rpre, knodes, scratch, hcache, fr, fid, top, tcs, tcl, end;
};
// top_words: the staged top level's codes (top_n * W * 2 words), followed by its child starts and
// lengths (top_n words each)
__host__ __device__ inline PqFrontLds pq_front_layout(uint32_t W, uint32_t cap, uint32_t top_words) {
    PqFrontLds L;
    L.hist = 0;
    L.rbase = ((W * 64 + 1) + 3) & ~3u;
    L.rpre = L.rbase + cap + 1;
    L.knodes = L.rpre + cap + 2;
    L.scratch = L.knodes + cap;
    L.hcache = L.scratch + 32;
    L.fr = (L.hcache + kTreeHCache / 2 + 3) & ~3u;
    L.fid = L.fr + kTreeHCache;
    L.top = L.fid + kTreeHCache;
    const uint32_t top_n = W ? top_words / (2 * W) : 0u;
    L.tcs = L.top + top_words;
    L.tcl = L.tcs + top_n;
    L.end = L.tcl + top_n;
    return L;
}

// Byte offset of pq_front_kernel's LDS kept across its phases: cqs[d4] | leaves[tcap4] |
// bounds[kPqTreeBlock] (pq_front_keep_bytes), past both the prep + descent layout and route_phase's.
__host__ __device__ inline uint32_t pq_front_keep_off(uint32_t P, uint32_t npos, uint32_t d, uint32_t W, uint32_t Mp,
                                                      uint32_t sort_cap, uint32_t nprobe, uint32_t cap,
                                                      uint32_t top_words) {
    const uint32_t prep = 4 * (32 + P + ((npos + 3) & ~3u) + 2 * ((d + 3) & ~3u));
    const uint32_t a = prep + 4 * pq_front_layout(W, cap, top_words).end;
    const uint32_t b = static_cast<uint32_t>(route_lds_bytes(d, W, Mp, sort_cap, nprobe));
    return ((a > b ? a : b) + 15) & ~15u;
}
__host__ __device__ inline uint32_t pq_front_keep_bytes(uint32_t d, uint32_t tcap) {
    return 4 * (((d + 3) & ~3u) + ((tcap + 3) & ~3u) + kPqTreeBlock);
}

// The per-query path's prep, tree descent and route in one launch for small batches (codes over
// the whole padded dimension): two workgroups per query run side by side. Workgroup qi (qi < nq)
// computes the query's rotation and code (wave 0, prep_wave_codes) while wave 1 adds up the
// rescore base sum(q * csq_min) in index order (prep_wave_tables' order) and the other waves
// stage the tree's top level in LDS; then it descends the centroid tree (block_tree_descent) and
// routes the query (route_phase). Workgroup nq + qi computes the rotation again and the FastScan
// table and sums (prep_wave) for the scan, so the table's sequential sums are off the routing
// path. Both write the same values to qbits, cqs and cqbase. The per-call counters are clear
// beforehand (the last pass's epilogue, or a reset launch).
// LDS: codes[16] u64 | x[P] | mins[npos4] | cqp[d4] | rqp[d4] | pq_front_layout; route_phase's
// layout from offset 0 once the descent is done; past both, the query's cqs, the descent's leaf
// list and the route's bounds (pq_front_keep_off), so the route reads none of them from memory
// (keep = 0: no such region, the route reads them from memory).
template <int NW>
__global__ void __launch_bounds__(kPqTreeBlock)
pq_front_kernel(DevArena A, Work Wk, KParams K, const float* __restrict__ queries, TreeDev T,
                const uint32_t* __restrict__ beams, uint32_t cap, uint32_t top_words, uint32_t keep) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t tid = threadIdx.x, nt = blockDim.x, lane = lane_id(), wv = tid / kWave;
    uint64_t* qw = reinterpret_cast<uint64_t*>(smem);
    float* xs = reinterpret_cast<float*>(qw + 16);
    if (blockIdx.x >= K.nq) {
        const uint32_t qi = blockIdx.x - K.nq;
        if (qi < K.nq && wv == 0) prep_wave<NW>(A, Wk, queries, qi, lane, xs, qw);
        return;
    }
    const uint32_t qi = blockIdx.x;
    const uint32_t prep_words = 32 + A.P + ((A.npos + 3) & ~3u) + 2 * ((A.d + 3) & ~3u);
    uint32_t* tr = reinterpret_cast<uint32_t*>(smem) + prep_words;
    const PqFrontLds L = pq_front_layout(NW, cap, top_words);
    uint64_t* top = reinterpret_cast<uint64_t*>(tr + L.top);
    float* cqs_l = keep ? reinterpret_cast<float*>(smem + pq_front_keep_off(A.P, A.npos, A.d, NW, A.Mp, K.sort_cap,
                                                                             K.nprobe, cap, top_words))
                        : nullptr;
    uint32_t* leaves = keep ? reinterpret_cast<uint32_t*>(cqs_l + ((A.d + 3) & ~3u)) : nullptr;
    float* bounds = keep ? reinterpret_cast<float*>(leaves + ((K.tcap + 3) & ~3u)) : nullptr;
    if (wv == 0) {
        prep_wave_codes<NW>(A, Wk, queries, qi, lane, xs, qw, cqs_l);
    } else if (wv == 1) {
        float* prod = reinterpret_cast<float*>(tr + L.fr);  // free until the descent
        float base = 0.0f;
        if (A.cent_sq8 != nullptr) {
            const float* q = queries + static_cast<uint64_t>(qi) * A.d;
            // four rounds of loads in flight together (indices past d read the last coordinate)
            for (uint32_t i0 = 0; i0 < A.d; i0 += 4 * kWave) {
                float qv[4], mv[4];
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u) {
                    const uint32_t i = min(i0 + u * kWave + lane, A.d - 1);
                    qv[u] = q[i];
                    mv[u] = A.csq_min[i];
                }
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u)
                    if (i0 + u * kWave + lane < A.d) prod[i0 + u * kWave + lane] = qv[u] * mv[u];
            }
            wave_sync();
            base = seq_sum_lds(prod, A.d, 0.0f);
        }
        if (lane == 0) Wk.cqbase[qi] = base;
    } else if (K.tree_list && top_words) {
        const uint64_t* src = T.lv_codes + static_cast<uint64_t>(T.lv_off[0]) * NW;
        for (uint32_t i = tid - 2 * kWave; i < top_words / 2; i += nt - 2 * kWave) top[i] = src[i];
        const uint32_t top_n = top_words / (2 * NW);
        for (uint32_t i = tid - 2 * kWave; i < top_n; i += nt - 2 * kWave) {
            tr[L.tcs + i] = T.lv_cs[T.lv_off[0] + i];
            tr[L.tcl + i] = T.lv_cl[T.lv_off[0] + i];
        }
    }
    __syncthreads();
    uint32_t n = 0;
    if (K.tree_list) {
        n = block_tree_descent(T, beams, K.want_c, qw, NW, tr + L.hist, tr + L.rbase, tr + L.rpre, tr + L.knodes,
                               Wk.tlist + static_cast<uint64_t>(qi) * K.tcap, reinterpret_cast<uint16_t*>(tr + L.hcache),
                               kTreeHCache, tr + L.scratch, tr + L.fr, tr + L.fid, kTreeHCache, top_words ? top : nullptr,
                               top_words ? tr + L.tcs : nullptr, top_words ? tr + L.tcl : nullptr, leaves);
        if (tid == 0) Wk.tcount[qi] = n;
        __syncthreads();
    }
    route_phase<NW>(A, Wk, K, qi, cqs_l, K.tree_list && keep ? leaves : nullptr, n, bounds);
}

// want-th smallest (1-based) of the n u32 values get(i), block-wide, four 8-bit radix passes.
// Values of 0xFFFFFFFF stand for absent entries; want must not exceed the present ones.
template <class Get>
__device__ uint32_t select_kth_u32(uint32_t n, uint32_t want, Get get, uint32_t* hist, uint32_t* scratch) {
    uint32_t prefix = 0, need = want;
    for (int pass = 3; pass >= 0; --pass) {
        const uint32_t shift = 8u * static_cast<uint32_t>(pass);
        const uint32_t hi_shift = shift + 8;
        for (uint32_t i = threadIdx.x; i < kHistBins; i += blockDim.x) hist[i] = 0;
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
            const uint32_t v = get(i);
            const bool match = hi_shift >= 32 || (v >> hi_shift) == (prefix >> hi_shift);
            if (match) atomicAdd(&hist[(v >> shift) & 0xFFu], 1u);
        }
        __syncthreads();
        const uint32_t c = threadIdx.x < kHistBins ? hist[threadIdx.x] : 0u;
        uint32_t total;
        const uint32_t ex = block_excl_scan_u32(c, scratch, &total);
        const uint32_t cand = (threadIdx.x < kHistBins && ex < need && ex + c >= need) ? threadIdx.x : kNone;
        const uint32_t digit = block_min_u32(cand, scratch);
        const uint32_t below = block_sum_u32(threadIdx.x == digit ? ex : 0u, scratch);
        prefix |= digit << shift;
        need -= below;
    }
    return prefix;
}

// An entry of cell c is skipped when its slot has another home already scanned for this query: a
// multi-home vector counts only at its first-ranked probed home (the seen! rule, src/index.rs:
// 1433-1447). `scanned` is the LDS bitset of the cells before c in the probe order.
__device__ __forceinline__ bool pq_seen(const DevArena& A, uint64_t e, uint32_t slot, uint32_t c,
                                        const uint32_t* scanned) {
    if (A.ma == 2) {
        const uint32_t h = A.entry_alt[e];
        return h != kNoAlt && h != c && ((scanned[h >> 5] >> (h & 31)) & 1u);
    }
    for (uint32_t j = 0; j < A.ma; ++j) {
        const uint32_t h = A.slot_cells[static_cast<uint64_t>(slot) * A.ma + j];
        if (h != kNone && h != c && ((scanned[h >> 5] >> (h & 31)) & 1u)) return true;
    }
    return false;
}

constexpr uint32_t kPqStage = 2048;  // survivor keys staged in LDS for the final selection

// pair: the pair table's W * 1024 words (W * 4 KB) at the end
// Bucket-queue bins of the per-query scan: h = d >> 6 of the FastScan distance, or (ham) the
// Hamming distance itself, 0 .. W * 64.
__host__ __device__ inline uint32_t pq_bins(uint32_t maxk, uint32_t W, bool ham) {
    return ham ? W * 64 + 1 : (maxk >> 6) + 1;
}

// The rounds variant of the scan (small batches): up to kRoundCells probed cells at a time, with
// at most 2 * kScanRoundThreads entries together (a single larger cell makes a round of its own).
constexpr uint32_t kScanRoundThreads = 1024;
constexpr uint32_t kRoundCells = 8;
constexpr uint32_t kRoundBudget = 2 * kScanRoundThreads;
constexpr uint32_t kRoundPre = 64;  // probe ranks whose cell and member range are staged in LDS

constexpr uint32_t kSplitCells = 16;  // probe ranks replayed together by the split scan's second kernel

// mode 0: cell by cell; 1: rounds; 2: the split scan's second kernel (no tables, no pair table)
__host__ __device__ inline uint32_t pq_scan_lds_words(uint32_t MW, uint32_t maxk, uint32_t nprobe, uint32_t W = 0,
                                                      bool pair = false, bool ham = false, uint32_t mode = 0) {
    const uint32_t nbins = pq_bins(maxk, W, ham);
    const uint32_t nb4 = (nbins + 3) & ~3u;
    const uint32_t np4 = (nprobe + 1 + 3) & ~3u;
    return ((MW + 3) & ~3u) + nb4 + np4 + kHistBins + 32 + 2 * kPqStage + (pair && mode != 2 ? W * 1024 : 0u) +
           (mode == 1 ? ((MW + 3) & ~3u) + kRoundCells * nb4 + 72 + 3 * kRoundPre : 0u) +
           (mode == 2 ? kSplitCells * nb4 + np4 + 4 * kSplitCells : 0u);
}

// LDS of pq_cells_kernel: earlier[MW4] | hist[bins4] (plus its static table)
__host__ __device__ inline uint32_t pq_cells_lds_words(uint32_t MW, uint32_t maxk, uint32_t W, bool ham) {
    return ((MW + 3) & ~3u) + ((pq_bins(maxk, W, ham) + 3) & ~3u);
}

// The FastScan scan of one query (src/index.rs:1689-1757), one workgroup: cells in probe order;
// after each cell the bucket queue on h = d >> 6 lowers tau while the entries below it already
// reach the target. The reference lowers it entry by entry; its value after a cell depends only on
// the entries scanned so far (tau = min(tau, the first u with #(h <= u) >= target)), so wave 0
// recomputes it from the LDS histogram with a prefix scan after each cell, then the adaptive stop.
// The next cell's first round of member data is loaded before that barrier. Survivors h <= tau;
// the target smallest (d, slot) of them go to the candidate list for finish.
// LDS: static table[W*256] | scanned[MW4] | hist[bins4] | suffix[np4] | hist2[256] | scratch[32] |
// stage[kPqStage] u64 | pair[W*2048] u16 (K.pq_pair).
// With K.pq_pair the lookups go through a table of position pairs built from the query's table.
// HAM: the Hamming branch instead (src/index.rs:1694-1760; an index without FastScan blocks): the
// distance of a member is its Hamming distance h to the query's code, the bucket queue runs on h
// itself from tau = W * 64, the adaptive stop compares with cos(pi * tau / dp) (the host's libm
// value, A.ham_cos[tau]), and every survivor h <= tau, ties included, goes to the rerank.
// RND (small batches, kScanRoundThreads threads): the probed cells in rounds of up to kRoundCells
// scanned together. Each round admits the entries with h <= tau as it stood before the round and
// counts them per cell; the cumulative counts give each cell's tau and adaptive decision exactly
// as the cell-by-cell loop would (tau after a cell depends only on the entries of the cells up to
// it, and an entry above the round's starting tau is above every later one). The first cell that
// stops ends the scan, and the round's entries of the cells after it are dropped. The keys of a
// round carry the cell's place in the round in bits 48-55. Extra LDS after pair: rbits[MW4] (the
// round's cells) | rhist[kRoundCells * bins4] | rinfo[72] | the first kRoundPre probe ranks'
// cell, first entry and length.
// MODE 2 (SPLIT, kScanRoundThreads threads): pq_cells_kernel scored every probed cell; the bucket
// queue is replayed from the cells' histograms in probe order (kSplitCells ranks at a time, one
// wave per rank), then the survivors of the ranks up to the stop are gathered from Wk.pqe into the
// stage (and the candidate buffer). Extra LDS after stage: C[kSplitCells * bins4] | the ranks'
// entry counts[np4] | decisions[4 * kSplitCells].
template <int NW, bool HAM = false, int MODE = 0>
__global__ void __launch_bounds__(MODE ? kScanRoundThreads : kScanThreads) pq_scan_kernel(DevArena A, Work Wk, KParams K) {
    constexpr bool RND = MODE == 1, SPLIT = MODE == 2;
    constexpr uint32_t TB = NW * 256;
    __shared__ __align__(16) uint8_t table[TB];
    extern __shared__ __align__(16) uint32_t pq_smem[];
    __shared__ uint32_t s_cnt, s_tau, s_kept, s_stop, s_w, s_round, s_over;
    const uint32_t qi = blockIdx.x;
    if (qi >= K.nq) return;
    const uint32_t tid = threadIdx.x, nt = blockDim.x, lane = lane_id();
    const uint32_t nbins = pq_bins(A.maxk, NW, HAM);
    auto bucket = [](uint32_t dv) { return HAM ? dv : dv >> 6; };
    uint32_t qd[2 * NW];
    if constexpr (HAM) {
        const uint32_t* qb = reinterpret_cast<const uint32_t*>(Wk.qbits + static_cast<uint64_t>(qi) * NW);
#pragma unroll
        for (int j = 0; j < 2 * NW; ++j) qd[j] = qb[j];
    }
    uint32_t* scanned = pq_smem;
    uint32_t* hist = scanned + ((A.MW + 3) & ~3u);
    float* suffix = reinterpret_cast<float*>(hist + ((nbins + 3) & ~3u));
    uint32_t* hist2 = reinterpret_cast<uint32_t*>(suffix + ((K.nprobe + 1 + 3) & ~3u));
    uint32_t* scratch = hist2 + kHistBins;
    uint64_t* stage = reinterpret_cast<uint64_t*>(scratch + 32);  // 8-byte aligned: every region is a multiple of 16 bytes
    uint16_t* pair = reinterpret_cast<uint16_t*>(stage + kPqStage);
    const uint32_t nb4 = (nbins + 3) & ~3u;
    uint32_t* rbits = reinterpret_cast<uint32_t*>(pair) + (K.pq_pair ? NW * 1024 : 0u);
    uint32_t* rhist = rbits + ((A.MW + 3) & ~3u);
    uint32_t* rinfo = rhist + kRoundCells * nb4;
    uint32_t* rc = rinfo;         // the round's cells
    uint32_t* re0 = rinfo + 8;    // their first entries
    uint32_t* roff = rinfo + 16;  // their offsets in the round's entry order (9)
    uint32_t* rn = rinfo + 25;    // entries admitted per cell
    uint32_t* rtau = rinfo + 33;
    uint32_t* rkept = rinfo + 41;
    uint32_t* rstop = rinfo + 49;
    uint32_t* rflag = rinfo + 57;
    uint32_t* pc = rinfo + 72;    // probe ranks < kRoundPre: cell, first entry, length
    uint32_t* pe0 = pc + kRoundPre;
    uint32_t* plen = pe0 + kRoundPre;
    if (!HAM && !SPLIT) {
        const uint4* src = reinterpret_cast<const uint4*>(Wk.lut + static_cast<uint64_t>(qi) * TB);
        for (uint32_t i = tid; i < TB / 16; i += nt) reinterpret_cast<uint4*>(table)[i] = src[i];
    }
    if (!HAM && !SPLIT && K.pq_pair) {
        // entry p*256 + (a | b << 4) = table[2p][a] + table[2p+1][b], two entries per thread per step
        __syncthreads();
        for (uint32_t i = 2 * tid; i < NW * 2048; i += 2 * nt) {
            const uint32_t pp = i >> 8, a = i & 15, b = (i >> 4) & 15;
            const uint32_t hi = table[(2 * pp + 1) * 16 + b];
            const uint32_t v0 = table[2 * pp * 16 + a] + hi, v1 = table[2 * pp * 16 + a + 1] + hi;
            *reinterpret_cast<uint32_t*>(pair + i) = v0 | (v1 << 16);
        }
    }
    for (uint32_t i = tid; i < A.MW; i += nt) scanned[i] = 0;
    for (uint32_t i = tid; i < nbins; i += nt) hist[i] = 0;
    const uint32_t nch = Wk.nchosen[qi];
    const uint32_t* chosen = Wk.chosen + static_cast<uint64_t>(qi) * K.nprobe;
    if constexpr (RND) {
        for (uint32_t i = tid; i < A.MW; i += nt) rbits[i] = 0;
        if (tid >= kWave && tid < kWave + kRoundPre) {
            const uint32_t r = tid - kWave;
            if (r < nch) {
                const uint32_t c = chosen[r];
                const uint32_t e0 = A.mem_off[c];
                pc[r] = c;
                pe0[r] = e0;
                plen[r] = A.mem_off[c + 1] - e0;
            }
        }
    }
    uint32_t* sC = reinterpret_cast<uint32_t*>(stage + kPqStage);  // SPLIT: kSplitCells x bins4
    uint32_t* sN = sC + kSplitCells * nb4;                         // SPLIT: entry count of each rank
    uint32_t* sD = sN + ((K.nprobe + 1 + 3) & ~3u);                // SPLIT: tau, kept, stop, flag per rank
    // SPLIT: the first kSplitCells ranks' counts of bin tid, and the first entries of rank (wave), in
    // flight through the setup
    uint32_t pre_h[kSplitCells];
    uint64_t pre_e[4];
    if constexpr (SPLIT) {
        const uint64_t qr = static_cast<uint64_t>(qi) * K.nprobe;
        for (uint32_t r = tid; r < nch; r += nt) sN[r] = Wk.pqn[qr + r];
#pragma unroll
        for (uint32_t j = 0; j < kSplitCells; ++j)
            pre_h[j] = j < nch && tid < nbins ? Wk.pqh[(qr + j) * nb4 + tid] : 0u;
        const uint32_t wv = tid / kWave, room = min(K.pq_room, 4u * kWave);
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t i = u * kWave + lane;
            pre_e[u] = wv < nch && i < room ? Wk.pqe[(qr + wv) * K.pq_room + i] : 0ull;
        }
    }
    const float delta = Wk.delta[qi], bias = Wk.bias[qi];
    // suffix maxima of the reachability bounds (src/index.rs:1466-1489), suffix[nch] = -inf: wave 0,
    // 64 probe ranks at a time from the end
    if (K.adaptive && tid < kWave) {
        const float* bnd = Wk.bnd + static_cast<uint64_t>(qi) * K.nprobe;
        float carry = -INFINITY;
        for (int32_t base = static_cast<int32_t>((nch + kWave - 1) / kWave) * kWave - kWave; base >= 0; base -= kWave) {
            const uint32_t i = static_cast<uint32_t>(base) + lane;
            float v = i < nch ? bnd[i] : -INFINITY;
            for (int o = 1; o < kWave; o <<= 1) {
                const float y = __shfl_down(v, o, kWave);
                if (lane + o < kWave) v = fmaxf(v, y);
            }
            v = fmaxf(v, carry);
            if (i < nch) suffix[i] = v;
            carry = __shfl(v, 0, kWave);
        }
        if (lane == 0) suffix[nch] = -INFINITY;
    }
    if (tid == 0) {
        s_cnt = 0;
        s_tau = HAM ? NW * 64 : A.maxk >> 6;
        s_kept = 0;
        s_stop = 0;
    }
    uint64_t* cbuf = Wk.pqc + static_cast<uint64_t>(qi) * K.pq_cap;
    const uint32_t target = K.target;
    bool flagged = false;
    // The bucket queue (src/index.rs:1712-1724), by one wave: from c = #(h <= t0) and the counts
    // h[0 .. t0], tau = min(t0, the first u with #(h <= u) >= target) and #(h <= tau). The walk
    // goes down from t0, 64 bins per step: lane l holds bin t - l, and an inclusive scan gives
    // #(h <= t - l - 1) = c - (the bins t - l .. t).
    auto walk = [&](const uint32_t* h, uint32_t t0, uint32_t c, uint32_t& t_out, uint32_t& kept_out) {
        uint32_t t = t0, kept = c;
        if (c >= target) {
            for (;;) {
                const int32_t bi = static_cast<int32_t>(t) - static_cast<int32_t>(lane);
                const uint32_t hv = bi >= 0 ? h[bi] : 0u;
                uint32_t incl = wave_incl_scan_u32(hv);
                // the walk stops at the first bin u = t - l whose lower neighbour's count
                // #(h <= u - 1) falls below the target (bin 0's lower count is 0)
                const uint64_t stopm = __ballot(bi >= 0 && c - incl < target);
                if (stopm) {
                    const int l = __ffsll(static_cast<long long>(stopm)) - 1;
                    const uint32_t below = __shfl(incl - hv, l, kWave);  // the bins t - l + 1 .. t
                    t = t - static_cast<uint32_t>(l);
                    kept = c - below;
                    break;
                }
                c -= __shfl(incl, kWave - 1, kWave);
                t -= kWave;
            }
        }
        t_out = t;
        kept_out = kept;
    };
    // the adaptive stop after a cell (:1727-1733), tau t with kept entries at or below it, and the
    // suffix maximum sx of the bounds of the cells after it; flag: the comparison is within the
    // host-check band
    auto adaptive_stop = [&](uint32_t t, uint32_t kept, float sx, bool& flag) -> bool {
        if (!K.adaptive || kept < target) return false;
        float thr;
        if constexpr (HAM) {
            thr = A.ham_cos[t];  // score_to_cos(hamming_score(tau)), src/index.rs:1782-1786
        } else {
            const uint32_t top = ((t + 1) << 6) - 1;
            const uint32_t worst = A.maxk > top ? A.maxk - top : 0u;
            const float est = delta * static_cast<float>(worst) + bias;
            thr = fminf(fmaxf(est / K.norm, -1.0f), 1.0f);
        }
        const float T = thr - K.at_margin;
        if (!K.pq_noflag && fabsf(sx - T) <= K.prune_band) flag = true;
        return sx < T;
    };
    // keeps the entries with h <= t (in place, in order) and sets s_cnt to their number
    auto compact_to = [&](uint32_t t) {
        const uint32_t n = s_cnt;
        __syncthreads();
        if (tid == 0) s_w = 0;
        __syncthreads();
        for (uint32_t base = 0; base < n; base += nt) {
            const uint32_t i = base + tid;
            const uint64_t key = i < n ? cbuf[i] : 0ull;
            const bool keepit = i < n && bucket(static_cast<uint32_t>(key >> 32) & 0xFFFFu) <= t;
            uint32_t tot;
            const uint32_t off = block_excl_scan_u32(keepit ? 1u : 0u, scratch, &tot);
            if (keepit) cbuf[s_w + off] = key;
            __syncthreads();
            if (tid == 0) s_w += tot;
            __syncthreads();
        }
        if (tid == 0) s_cnt = s_w;
        __syncthreads();
    };
    // one member's data; the first round of the next cell is loaded ahead
    struct Mem {
        Code<NW> code;
        uint32_t slot, alt, tag;
        bool have;
    };
    auto load_mem = [&](uint32_t e0, uint32_t len, uint32_t base, Mem& m) {
        const uint32_t i = base + tid;
        m.have = i < len;
        if (m.have) {
            const uint64_t e = static_cast<uint64_t>(e0) + i;
            m.code.load(A.codes + e * (2 * NW));
            m.slot = A.members[e];
            m.alt = A.ma == 2 ? A.entry_alt[e] : 0u;
            m.tag = K.filter ? A.entry_tag[e] : 0u;
        }
    };
    Mem nxt;
    nxt.have = false;
    // The probe list in a three-stage pipeline, so that no cell waits on its own id or range: a
    // cell's id is read two cells ahead, its member range one cell ahead, and its first round of
    // member data before the previous cell's barrier.
    uint32_t c_cur = 0, e0_cur = 0, len_cur = 0;  // this cell
    uint32_t c_n1 = 0, e0_n1 = 0, len_n1 = 0;     // the next one
    uint32_t c_n2 = 0;                            // the one after
    if (!RND && nch > 0) {
        c_cur = chosen[0];
        e0_cur = A.mem_off[c_cur];
        len_cur = A.mem_off[c_cur + 1] - e0_cur;
        load_mem(e0_cur, len_cur, 0, nxt);
    }
    if (!RND && nch > 1) {
        c_n1 = chosen[1];
        e0_n1 = A.mem_off[c_n1];
        len_n1 = A.mem_off[c_n1 + 1] - e0_n1;
    }
    if (!RND && nch > 2) c_n2 = chosen[2];
    __syncthreads();
    // #(h <= tau) over every admitted entry, and s_cnt when it was last counted in (wave 0 keeps
    // both; s_cnt is read only where no admission is in flight: after a cell's barrier, after a
    // compaction)
    uint32_t cum = 0, cnt_prev = 0;
    if constexpr (SPLIT) {
        const uint32_t wv = tid / kWave;
        const uint64_t qr = static_cast<uint64_t>(qi) * K.nprobe;
        uint32_t r0 = 0, last = nch;  // ranks below last are scanned
        while (r0 < nch) {
            const uint32_t nr = min(nch - r0, kSplitCells), tau0 = s_tau;
            // C[j][b] = hist[b] + the counts of ranks r0 .. r0 + j, for the bins up to tau0 (the
            // others no longer count); bin b by thread b (nbins <= nt)
            if (tid <= tau0) {
                const uint32_t b = tid;
                uint32_t v[kSplitCells];
#pragma unroll
                for (uint32_t j = 0; j < kSplitCells; ++j)
                    v[j] = r0 == 0 ? pre_h[j] : j < nr ? Wk.pqh[(qr + r0 + j) * nb4 + b] : 0u;
                uint32_t acc = hist[b];
#pragma unroll
                for (uint32_t j = 0; j < kSplitCells; ++j) {
                    acc += v[j];
                    if (j < nr) sC[j * nb4 + b] = acc;
                }
            }
            __syncthreads();
            // each rank's tau and adaptive decision, one wave per rank
            for (uint32_t j = wv; j < nr; j += nt / kWave) {
                // tau = min(tau0, the first u with #(h <= u) >= target), by one forward pass: lane l
                // holds bins [l * bpl, (l + 1) * bpl) up to tau0, an inclusive scan of their sums
                // finds the lane where the count reaches the target, and that lane walks its bins
                const uint32_t* cj = sC + j * nb4;
                const uint32_t bpl = (tau0 + kWave) / kWave;
                const uint32_t b0 = min(lane * bpl, tau0 + 1), b1 = min(b0 + bpl, tau0 + 1);
                uint32_t mine = 0;
                for (uint32_t b = b0; b < b1; ++b) mine += cj[b];
                uint32_t incl = wave_incl_scan_u32(mine);
                const uint32_t c = __shfl(incl, kWave - 1, kWave);
                uint32_t t = tau0, kept = c;
                const uint64_t hm = __ballot(incl >= target);
                if (c >= target) {
                    const int L = __ffsll(static_cast<long long>(hm)) - 1;
                    uint32_t tl = 0, kl = 0;
                    if (lane == static_cast<uint32_t>(L)) {
                        uint32_t cum = incl - mine;
                        for (uint32_t b = b0; b < b1; ++b) {
                            cum += cj[b];
                            if (cum >= target) {
                                tl = b;
                                kl = cum;
                                break;
                            }
                        }
                    }
                    t = __shfl(tl, L, kWave);
                    kept = __shfl(kl, L, kWave);
                }
                bool flag = false;
                const bool stp = adaptive_stop(t, kept, suffix[r0 + j + 1], flag);
                if (lane == 0) {
                    sD[j] = t;
                    sD[kSplitCells + j] = kept;
                    sD[2 * kSplitCells + j] = stp ? 1u : 0u;
                    sD[3 * kSplitCells + j] = flag ? 1u : 0u;
                }
            }
            __syncthreads();
            // the first rank that stops is the last one scanned (every wave finds it by ballot)
            const uint64_t stopm = __ballot(lane < nr && sD[2 * kSplitCells + lane] != 0);
            const uint32_t js = stopm ? static_cast<uint32_t>(__ffsll(static_cast<long long>(stopm)) - 1) : nr - 1;
            const uint32_t stp = stopm ? 1u : 0u;
            const uint64_t flagm = __ballot(lane <= js && sD[3 * kSplitCells + lane] != 0);
            if (tid == 0) {
                flagged = flagged || flagm != 0;
                s_tau = sD[js];
                s_stop = stp;
            }
            for (uint32_t b = tid; b <= tau0; b += nt) hist[b] = sC[js * nb4 + b];
            __syncthreads();
            if (stp) {
                last = r0 + js + 1;
                break;
            }
            r0 += nr;
        }
        // the survivors (h <= tau) of the scanned ranks, a wave per rank with four entries per lane
        // in flight: into the stage and the candidate buffer
        const uint32_t tfin = s_tau;
        if (tid == 0) s_cnt = 0;
        __syncthreads();
        for (uint32_t r = wv; r < last; r += nt / kWave) {
            const uint32_t n_r = sN[r];
            const uint64_t* src = Wk.pqe + (qr + r) * K.pq_room;
            for (uint32_t i0 = 0; i0 < n_r; i0 += 4 * kWave) {
                uint64_t v[4];
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u) {
                    const uint32_t i = i0 + u * kWave + lane;
                    v[u] = r == wv && i0 == 0 ? pre_e[u] : i < n_r ? src[i] : 0ull;
                }
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u) {
                    const uint32_t i = i0 + u * kWave + lane;
                    const bool ok = i < n_r && bucket(static_cast<uint32_t>(v[u] >> 32) & 0xFFFFu) <= tfin;
                    const uint64_t bm = __ballot(ok);
                    if (!bm) continue;
                    uint32_t wb = 0;
                    if (lane == 0) wb = atomicAdd(&s_cnt, static_cast<uint32_t>(__popcll(bm)));
                    wb = __shfl(wb, 0, kWave);
                    if (ok) {
                        const uint32_t pos = wb + lanes_below(bm);
                        if (pos < kPqStage) stage[pos] = v[u];
                        if (pos < K.pq_cap) cbuf[pos] = v[u];
                    }
                }
            }
        }
        __syncthreads();
        if (tid == 0 && s_cnt > K.pq_cap) {
            s_stop = 2;
            s_over = s_cnt;
        }
    } else if constexpr (RND) {
        // ---- rounds of up to kRoundCells cells (cum: #(h <= s_tau) over every admitted entry)
        const uint32_t wv = tid / kWave;
        uint32_t r0 = 0;
        while (r0 < nch) {
            // the round: the cells from rank r0 whose entries stay within the budget (at least one)
            if (tid < kWave) {
                const uint32_t j = lane, rk = r0 + j;
                const bool have = j < kRoundCells && rk < nch;
                uint32_t c = 0, e0 = 0, len = 0;
                if (have) {
                    if (rk < kRoundPre) {
                        c = pc[rk];
                        e0 = pe0[rk];
                        len = plen[rk];
                    } else {
                        c = chosen[rk];
                        e0 = A.mem_off[c];
                        len = A.mem_off[c + 1] - e0;
                    }
                }
                uint32_t incl = wave_incl_scan_u32(len);
                // a prefix of the lanes: have and the running total are both monotone in j
                const bool fits = have && (j == 0 || incl <= kRoundBudget);
                const uint32_t nr = static_cast<uint32_t>(__popcll(__ballot(fits)));
                if (j < nr) {
                    rc[j] = c;
                    re0[j] = e0;
                    roff[j] = incl - len;
                    rn[j] = 0;
                    atomicOr(&rbits[c >> 5], 1u << (c & 31));
                }
                if (j + 1 == nr) roff[nr] = incl;
                if (lane == 0) s_round = nr;
            }
            for (uint32_t i = tid; i < kRoundCells * nb4; i += nt) rhist[i] = 0;
            __syncthreads();
            const uint32_t nr = s_round, total = roff[nr], tau0 = s_tau;
            // room for the round's entries: drop the entries above tau, else the buffer grows (host)
            if (s_cnt + total > K.pq_cap) {
                compact_to(tau0);
                if (s_cnt + total > K.pq_cap) {
                    if (tid == 0) {
                        s_stop = 2;
                        s_over = s_cnt + total;
                    }
                    break;
                }
            }
            const uint32_t round_base = s_cnt;
            // the round's entries, concatenated in rank order, nt at a time; admitted: h <= tau0.
            // Two chunks' member data are loaded before the first is used (a round has at most two
            // chunks unless one cell alone is larger); one for the widest codes (registers).
            constexpr uint32_t kCh = NW >= 16 ? 1 : 2;
            for (uint32_t base0 = 0; base0 < total; base0 += kCh * nt) {
                Code<NW> code[kCh];
                uint32_t jv[kCh], slot[kCh], alt[kCh], tag[kCh];
#pragma unroll
                for (uint32_t u = 0; u < kCh; ++u) {
                    const uint32_t i = base0 + u * nt + tid;
                    uint32_t j = 0;
#pragma unroll
                    for (uint32_t r = 1; r < kRoundCells; ++r) j += (r < nr && roff[r] <= i) ? 1u : 0u;
                    jv[u] = j;
                    slot[u] = alt[u] = tag[u] = 0u;
                    if (i < total) {
                        const uint64_t e = static_cast<uint64_t>(re0[j]) + (i - roff[j]);
                        code[u].load(A.codes + e * (2 * NW));
                        slot[u] = A.members[e];
                        alt[u] = A.ma == 2 ? A.entry_alt[e] : 0u;
                        tag[u] = K.filter ? A.entry_tag[e] : 0u;
                    }
                }
#pragma unroll
                for (uint32_t u = 0; u < kCh; ++u) {
                    const uint32_t i = base0 + u * nt + tid;
                    const uint32_t j = jv[u];
                    bool ok = false;
                    uint32_t dv = 0;
                    if (i < total) {
                        const uint32_t c = rc[j];
                        if constexpr (HAM)
                            dv = code_hamming<NW>(code[u], qd);
                        else
                            dv = A.maxk - (K.pq_pair ? lut_sum_pair<NW>(code[u], pair) : lut_sum1<NW>(code[u], table));
                        if (bucket(dv) <= tau0) {
                            ok = !K.filter || (tag[u] >= K.tag_lo && tag[u] <= K.tag_hi);
                            // the first-ranked probed home counts (src/index.rs:1433-1447): homes in
                            // earlier rounds, or earlier in this one
                            auto seen = [&](uint32_t h) {
                                if (h == c) return false;
                                if ((scanned[h >> 5] >> (h & 31)) & 1u) return true;
                                if (!((rbits[h >> 5] >> (h & 31)) & 1u)) return false;
                                for (uint32_t r = 0; r < j; ++r)
                                    if (rc[r] == h) return true;
                                return false;
                            };
                            if (ok && A.ma == 2) {
                                ok = !(alt[u] != kNoAlt && seen(alt[u]));
                            } else if (ok && A.ma > 2) {
                                for (uint32_t hj = 0; hj < A.ma && ok; ++hj) {
                                    const uint32_t h = A.slot_cells[static_cast<uint64_t>(slot[u]) * A.ma + hj];
                                    if (h != kNone && seen(h)) ok = false;
                                }
                            }
                        }
                    }
                    const uint64_t bm = __ballot(ok);
                    if (bm) {
                        uint32_t wb = 0;
                        if (lane == 0) wb = atomicAdd(&s_cnt, static_cast<uint32_t>(__popcll(bm)));
                        wb = __shfl(wb, 0, kWave);
                        if (ok) {
                            const uint32_t pos = wb + lanes_below(bm);
                            if (pos < K.pq_cap)
                                cbuf[pos] = (static_cast<uint64_t>(j) << 48) | (static_cast<uint64_t>(dv) << 32) | slot[u];
                            atomicAdd(&rhist[j * nb4 + bucket(dv)], 1u);
                        }
                        // admissions per cell: j does not decrease over the wave's lanes
                        const uint32_t jlo = __shfl(j, 0, kWave), jhi = __shfl(j, kWave - 1, kWave);
                        for (uint32_t jj = jlo; jj <= jhi; ++jj) {
                            const uint32_t cnt = static_cast<uint32_t>(__popcll(__ballot(ok && j == jj)));
                            if (lane == 0 && cnt) atomicAdd(&rn[jj], cnt);
                        }
                    }
                }
            }
            __syncthreads();
            // cumulative counts through each cell of the round: rhist[j][b] = hist[b] + the round's
            // cells 0 .. j
            for (uint32_t b = tid; b < nbins; b += nt) {
                uint32_t acc = hist[b];
                for (uint32_t r = 0; r < nr; ++r) {
                    acc += rhist[r * nb4 + b];
                    rhist[r * nb4 + b] = acc;
                }
            }
            __syncthreads();
            // each cell's tau and adaptive decision, one wave per cell
            for (uint32_t j = wv; j < nr; j += nt / kWave) {
                uint32_t c = cum;
                for (uint32_t r = 0; r <= j; ++r) c += rn[r];
                uint32_t t, kept;
                walk(rhist + j * nb4, tau0, c, t, kept);
                bool flag = false;
                const bool stp = adaptive_stop(t, kept, suffix[r0 + j + 1], flag);
                if (lane == 0) {
                    rtau[j] = t;
                    rkept[j] = kept;
                    rstop[j] = stp ? 1u : 0u;
                    rflag[j] = flag ? 1u : 0u;
                }
            }
            __syncthreads();
            // the first cell that stops is the last one scanned
            uint32_t js = nr - 1, stp = 0;
            for (uint32_t r = 0; r < nr; ++r) {
                if (rstop[r]) {
                    js = r;
                    stp = 1;
                    break;
                }
            }
            if (tid == 0) {
                for (uint32_t r = 0; r <= js; ++r) flagged = flagged || rflag[r] != 0;
                s_tau = rtau[js];
                s_stop = stp;
            }
            cum = rkept[js];
            for (uint32_t b = tid; b < nbins; b += nt) hist[b] = rhist[js * nb4 + b];
            if (tid < nr) {
                const uint32_t c = rc[tid];
                atomicAnd(&rbits[c >> 5], ~(1u << (c & 31)));
                if (tid <= js) atomicOr(&scanned[c >> 5], 1u << (c & 31));
            }
            if (stp && js + 1 < nr) {
                // drop the round's entries of the cells after js (the round has two cells or more,
                // so at most kRoundBudget entries: two per thread)
                const uint32_t n_r = s_cnt - round_base;
                uint64_t v[2];
                bool kp[2];
#pragma unroll
                for (uint32_t u = 0; u < 2; ++u) {
                    const uint32_t i = tid + u * nt;
                    v[u] = i < n_r ? cbuf[round_base + i] : 0ull;
                    kp[u] = i < n_r && static_cast<uint32_t>(v[u] >> 48) <= js;
                }
                __syncthreads();
                if (tid == 0) s_w = round_base;
                __syncthreads();
#pragma unroll
                for (uint32_t u = 0; u < 2; ++u)
                    if (kp[u]) cbuf[atomicAdd(&s_w, 1u)] = v[u];
                __syncthreads();
                if (tid == 0) s_cnt = s_w;
            }
            __syncthreads();
            if (s_stop) break;
            r0 += nr;
        }
    } else {
    for (uint32_t ci_i = 0; ci_i < nch; ++ci_i) {
        const uint32_t c = c_cur, e0 = e0_cur, len = len_cur;
        const uint32_t tau = s_tau;
        for (uint32_t base = 0; base < len; base += nt) {
            Mem m;
            if (base == 0)
                m = nxt;
            else
                load_mem(e0, len, base, m);
            bool ok = false;
            uint32_t dv = 0;
            if (m.have) {
                const uint64_t e = static_cast<uint64_t>(e0) + base + tid;
                if constexpr (HAM)
                    dv = code_hamming<NW>(m.code, qd);
                else
                    dv = A.maxk - (K.pq_pair ? lut_sum_pair<NW>(m.code, pair) : lut_sum1<NW>(m.code, table));
                if (bucket(dv) <= tau) {
                    ok = !K.filter || (m.tag >= K.tag_lo && m.tag <= K.tag_hi);
                    if (ok && A.ma > 1) {
                        if (A.ma == 2)
                            ok = !(m.alt != kNoAlt && m.alt != c && ((scanned[m.alt >> 5] >> (m.alt & 31)) & 1u));
                        else
                            ok = !pq_seen(A, e, m.slot, c, scanned);
                    }
                }
            }
            // one counter update per wave
            const uint64_t bm = __ballot(ok);
            if (bm) {
                uint32_t wb = 0;
                if (lane == 0) wb = atomicAdd(&s_cnt, static_cast<uint32_t>(__popcll(bm)));
                wb = __shfl(wb, 0, kWave);
                if (ok) {
                    const uint32_t pos = wb + lanes_below(bm);
                    if (pos < K.pq_cap) cbuf[pos] = (static_cast<uint64_t>(dv) << 32) | m.slot;
                    atomicAdd(&hist[bucket(dv)], 1u);
                }
            }
        }
        // the next cell's first round, in flight across the barrier and the bucket-queue update;
        // the range of the cell after it and the id of the third
        nxt.have = false;
        if (ci_i + 1 < nch) load_mem(e0_n1, len_n1, 0, nxt);
        c_cur = c_n1;
        e0_cur = e0_n1;
        len_cur = len_n1;
        if (ci_i + 2 < nch) {
            c_n1 = c_n2;
            e0_n1 = A.mem_off[c_n1];
            len_n1 = A.mem_off[c_n1 + 1] - e0_n1;
        }
        if (ci_i + 3 < nch) c_n2 = chosen[ci_i + 3];
        __syncthreads();
        if (tid < kWave) {
            // hist only grows by entries with h <= tau and tau only falls, so #(h <= tau) is carried
            // from cell to cell (cum, plus this cell's admissions)
            cum += s_cnt - cnt_prev;
            cnt_prev = s_cnt;
            uint32_t t, kept;
            walk(hist, tau, cum, t, kept);
            cum = kept;
            uint32_t stop = adaptive_stop(t, kept, suffix[ci_i + 1], flagged) ? 1u : 0u;
            if (s_cnt > K.pq_cap) stop = 2;
            if (lane == 0) {
                s_tau = t;
                s_kept = kept;
                s_stop = stop;
                scanned[c >> 5] |= 1u << (c & 31);
            }
        }
        __syncthreads();
        if (s_stop == 2) break;
        // room for the next cell: drop the entries above tau
        if (s_stop == 0 && ci_i + 1 < nch && s_cnt + K.pq_room > K.pq_cap) {
            compact_to(s_tau);
            if (tid == 0 && s_cnt + K.pq_room > K.pq_cap) s_stop = 2;  // the next cell might not fit
            __syncthreads();
            cnt_prev = s_cnt;  // the entries above tau are gone; cum is unchanged
            if (s_stop == 2) break;
        }
        if (s_stop) break;
    }
    }
    __syncthreads();
    if (tid == 0) {
        if (s_stop == 2) atomicMax(&Wk.ctl->pq_overflow, MODE ? s_over : s_cnt + K.pq_room);
    }
    if (tid == 0 && flagged) Wk.flag_prune[atomicAdd(&Wk.ctl->nflag_prune, 1u)] = qi;
    uint2* cand = Wk.cand + static_cast<uint64_t>(qi) * K.cand_cap;
    if (s_stop == 2) {
        if (tid == 0) {
            Wk.cand_cnt[qi] = 0;
            Wk.seed_cnt[qi] = 0;
        }
        return;
    }
    if constexpr (RND) {
        // a round admits against the tau before it: keep the survivors (h <= tau) alone, so the
        // selection below sees about as many entries as the cell-by-cell loop leaves
        if (s_cnt > target) compact_to(s_tau);
    }
    // survivors h <= tau; the target smallest (d, slot) when more (src/index.rs:1743-1757; ties at
    // the cut by ascending slot)
    const uint32_t n = s_cnt, t = s_tau;
    // the keys in LDS when they fit (every pass below reads them), with all of a thread's loads in flight
    const bool staged = n <= kPqStage;
    if (staged && !SPLIT) {  // the split scan gathered its survivors into the stage already
        constexpr uint32_t PER = kPqStage / kScanThreads;
        uint64_t v[PER];
#pragma unroll
        for (uint32_t k = 0; k < PER; ++k) {
            const uint32_t i = tid + k * nt;
            v[k] = i < n ? cbuf[i] : 0ull;
        }
#pragma unroll
        for (uint32_t k = 0; k < PER; ++k) {
            const uint32_t i = tid + k * nt;
            if (i < n) stage[i] = v[k];
        }
        __syncthreads();
    }
    auto key = [&](uint32_t i) -> uint64_t { return staged ? stage[i] : cbuf[i]; };
    auto surv_d = [&](uint32_t i) -> uint32_t {
        const uint32_t dv = static_cast<uint32_t>(key(i) >> 32) & 0xFFFFu;
        return bucket(dv) <= t ? dv : 0xFFFFFFFFu;
    };
    if (staged) {
        // wave 0 alone: the survivors' d (and slots) in registers, KPL per lane for the smallest KPL
        // that holds them, both cuts by ballot radix selects, and the compaction by ballots; the
        // other waves are done
        auto wave_end = [&](auto kpl) {
            constexpr uint32_t KPL = decltype(kpl)::value;
            uint32_t dv[KPL];
            uint32_t m = 0;
#pragma unroll
            for (uint32_t r = 0; r < KPL; ++r) {
                const uint32_t i = r * kWave + lane;
                dv[r] = i < n ? surv_d(i) : 0xFFFFFFFFu;
                m += static_cast<uint32_t>(__popcll(__ballot(dv[r] != 0xFFFFFFFFu)));
            }
            uint32_t dcut = 0xFFFFFFFFu, scut = 0xFFFFFFFFu;
            if (!HAM && m > target) {
                dcut = wave_select_kth<KPL>(dv, target);
                uint32_t below = 0, eq = 0;
#pragma unroll
                for (uint32_t r = 0; r < KPL; ++r) {
                    below += static_cast<uint32_t>(__popcll(__ballot(dv[r] < dcut)));
                    eq += static_cast<uint32_t>(__popcll(__ballot(dv[r] == dcut)));
                }
                if (eq > target - below) {
                    // ties at the cut by ascending slot
                    uint32_t sv[KPL];
#pragma unroll
                    for (uint32_t r = 0; r < KPL; ++r)
                        sv[r] = dv[r] == dcut ? static_cast<uint32_t>(stage[r * kWave + lane]) : 0xFFFFFFFFu;
                    scut = wave_select_kth<KPL, 32>(sv, target - below);
                }
            }
            uint32_t w = 0;
#pragma unroll
            for (uint32_t r = 0; r < KPL; ++r) {
                const uint32_t i = r * kWave + lane;
                const uint32_t slot = i < n ? static_cast<uint32_t>(stage[i]) : 0u;
                const bool take = dv[r] != 0xFFFFFFFFu && (dv[r] < dcut || (dv[r] == dcut && slot <= scut));
                const uint64_t bm = __ballot(take);
                if (take && w + lanes_below(bm) < K.cand_cap) cand[w + lanes_below(bm)] = make_uint2(dv[r], slot);
                w += static_cast<uint32_t>(__popcll(bm));
            }
            if (lane == 0) {
                Wk.cand_cnt[qi] = w;
                Wk.seed_cnt[qi] = 0;
            }
        };
        if (tid < kWave) {
            if (n <= 4 * kWave)
                wave_end(std::integral_constant<uint32_t, 4>{});
            else if (n <= 16 * kWave)
                wave_end(std::integral_constant<uint32_t, 16>{});
            else
                wave_end(std::integral_constant<uint32_t, kPqStage / kWave>{});
        }
        return;
    }
    uint32_t m = 0;
    for (uint32_t i = tid; i < n; i += nt) m += surv_d(i) != 0xFFFFFFFFu;
    m = block_sum_u32(m, scratch);
    uint32_t dcut = 0xFFFFFFFFu, scut = 0xFFFFFFFFu;
    if (!HAM && m > target) {
        dcut = select_kth(n, target, [&](uint32_t i) { const uint32_t v = surv_d(i); return v == 0xFFFFFFFFu ? 0xFFFFu : v; },
                          hist2, scratch);
        uint32_t below = 0;
        for (uint32_t i = tid; i < n; i += nt) below += surv_d(i) < dcut;
        below = block_sum_u32(below, scratch);
        scut = select_kth_u32(n, target - below,
                              [&](uint32_t i) { return surv_d(i) == dcut ? static_cast<uint32_t>(key(i)) : 0xFFFFFFFFu; },
                              hist2, scratch);
    }
    if (tid == 0) s_w = 0;
    __syncthreads();
    for (uint32_t base = 0; base < n; base += nt) {
        const uint32_t i = base + tid;
        bool take = false;
        uint2 e = make_uint2(0, 0);
        if (i < n) {
            const uint32_t dv = surv_d(i);
            const uint32_t slot = static_cast<uint32_t>(key(i));
            take = dv != 0xFFFFFFFFu && (dv < dcut || (dv == dcut && slot <= scut));
            e = make_uint2(dv, slot);
        }
        uint32_t tot;
        const uint32_t off = block_excl_scan_u32(take ? 1u : 0u, scratch, &tot);
        if (take && s_w + off < K.cand_cap) cand[s_w + off] = e;
        __syncthreads();
        if (tid == 0) s_w += tot;
        __syncthreads();
    }
    if (tid == 0) {
        Wk.cand_cnt[qi] = s_w;
        Wk.seed_cnt[qi] = 0;
    }
}

// The split scan's first kernel (small batches): one workgroup per (probe rank, query) scores
// the probed cell's members against the query's FastScan table (or by Hamming distance, HAM) and
// admits those the tag filter and the first-ranked-home rule keep (src/index.rs:1433-1447: a home
// at a lower probe rank was scanned before), with no threshold. It writes them (d << 32 | slot) at
// rank * pq_room in the query's region of Wk.pqe, their histogram over the bucket-queue bins to
// Wk.pqh and their count to Wk.pqn; pq_scan_kernel<NW, HAM, 2> replays the bucket queue from these.
// The nibble tables serve the lookups: a cell's few hundred members do not repay a pair table.
// LDS: static table[W*256] | earlier[MW4] (the cells at lower ranks) | hist[bins4].
template <int NW, bool HAM = false>
__global__ void __launch_bounds__(kScanThreads) pq_cells_kernel(DevArena A, Work Wk, KParams K) {
    constexpr uint32_t TB = NW * 256;
    __shared__ __align__(16) uint8_t table[TB];
    extern __shared__ __align__(16) uint32_t pc_smem[];
    __shared__ uint32_t s_n;
    const uint32_t r = blockIdx.x, qi = blockIdx.y;
    if (qi >= K.nq) return;
    const uint32_t nch = Wk.nchosen[qi];
    if (r >= nch) return;  // uniform over the workgroup
    const uint32_t tid = threadIdx.x, nt = blockDim.x, lane = lane_id();
    const uint32_t nbins = pq_bins(A.maxk, NW, HAM), nb4 = (nbins + 3) & ~3u;
    auto bucket = [](uint32_t dv) { return HAM ? dv : dv >> 6; };
    const uint32_t* chosen = Wk.chosen + static_cast<uint64_t>(qi) * K.nprobe;
    const uint32_t c = chosen[r];
    const uint32_t e0 = A.mem_off[c], len = A.mem_off[c + 1] - e0;
    uint32_t* earlier = pc_smem;
    uint32_t* hist = earlier + ((A.MW + 3) & ~3u);
    // one member's data; the first chunk's is in flight while the tables are set up
    Code<NW> code;
    uint32_t slot = 0, alt = 0, tag = 0;
    auto load = [&](uint32_t i) {
        if (i < len) {
            const uint64_t e = static_cast<uint64_t>(e0) + i;
            code.load(A.codes + e * (2 * NW));
            slot = A.members[e];
            alt = A.ma == 2 ? A.entry_alt[e] : 0u;
            tag = K.filter ? A.entry_tag[e] : 0u;
        }
    };
    load(tid);
    uint32_t qd[2 * NW];
    if constexpr (HAM) {
        const uint32_t* qb = reinterpret_cast<const uint32_t*>(Wk.qbits + static_cast<uint64_t>(qi) * NW);
#pragma unroll
        for (int j = 0; j < 2 * NW; ++j) qd[j] = qb[j];
    } else {
        const uint4* src = reinterpret_cast<const uint4*>(Wk.lut + static_cast<uint64_t>(qi) * TB);
        for (uint32_t i = tid; i < TB / 16; i += nt) reinterpret_cast<uint4*>(table)[i] = src[i];
    }
    for (uint32_t i = tid; i < A.MW; i += nt) earlier[i] = 0;
    for (uint32_t i = tid; i < nbins; i += nt) hist[i] = 0;
    if (tid == 0) s_n = 0;
    __syncthreads();
    for (uint32_t i = tid; i < r; i += nt) {
        const uint32_t h = chosen[i];
        atomicOr(&earlier[h >> 5], 1u << (h & 31));
    }
    __syncthreads();
    auto seen = [&](uint32_t h) { return h != c && ((earlier[h >> 5] >> (h & 31)) & 1u); };
    uint64_t* out = Wk.pqe + (static_cast<uint64_t>(qi) * K.nprobe + r) * K.pq_room;
    for (uint32_t base = 0; base < len; base += nt) {
        const uint32_t i = base + tid;
        if (base > 0) load(i);
        bool ok = false;
        uint32_t dv = 0;
        if (i < len) {
            if constexpr (HAM)
                dv = code_hamming<NW>(code, qd);
            else
                dv = A.maxk - lut_sum1<NW>(code, table);
            ok = !K.filter || (tag >= K.tag_lo && tag <= K.tag_hi);
            if (ok && A.ma == 2) {
                ok = !(alt != kNoAlt && seen(alt));
            } else if (ok && A.ma > 2) {
                for (uint32_t hj = 0; hj < A.ma && ok; ++hj) {
                    const uint32_t h = A.slot_cells[static_cast<uint64_t>(slot) * A.ma + hj];
                    if (h != kNone && seen(h)) ok = false;
                }
            }
        }
        const uint64_t bm = __ballot(ok);
        if (bm) {
            uint32_t wb = 0;
            if (lane == 0) wb = atomicAdd(&s_n, static_cast<uint32_t>(__popcll(bm)));
            wb = __shfl(wb, 0, kWave);
            if (ok) {
                out[wb + lanes_below(bm)] = (static_cast<uint64_t>(dv) << 32) | slot;
                atomicAdd(&hist[bucket(dv)], 1u);
            }
        }
    }
    __syncthreads();
    uint32_t* gh = Wk.pqh + (static_cast<uint64_t>(qi) * K.nprobe + r) * nb4;
    for (uint32_t b = tid; b < nb4; b += nt) gh[b] = b < nbins ? hist[b] : 0u;
    if (tid == 0) Wk.pqn[static_cast<uint64_t>(qi) * K.nprobe + r] = s_n;
}

}  // namespace maivs_dev
