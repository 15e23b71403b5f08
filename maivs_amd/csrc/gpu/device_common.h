// Device-side helpers shared by the search kernels: wave64 reductions, block scans, bitonic
// sort of 64-bit keys, and the exact f32 arithmetic the reference's CPU path uses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace maivs_dev {

constexpr int kWave = 64;
constexpr uint32_t kNone = 0xFFFFFFFFu;
constexpr uint64_t kKeyMax = ~0ull;

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// Number of set lanes of `mask` below this lane.
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// The value of lane (lane ^ M) for M a power of two below 64, without the LDS crossbar where the
// wave's DPP row permutations reach: M = 1, 2 a quad permutation; 4 = half-row mirror then quad
// reversal (i ^ 7 ^ 3); 8 = row mirror then half-row mirror (i ^ 15 ^ 7); 16 a swizzle within 32
// lanes (xor mask 16); 32 a permute. Every lane of the wave must be active.
template <int M>
__device__ __forceinline__ float xor_lanes(float x) {
    static_assert(M >= 1 && M <= 32 && (M & (M - 1)) == 0, "a lane distance of 1, 2, 4, 8, 16 or 32");
    const int v = __float_as_int(x);
    int r;
    if constexpr (M == 1)
        r = __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);
    else if constexpr (M == 2)
        r = __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);
    else if constexpr (M == 4)
        r = __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true), 0x1B, 0xF, 0xF, true);
    else if constexpr (M == 8)
        r = __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true), 0x141, 0xF, 0xF, true);
    else if constexpr (M == 16)
        r = __builtin_amdgcn_ds_swizzle(v, 0x401F);
    else
        r = __shfl_xor(v, 32, kWave);
    return __int_as_float(r);
}

// Inclusive prefix sum over the wave's 64 lanes without the LDS crossbar: row shifts by 1, 2, 4
// and 8 lanes scan each row of 16, then row 15's total is broadcast into rows 1 and 3 and lane
// 31's into rows 2 and 3. Every lane of the wave must be active.
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t x) {
    int v = static_cast<int>(x);
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
    return static_cast<uint32_t>(v);
}

// lane ^ M's value of a 32-bit integer (xor_lanes)
template <int M>
__device__ __forceinline__ uint32_t xor_lanes_u32(uint32_t x) {
    return __float_as_uint(xor_lanes<M>(__uint_as_float(x)));
}

// Whole-wave reductions by lane exchanges at distances 32 .. 1 (every lane active)
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
    v += xor_lanes_u32<32>(v);
    v += xor_lanes_u32<16>(v);
    v += xor_lanes_u32<8>(v);
    v += xor_lanes_u32<4>(v);
    v += xor_lanes_u32<2>(v);
    v += xor_lanes_u32<1>(v);
    return v;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, xor_lanes_u32<32>(v));
    v = min(v, xor_lanes_u32<16>(v));
    v = min(v, xor_lanes_u32<8>(v));
    v = min(v, xor_lanes_u32<4>(v));
    v = min(v, xor_lanes_u32<2>(v));
    v = min(v, xor_lanes_u32<1>(v));
    return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, xor_lanes_u32<32>(v));
    v = max(v, xor_lanes_u32<16>(v));
    v = max(v, xor_lanes_u32<8>(v));
    v = max(v, xor_lanes_u32<4>(v));
    v = max(v, xor_lanes_u32<2>(v));
    v = max(v, xor_lanes_u32<1>(v));
    return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, xor_lanes<32>(v));
    v = fmaxf(v, xor_lanes<16>(v));
    v = fmaxf(v, xor_lanes<8>(v));
    v = fmaxf(v, xor_lanes<4>(v));
    v = fmaxf(v, xor_lanes<2>(v));
    v = fmaxf(v, xor_lanes<1>(v));
    return v;
}

// Block-wide reductions through LDS `scratch` (>= blockDim/64 entries). All threads get the result.
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t* scratch) {
    v = wave_sum_u32(v);
    const uint32_t w = threadIdx.x / kWave, nw = (blockDim.x + kWave - 1) / kWave;
    __syncthreads();
    if (lane_id() == 0) scratch[w] = v;
    __syncthreads();
    uint32_t s = 0;
    for (uint32_t i = 0; i < nw; ++i) s += scratch[i];
    __syncthreads();
    return s;
}
__device__ __forceinline__ uint32_t block_min_u32(uint32_t v, uint32_t* scratch) {
    v = wave_min_u32(v);
    const uint32_t w = threadIdx.x / kWave, nw = (blockDim.x + kWave - 1) / kWave;
    __syncthreads();
    if (lane_id() == 0) scratch[w] = v;
    __syncthreads();
    uint32_t s = kNone;
    for (uint32_t i = 0; i < nw; ++i) s = min(s, scratch[i]);
    __syncthreads();
    return s;
}
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* scratch) {
    v = wave_max_u32(v);
    const uint32_t w = threadIdx.x / kWave, nw = (blockDim.x + kWave - 1) / kWave;
    __syncthreads();
    if (lane_id() == 0) scratch[w] = v;
    __syncthreads();
    uint32_t s = 0;
    for (uint32_t i = 0; i < nw; ++i) s = max(s, scratch[i]);
    __syncthreads();
    return s;
}
__device__ __forceinline__ float block_max_f32(float v, float* scratch) {
    v = wave_max_f32(v);
    const uint32_t w = threadIdx.x / kWave, nw = (blockDim.x + kWave - 1) / kWave;
    __syncthreads();
    if (lane_id() == 0) scratch[w] = v;
    __syncthreads();
    float s = -INFINITY;
    for (uint32_t i = 0; i < nw; ++i) s = fmaxf(s, scratch[i]);
    __syncthreads();
    return s;
}

// Exclusive prefix sum of one value per thread, block-wide; returns the total in *total.
__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, uint32_t* scratch, uint32_t* total) {
    const uint32_t lane = lane_id(), w = threadIdx.x / kWave, nw = (blockDim.x + kWave - 1) / kWave;
    const uint32_t x = wave_incl_scan_u32(v);
    __syncthreads();
    if (lane == kWave - 1) scratch[w] = x;
    __syncthreads();
    uint32_t before = 0, all = 0;
    for (uint32_t i = 0; i < nw; ++i) {
        if (i < w) before += scratch[i];
        all += scratch[i];
    }
    __syncthreads();
    *total = all;
    return before + x - v;
}

// The bitonic network of bitonic_sort_u64 for n = KPT * blockDim.x keys (blockDim.x a multiple of
// 64): thread t holds elements t*KPT .. t*KPT + KPT - 1 in registers. Partners closer than KPT are
// in the thread, closer than 64*KPT in the wave (shuffles); only the wider stages go through LDS,
// so most of the network needs no barrier. Element i keeps min(i, i ^ stride) when i is the lower
// of the pair and the run (i & size) ascends, or when it is the upper and the run descends.
template <int KPT>
__device__ __forceinline__ void bitonic_sort_u64_regs(uint64_t* keys, uint32_t n) {
    const uint32_t t = threadIdx.x;
    uint64_t v[KPT];
    __syncthreads();
#pragma unroll
    for (int e = 0; e < KPT; ++e) v[e] = keys[t * KPT + e];
    for (uint32_t size = 2; size <= n; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            if (stride < static_cast<uint32_t>(KPT)) {
#pragma unroll
                for (int e = 0; e < KPT; ++e) {
#pragma unroll
                    for (int f = e + 1; f < KPT; ++f) {
                        if (static_cast<uint32_t>(e ^ f) != stride) continue;
                        const bool up = ((t * KPT + e) & size) == 0;
                        const uint64_t a = v[e], b = v[f];
                        if ((a > b) == up) {
                            v[e] = b;
                            v[f] = a;
                        }
                    }
                }
            } else if (stride < 64u * KPT) {
                const int ld = static_cast<int>(stride / KPT);  // lane distance of the partner
#pragma unroll
                for (int e = 0; e < KPT; ++e) {
                    const uint32_t i = t * KPT + e;
                    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v[e]), ld, 64);
                    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v[e] >> 32), ld, 64);
                    const uint64_t o = (static_cast<uint64_t>(hi) << 32) | lo;
                    const bool keep_min = ((i & stride) == 0) == ((i & size) == 0);
                    v[e] = keep_min ? (o < v[e] ? o : v[e]) : (o > v[e] ? o : v[e]);
                }
            } else {
                __syncthreads();
#pragma unroll
                for (int e = 0; e < KPT; ++e) keys[t * KPT + e] = v[e];
                __syncthreads();
#pragma unroll
                for (int e = 0; e < KPT; ++e) {
                    const uint32_t i = t * KPT + e;
                    const uint64_t o = keys[i ^ stride];
                    const bool keep_min = ((i & stride) == 0) == ((i & size) == 0);
                    v[e] = keep_min ? (o < v[e] ? o : v[e]) : (o > v[e] ? o : v[e]);
                }
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < KPT; ++e) keys[t * KPT + e] = v[e];
    __syncthreads();
}

// Ascending bitonic sort of n = power-of-two 64-bit keys (LDS or global), block-wide. With n = 1 or
// 2 times the block size (a multiple of 64) the network runs mostly in registers. (At 8 keys per
// thread the shuffles cost more than the barriers they save: measured 127k against 91k cycles.)
__device__ __forceinline__ void bitonic_sort_u64(uint64_t* keys, uint32_t n) {
    const uint32_t nt = blockDim.x;
    if (nt % 64 == 0) {
        if (n == nt) return bitonic_sort_u64_regs<1>(keys, n);
        if (n == 2 * nt) return bitonic_sort_u64_regs<2>(keys, n);
    }
    for (uint32_t size = 2; size <= n; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (uint32_t t = threadIdx.x; t < n / 2; t += blockDim.x) {
                uint32_t lo = 2 * t - (t & (stride - 1));
                uint32_t hi = lo + stride;
                bool up = (lo & size) == 0;
                uint64_t a = keys[lo], b = keys[hi];
                if ((a > b) == up) {
                    keys[lo] = b;
                    keys[hi] = a;
                }
            }
        }
    }
    __syncthreads();
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

// Order-preserving key of an f32 for DESCENDING score, ties broken by the low 32 bits
// (the id, ascending). -0.0 and +0.0 compare equal in the reference, so they share a key.
__device__ __forceinline__ uint64_t desc_score_key(float s, uint32_t id) {
    uint32_t b = __float_as_uint(s == 0.0f ? 0.0f : s);
    uint32_t asc = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (static_cast<uint64_t>(~asc) << 32) | id;
}
__device__ __forceinline__ float key_score(uint64_t key) {
    uint32_t asc = ~static_cast<uint32_t>(key >> 32);
    uint32_t b = (asc & 0x80000000u) ? (asc & 0x7FFFFFFFu) : ~asc;
    return __uint_as_float(b);
}

// 8-lane FMA dot with the hsum order ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) and a sequential
// tail, computed by the 8 consecutive lanes of a group (lane l of the group owns acc_l).
// Every lane of the group returns the full result. `a` is indexed by element, `b` likewise.
template <class LoadA, class LoadB>
__device__ __forceinline__ float dot8_group(uint32_t n, uint32_t l, LoadA la, LoadB lb) {
    float acc = 0.0f;
    uint32_t n8 = n & ~7u;
    for (uint32_t i = l; i < n8; i += 8) acc = __builtin_fmaf(la(i), lb(i), acc);
    float a4 = __shfl_xor(acc, 4, 8);     // partner l^4
    float s = acc + a4;                   // lanes 0..3: a_l + a_{l+4}
    float s2 = __shfl_xor(s, 2, 8);       // partner l^2
    float t = (l & 2) ? (s2 + s) : (s + s2);  // lanes 0,1: (a0+a4)+(a2+a6), (a1+a5)+(a3+a7)
    float t1 = __shfl_xor(t, 1, 8);
    float r = (l & 1) ? (t1 + t) : (t + t1);
    for (uint32_t i = n8; i < n; ++i) r += la(i) * lb(i);
    return r;
}

}  // namespace maivs_dev
