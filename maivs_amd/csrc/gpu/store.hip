// libmaivs_gpu.so, the row store: the index's per-slot rows kept in HBM through the build, and the
// build steps that read them there (no counterpart in the reference, whose rows live in host
// memory; each step restates the reference's arithmetic bit for bit):
//   store_write       placement's rows, written at their slots (add_batch, src/index.rs:3077-3199)
//   cell sums         add_batch's primary sums, input order within a cell (:2643-2667, 3186-3196)
//   store_radii       recompute_radii's member dots and their order statistics (:817-861)
//   store_compact     compact_arena's row moves and FastScan packing (:929-1112,
//                     src/quantize.rs:238-265)
#include <hip/hip_runtime.h>

#include <rocprim/device/device_radix_sort.hpp>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <vector>

#include "ctx.h"
#include "device_common.h"
#include "store.h"

using namespace maivs_host;
using namespace maivs_dev;

namespace {

constexpr uint32_t kStoreThreads = 256;

// ---------------------------------------------------------------- kernels

// Rows i of the placed batch into the store at slots[i] (each present array of the layout).
__global__ void __launch_bounds__(kStoreThreads)
store_scatter_kernel(const float* __restrict__ x, const uint64_t* __restrict__ bits, const int8_t* __restrict__ codes,
                     const uint32_t* __restrict__ slots, uint32_t n, uint32_t d, uint32_t W, float* __restrict__ sf,
                     uint64_t* __restrict__ sb, int8_t* __restrict__ sc) {
    for (uint32_t i = blockIdx.x; i < n; i += gridDim.x) {
        const uint64_t s = slots[i];
        if (sf)
            for (uint32_t j = threadIdx.x; j < d; j += blockDim.x) sf[s * d + j] = x[static_cast<uint64_t>(i) * d + j];
        if (sc)
            for (uint32_t j = threadIdx.x; j < d; j += blockDim.x) sc[s * d + j] = codes[static_cast<uint64_t>(i) * d + j];
        if (sb)
            for (uint32_t w = threadIdx.x; w < W; w += blockDim.x) sb[s * W + w] = bits[static_cast<uint64_t>(i) * W + w];
    }
}

// Sort input of the primary sums: key = vector i's primary home, value = i.
__global__ void primary_key_kernel(const uint32_t* __restrict__ homes, uint32_t ma, uint32_t n, uint32_t* __restrict__ key,
                                   uint32_t* __restrict__ pos) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        key[i] = homes[static_cast<uint64_t>(i) * ma];
        pos[i] = i;
    }
}

__global__ void zero_u32_kernel(uint32_t* __restrict__ p, uint32_t n) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

// [start, end) of every key's run in the sorted keys (keys without a run keep 0, 0).
__global__ void run_bounds_kernel(const uint32_t* __restrict__ skey, uint32_t n, uint32_t* __restrict__ start,
                                  uint32_t* __restrict__ end) {
    for (uint32_t p = blockIdx.x * blockDim.x + threadIdx.x; p < n; p += gridDim.x * blockDim.x) {
        const uint32_t k = skey[p];
        if (p == 0 || skey[p - 1] != k) start[k] = p;
        if (p + 1 == n || skey[p + 1] != k) end[k] = p + 1;
    }
}

// One workgroup per cell: each dimension's running sum takes the cell's vectors in input order,
// one f32 add each, from the sum it had (the reference's `*sv += x`).
__global__ void __launch_bounds__(kStoreThreads)
cell_sum_kernel(const float* __restrict__ x, const uint32_t* __restrict__ spos, const uint32_t* __restrict__ start,
                const uint32_t* __restrict__ end, uint32_t d, float* __restrict__ sums) {
    const uint32_t c = blockIdx.x, s0 = start[c], s1 = end[c];
    if (s0 >= s1) return;
    for (uint32_t j = threadIdx.x; j < d; j += blockDim.x) {
        float acc = sums[static_cast<uint64_t>(c) * d + j];
        constexpr uint32_t kAhead = 8;
        for (uint32_t t = s0; t < s1; t += kAhead) {
            float v[kAhead];
#pragma unroll
            for (uint32_t q = 0; q < kAhead; ++q) {
                const uint32_t tt = min(t + q, s1 - 1);
                v[q] = x[static_cast<uint64_t>(spos[tt]) * d + j];
            }
#pragma unroll
            for (uint32_t q = 0; q < kAhead; ++q)
                if (t + q < s1) acc = acc + v[q];
        }
        sums[static_cast<uint64_t>(c) * d + j] = acc;
    }
}

// Order-preserving u32 key of an f32 (ascending), and back.
__device__ __forceinline__ uint32_t asc_key(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_f32(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

struct RadiiArgs {
    const uint32_t* mem_off;
    const uint32_t* members;
    const float* cents;
    const float* sq_min;
    const float* sq_step;
    const float* rows;    // store f32 rows (mode 0)
    const int8_t* codes;  // store i8 / SQ8 rows (modes 1, 2)
    uint32_t* keys;       // mem_off[M]: the clamped dots' keys
    float* p99;
    float* mn;
    uint32_t M, d, mode;
    float inv;
};

// One workgroup of 256 threads per cell: the members' dots with the centroid by 8-lane groups in
// the reference's FMA order for the mode (src/index.rs:817-846), clamped to [-1, 1]; then the
// (p99 + 1)-th largest by a four-pass radix select over their keys, and the smallest.
// LDS: w[d] (mode 1: sq_step * centroid).
__global__ void __launch_bounds__(kStoreThreads) radii_kernel(RadiiArgs a) {
    extern __shared__ float w[];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t scratch[16];
    __shared__ float s_base;
    const uint32_t c = blockIdx.x, tid = threadIdx.x, d = a.d;
    const uint32_t e0 = a.mem_off[c], len = a.mem_off[c + 1] - e0;
    if (len == 0) {
        if (tid == 0) {
            a.p99[c] = 0.0f;
            a.mn[c] = 0.0f;
        }
        return;
    }
    const float* mu = a.cents + static_cast<uint64_t>(c) * d;
    if (a.mode == 1) {
        for (uint32_t j = tid; j < d; j += blockDim.x) w[j] = a.sq_step[j] * mu[j];
        if (tid == 0) {
            // the reference's iterator sum from -0.0, one product and one add per term
            float b = -0.0f;
            for (uint32_t j = 0; j < d; ++j) {
                const float p = a.sq_min[j] * mu[j];
                b = b + p;
            }
            s_base = b;
        }
    }
    __syncthreads();
    const float base = a.mode == 1 ? s_base : 0.0f;
    const uint32_t l = tid & 7, g = tid >> 3, ngrp = blockDim.x >> 3;
    for (uint32_t i0 = 0; i0 < len; i0 += ngrp) {
        const uint32_t i = i0 + g;
        const uint64_t off = static_cast<uint64_t>(a.members[e0 + min(i, len - 1)]) * d;
        float dot;
        if (a.mode == 0) {
            const float* r = a.rows + off;
            dot = dot8_group(d, l, [&](uint32_t j) { return mu[j]; }, [&](uint32_t j) { return r[j]; });
        } else if (a.mode == 1) {
            const uint8_t* r = reinterpret_cast<const uint8_t*>(a.codes + off);
            dot = dot8_group(d, l, [&](uint32_t j) { return w[j]; }, [&](uint32_t j) { return static_cast<float>(r[j]); }) +
                  base;
        } else {
            const int8_t* r = a.codes + off;
            dot = dot8_group(d, l, [&](uint32_t j) { return mu[j]; }, [&](uint32_t j) { return static_cast<float>(r[j]); }) *
                  a.inv;
        }
        // clamp(-1, 1) as max then min
        const float cl = dot < -1.0f ? -1.0f : dot;
        const float cv = 1.0f < cl ? 1.0f : cl;
        if (i < len && l == 0) a.keys[e0 + i] = asc_key(cv);
    }
    __syncthreads();
    // p99 = min(ceil(len * 0.99) - 1, len - 1) in f32, saturating at 0 (src/index.rs:849-851)
    const uint32_t up = static_cast<uint32_t>(ceilf(static_cast<float>(len) * 0.99f));
    const uint32_t p99 = min(up > 0 ? up - 1 : 0u, len - 1);
    uint32_t prefix = 0, need = len - p99;  // the (p99 + 1)-th largest is the (len - p99)-th smallest
    for (int pass = 3; pass >= 0; --pass) {
        const uint32_t shift = 8u * static_cast<uint32_t>(pass);
        hist[tid] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < len; i += blockDim.x) {
            const uint32_t v = a.keys[e0 + i];
            if (pass == 3 || (v >> (shift + 8)) == (prefix >> (shift + 8))) atomicAdd(&hist[(v >> shift) & 0xFFu], 1u);
        }
        __syncthreads();
        const uint32_t cnt = hist[tid];
        uint32_t total;
        const uint32_t ex = block_excl_scan_u32(cnt, scratch, &total);
        const uint32_t digit = block_min_u32(ex < need && ex + cnt >= need ? tid : kNone, scratch);
        const uint32_t below = block_sum_u32(tid == digit ? ex : 0u, scratch);
        prefix |= digit << shift;
        need -= below;
    }
    uint32_t lo = kNone;
    for (uint32_t i = tid; i < len; i += blockDim.x) lo = min(lo, a.keys[e0 + i]);
    lo = block_min_u32(lo, scratch);
    if (tid == 0) {
        a.p99[c] = key_f32(prefix);
        a.mn[c] = key_f32(lo);
    }
}

// Row i of dst = row old_of_new[i] of src (width elements per row).
template <class T>
__global__ void __launch_bounds__(kStoreThreads)
gather_rows_kernel(const T* __restrict__ src, const uint32_t* __restrict__ old_of_new, uint32_t n_new, uint32_t width,
                   T* __restrict__ dst) {
    for (uint32_t i = blockIdx.x; i < n_new; i += gridDim.x) {
        const T* s = src + static_cast<uint64_t>(old_of_new[i]) * width;
        T* o = dst + static_cast<uint64_t>(i) * width;
        for (uint32_t j = threadIdx.x; j < width; j += blockDim.x) o[j] = s[j];
    }
}

// One workgroup per cell: its FastScan blocks from the members' sign codes. Byte p*32 + half*16 + i
// of a block holds nibble j = 2p + half of the block's member i (low half) and member i + 16 (high
// half); absent members give 0 (fs_pack_block, src/quantize.rs:238-265).
__global__ void __launch_bounds__(kStoreThreads)
fs_pack_kernel(const uint64_t* __restrict__ bits, const uint32_t* __restrict__ mem_off, const uint32_t* __restrict__ members,
               const uint32_t* __restrict__ fs_off, uint32_t W, uint8_t* __restrict__ fs) {
    const uint32_t c = blockIdx.x;
    const uint32_t e0 = mem_off[c], len = mem_off[c + 1] - e0;
    const uint32_t nb = fs_off[c + 1] - fs_off[c], bb = W * 256;
    auto nib = [&](uint32_t m, uint32_t j) -> uint32_t {
        if (m >= len) return 0u;
        const uint64_t* code = bits + static_cast<uint64_t>(members[e0 + m]) * W;
        return static_cast<uint32_t>((code[j >> 4] >> ((j & 15u) * 4u)) & 0xFu);
    };
    for (uint32_t idx = threadIdx.x; idx < nb * bb; idx += blockDim.x) {
        const uint32_t b = idx / bb, off = idx - b * bb;
        const uint32_t p = off / 32, half = (off % 32) / 16, i = off % 16, j = 2 * p + half;
        const uint32_t lo = nib(b * 32 + i, j), hi = nib(b * 32 + i + 16, j);
        fs[(static_cast<uint64_t>(fs_off[c]) + b) * bb + off] = static_cast<uint8_t>(lo | (hi << 4));
    }
}

uint32_t grid_rows(uint64_t n) { return static_cast<uint32_t>(std::max<uint64_t>(1, std::min<uint64_t>(n, 65535))); }
uint32_t grid_elems(uint64_t n) {
    return static_cast<uint32_t>(std::max<uint64_t>(1, std::min<uint64_t>((n + 255) / 256, 65535)));
}

// Tokens are unique across contexts: one counter for the process.
uint64_t next_token() {
    static std::atomic<uint64_t> counter{0};
    return ++counter;
}

// Buffers of one call, freed when it returns (after the stream drains).
struct Tmp {
    maivs_gpu_ctx* ctx;
    std::vector<void*> allocs;
    explicit Tmp(maivs_gpu_ctx* c) : ctx(c) {}
    ~Tmp() {
        if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
        free_all(allocs);
    }
    template <class T>
    int alloc(T** p, size_t n) { return dalloc(ctx, allocs, p, n); }
    template <class T>
    int upload(T** p, const T* src, size_t n) {
        int rc = alloc(p, n);
        if (rc) return rc;
        if (n) HIP_TRY(ctx, hipMemcpyAsync(*p, src, n * sizeof(T), hipMemcpyHostToDevice, ctx->stream));
        return 0;
    }
};

// New buffers of `cap` slots for every array of the layout; the first `keep` slots are copied over.
int store_realloc(maivs_gpu_ctx* ctx, uint32_t cap, uint32_t keep) {
    RowStore& R = ctx->store;
    std::vector<void*> fresh;
    float* f = nullptr;
    int8_t* k = nullptr;
    uint64_t* b = nullptr;
    int rc = 0;
    if ((R.flags & MAIVS_STORE_F32) && (rc = dalloc(ctx, fresh, &f, static_cast<size_t>(cap) * R.dim))) return rc;
    if ((R.flags & MAIVS_STORE_CODES) && (rc = dalloc(ctx, fresh, &k, static_cast<size_t>(cap) * R.dim))) {
        free_all(fresh);
        return rc;
    }
    if ((R.flags & MAIVS_STORE_BITS) && (rc = dalloc(ctx, fresh, &b, static_cast<size_t>(cap) * R.W))) {
        free_all(fresh);
        return rc;
    }
    if (keep) {
        if (f) HIP_TRY(ctx, hipMemcpyAsync(f, R.f32, static_cast<size_t>(keep) * R.dim * 4, hipMemcpyDeviceToDevice, ctx->stream));
        if (k) HIP_TRY(ctx, hipMemcpyAsync(k, R.codes, static_cast<size_t>(keep) * R.dim, hipMemcpyDeviceToDevice, ctx->stream));
        if (b) HIP_TRY(ctx, hipMemcpyAsync(b, R.bits, static_cast<size_t>(keep) * R.W * 8, hipMemcpyDeviceToDevice, ctx->stream));
    }
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    free_all(R.allocs);
    R.allocs = fresh;
    R.f32 = f;
    R.codes = k;
    R.bits = b;
    R.cap = cap;
    return 0;
}

}  // namespace

namespace maivs_host {

int store_write(maivs_gpu_ctx* ctx, const uint32_t* h_slots, uint32_t n, const float* d_x, const uint64_t* d_bits,
                const int8_t* d_codes, bool has_codes) {
    RowStore& R = ctx->store;
    if (!R.token) return fail(ctx, MAIVS_ERR_ARG, "the row store was never reset");
    if ((R.flags & MAIVS_STORE_CODES) && !has_codes)
        return fail(ctx, MAIVS_ERR_ARG, "the row store keeps i8 / SQ8 rows but the placement makes none");
    if (n == 0) return 0;
    uint32_t top = R.n;
    for (uint32_t i = 0; i < n; ++i) {
        if (h_slots[i] >= (1u << 31)) return fail(ctx, MAIVS_ERR_ARG, "store slot %u out of range", h_slots[i]);
        top = std::max(top, h_slots[i] + 1);
    }
    int rc;
    const uint32_t grown = static_cast<uint32_t>(std::min<uint64_t>(2ull * R.cap, 1ull << 31));
    if (top > R.cap && (rc = store_realloc(ctx, std::max(top, grown), R.n))) return rc;
    Tmp T(ctx);
    uint32_t* d_slots;
    if ((rc = T.upload(&d_slots, h_slots, n))) return rc;
    hipLaunchKernelGGL(store_scatter_kernel, dim3(grid_rows(n)), dim3(kStoreThreads), 0, ctx->stream, d_x, d_bits, d_codes,
                       d_slots, n, R.dim, R.W, (R.flags & MAIVS_STORE_F32) ? R.f32 : nullptr,
                       (R.flags & MAIVS_STORE_BITS) ? R.bits : nullptr, (R.flags & MAIVS_STORE_CODES) ? R.codes : nullptr);
    HIP_TRY(ctx, hipGetLastError());
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    R.n = top;
    R.token = next_token();
    return 0;
}

int cell_sums(maivs_gpu_ctx* ctx, const float* d_x, const uint32_t* d_homes, uint32_t ma, uint32_t n, uint32_t M,
              uint32_t d, float* h_sums) {
    if (n == 0) return 0;
    Tmp T(ctx);
    float* d_sums;
    uint32_t *key, *pos, *skey, *spos, *start, *end;
    int rc;
    if ((rc = T.upload(&d_sums, h_sums, static_cast<size_t>(M) * d)) || (rc = T.alloc(&key, n)) ||
        (rc = T.alloc(&pos, n)) || (rc = T.alloc(&skey, n)) || (rc = T.alloc(&spos, n)) || (rc = T.alloc(&start, M)) ||
        (rc = T.alloc(&end, M)))
        return rc;
    hipLaunchKernelGGL(primary_key_kernel, dim3(grid_elems(n)), dim3(256), 0, ctx->stream, d_homes, ma, n, key, pos);
    hipLaunchKernelGGL(zero_u32_kernel, dim3(grid_elems(M)), dim3(256), 0, ctx->stream, start, M);
    hipLaunchKernelGGL(zero_u32_kernel, dim3(grid_elems(M)), dim3(256), 0, ctx->stream, end, M);
    unsigned end_bit = 1;
    while (end_bit < 32 && (1ull << end_bit) < M) ++end_bit;
    size_t tmp_bytes = 0;
    HIP_TRY(ctx, rocprim::radix_sort_pairs(nullptr, tmp_bytes, key, skey, pos, spos, n, 0u, end_bit, ctx->stream));
    uint8_t* d_tmp;
    if ((rc = T.alloc(&d_tmp, std::max<size_t>(tmp_bytes, 1)))) return rc;
    HIP_TRY(ctx, rocprim::radix_sort_pairs(d_tmp, tmp_bytes, key, skey, pos, spos, n, 0u, end_bit, ctx->stream));
    hipLaunchKernelGGL(run_bounds_kernel, dim3(grid_elems(n)), dim3(256), 0, ctx->stream, skey, n, start, end);
    hipLaunchKernelGGL(cell_sum_kernel, dim3(M), dim3(kStoreThreads), 0, ctx->stream, d_x, spos, start, end, d, d_sums);
    HIP_TRY(ctx, hipGetLastError());
    HIP_TRY(ctx, hipMemcpyAsync(h_sums, d_sums, static_cast<size_t>(M) * d * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

}  // namespace maivs_host

extern "C" {

int maivs_gpu_store_reset(maivs_gpu_ctx* ctx, uint32_t dim, uint32_t n_words, uint32_t flags) {
    if (!ctx) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    if (dim == 0 || (flags & ~7u) || ((flags & MAIVS_STORE_BITS) && n_words == 0))
        return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_reset: dim %u, n_words %u, flags %u", dim, n_words, flags);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (ctx->stream) HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    RowStore& R = ctx->store;
    free_all(R.allocs);
    R.f32 = nullptr;
    R.codes = nullptr;
    R.bits = nullptr;
    R.dim = dim;
    R.W = n_words;
    R.flags = flags;
    R.n = 0;
    R.cap = 0;
    R.token = next_token();
    return 0;
}

int maivs_gpu_store_info(maivs_gpu_ctx* ctx, uint64_t* token, uint32_t* n_slots) {
    if (!ctx) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    if (token) *token = ctx->store.token;
    if (n_slots) *n_slots = ctx->store.n;
    return 0;
}

int maivs_gpu_store_radii(maivs_gpu_ctx* ctx, const maivs_radii_desc* D, float* p99_dot, float* min_dot) {
    if (!ctx) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    if (!D || !p99_dot || !min_dot || !D->mem_off || (D->n_cells && (!D->centroids || !D->members)))
        return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_radii: null buffer");
    const RowStore& R = ctx->store;
    const uint32_t M = D->n_cells, d = D->dim;
    if (M == 0) return 0;
    if (d != R.dim || D->mode > 2) return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_radii: dim %u / mode %u", d, D->mode);
    if (D->mode == 0 ? !(R.flags & MAIVS_STORE_F32) : !(R.flags & MAIVS_STORE_CODES))
        return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_radii: the store keeps no rows of mode %u", D->mode);
    if (D->mode == 1 && (!D->sq_min || !D->sq_step)) return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_radii: SQ8 ranges missing");
    const uint64_t E = D->mem_off[M];
    for (uint32_t c = 0; c < M; ++c)
        if (D->mem_off[c + 1] < D->mem_off[c]) return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_radii: mem_off decreases");
    for (uint64_t e = 0; e < E; ++e)
        if (D->members[e] >= R.n) return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_radii: member %u >= %u slots", D->members[e], R.n);
    if (static_cast<size_t>(d) * 4 > 64 * 1024) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "maivs_gpu_store_radii: dim %u", d);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    Tmp T(ctx);
    RadiiArgs a{};
    uint32_t *mem_off, *members, *keys;
    float *cents, *sq_min = nullptr, *sq_step = nullptr, *p99, *mn;
    int rc;
    if ((rc = T.upload(&mem_off, D->mem_off, static_cast<size_t>(M) + 1)) || (rc = T.upload(&members, D->members, E)) ||
        (rc = T.upload(&cents, D->centroids, static_cast<size_t>(M) * d)) || (rc = T.alloc(&keys, E)) ||
        (rc = T.alloc(&p99, M)) || (rc = T.alloc(&mn, M)))
        return rc;
    if (D->mode == 1 && ((rc = T.upload(&sq_min, D->sq_min, d)) || (rc = T.upload(&sq_step, D->sq_step, d)))) return rc;
    a.mem_off = mem_off;
    a.members = members;
    a.cents = cents;
    a.sq_min = sq_min;
    a.sq_step = sq_step;
    a.rows = R.f32;
    a.codes = R.codes;
    a.keys = keys;
    a.p99 = p99;
    a.mn = mn;
    a.M = M;
    a.d = d;
    a.mode = D->mode;
    a.inv = D->inv_scale;
    hipLaunchKernelGGL(radii_kernel, dim3(M), dim3(kStoreThreads), static_cast<size_t>(d) * 4, ctx->stream, a);
    HIP_TRY(ctx, hipGetLastError());
    HIP_TRY(ctx, hipMemcpyAsync(p99_dot, p99, static_cast<size_t>(M) * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(min_dot, mn, static_cast<size_t>(M) * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

int maivs_gpu_store_compact(maivs_gpu_ctx* ctx, const uint32_t* old_of_new, uint32_t n_new, uint32_t n_cells,
                            const uint32_t* mem_off, const uint32_t* members, const uint32_t* fs_off, uint8_t* fs_codes,
                            float* rows_out, int8_t* codes_out, uint64_t* bits_out) {
    if (!ctx) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    RowStore& R = ctx->store;
    if (!R.token) return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_compact: the row store was never reset");
    if (n_new && !old_of_new) return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_compact: null buffer");
    for (uint32_t i = 0; i < n_new; ++i)
        if (old_of_new[i] >= R.n) return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_compact: old slot %u >= %u", old_of_new[i], R.n);
    if ((rows_out && !(R.flags & MAIVS_STORE_F32)) || (codes_out && !(R.flags & MAIVS_STORE_CODES)) ||
        (bits_out && !(R.flags & MAIVS_STORE_BITS)))
        return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_compact: the store keeps no such rows");
    const bool pack = fs_codes != nullptr;
    uint64_t E = 0, B = 0;
    if (pack) {
        if (!(R.flags & MAIVS_STORE_BITS) || !mem_off || !fs_off || (n_cells && !members))
            return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_compact: FastScan packing needs sign codes, members and fs_off");
        E = mem_off[n_cells];
        B = fs_off[n_cells];
        for (uint32_t c = 0; c < n_cells; ++c) {
            if (mem_off[c + 1] < mem_off[c] || fs_off[c + 1] < fs_off[c] ||
                fs_off[c + 1] - fs_off[c] != (mem_off[c + 1] - mem_off[c] + 31) / 32)
                return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_compact: cell %u's offsets", c);
        }
        for (uint64_t e = 0; e < E; ++e)
            if (members[e] >= n_new) return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_store_compact: member %u >= %u", members[e], n_new);
    }
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    int rc;
    {
        Tmp T(ctx);
        uint32_t* d_map;
        if ((rc = T.upload(&d_map, old_of_new, n_new))) return rc;
        // the compacted rows go to fresh buffers, which then become the store
        std::vector<void*> fresh;
        float* f = nullptr;
        int8_t* k = nullptr;
        uint64_t* b = nullptr;
        const uint32_t cap = std::max<uint32_t>(n_new, 1);
        if (((R.flags & MAIVS_STORE_F32) && (rc = dalloc(ctx, fresh, &f, static_cast<size_t>(cap) * R.dim))) ||
            ((R.flags & MAIVS_STORE_CODES) && (rc = dalloc(ctx, fresh, &k, static_cast<size_t>(cap) * R.dim))) ||
            ((R.flags & MAIVS_STORE_BITS) && (rc = dalloc(ctx, fresh, &b, static_cast<size_t>(cap) * R.W)))) {
            free_all(fresh);
            return rc;
        }
        if (n_new) {
            if (f)
                hipLaunchKernelGGL(gather_rows_kernel<float>, dim3(grid_rows(n_new)), dim3(kStoreThreads), 0, ctx->stream, R.f32,
                                   d_map, n_new, R.dim, f);
            if (k)
                hipLaunchKernelGGL(gather_rows_kernel<int8_t>, dim3(grid_rows(n_new)), dim3(kStoreThreads), 0, ctx->stream,
                                   R.codes, d_map, n_new, R.dim, k);
            if (b)
                hipLaunchKernelGGL(gather_rows_kernel<uint64_t>, dim3(grid_rows(n_new)), dim3(kStoreThreads), 0, ctx->stream,
                                   R.bits, d_map, n_new, R.W, b);
        }
        const hipError_t e = hipGetLastError();
        const hipError_t s = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess || s != hipSuccess) {
            free_all(fresh);
            return fail(ctx, MAIVS_ERR_HIP, "maivs_gpu_store_compact: %s", hipGetErrorString(e != hipSuccess ? e : s));
        }
        free_all(R.allocs);
        R.allocs = fresh;
        R.f32 = f;
        R.codes = k;
        R.bits = b;
        R.n = n_new;
        R.cap = cap;
        R.token = next_token();
    }
    Tmp T(ctx);
    if (pack && n_cells) {
        uint32_t *d_off, *d_mem, *d_fs_off;
        uint8_t* d_fs;
        if ((rc = T.upload(&d_off, mem_off, static_cast<size_t>(n_cells) + 1)) || (rc = T.upload(&d_mem, members, E)) ||
            (rc = T.upload(&d_fs_off, fs_off, static_cast<size_t>(n_cells) + 1)) ||
            (rc = T.alloc(&d_fs, B * R.W * 256)))
            return rc;
        hipLaunchKernelGGL(fs_pack_kernel, dim3(n_cells), dim3(kStoreThreads), 0, ctx->stream, R.bits, d_off, d_mem, d_fs_off,
                           R.W, d_fs);
        HIP_TRY(ctx, hipGetLastError());
        if (B) HIP_TRY(ctx, hipMemcpyAsync(fs_codes, d_fs, B * R.W * 256, hipMemcpyDeviceToHost, ctx->stream));
    }
    if (n_new) {
        if (rows_out)
            HIP_TRY(ctx, hipMemcpyAsync(rows_out, R.f32, static_cast<size_t>(n_new) * R.dim * 4, hipMemcpyDeviceToHost, ctx->stream));
        if (codes_out)
            HIP_TRY(ctx, hipMemcpyAsync(codes_out, R.codes, static_cast<size_t>(n_new) * R.dim, hipMemcpyDeviceToHost, ctx->stream));
        if (bits_out)
            HIP_TRY(ctx, hipMemcpyAsync(bits_out, R.bits, static_cast<size_t>(n_new) * R.W * 8, hipMemcpyDeviceToHost, ctx->stream));
    }
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

}  // extern "C"
