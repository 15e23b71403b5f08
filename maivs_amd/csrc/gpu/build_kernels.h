// Device kernels of the index build: batched spherical Lloyd k-means (src/tree.rs:179-248).
//
// Every result is bit-identical to the reference's CPU arithmetic:
//   * a score is the 8-lane FMA dot (lane l accumulates elements l, l+8, ...), summed as
//     ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)), plus a sequential tail (src/index.rs:136-152);
//   * the best centroid is the first maximum (strict >, ascending centroid index, from -inf);
//   * a cluster sum starts at +0.0 and adds its points in ascending point order, one f32 add
//     per point and dimension;
//   * the norm starts at -0.0 and adds x*x in dimension order (no FMA), then one correctly
//     rounded sqrt and one correctly rounded division per dimension when the norm > 1e-12;
//   * empty clusters take the point at xorshift64(state) % n, the state advancing once per empty
//     cluster in ascending cluster order and carried across iterations.
// Many independent problems ("jobs") run in one launch: one per group of the second k-means
// level, or a single one.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.h"

namespace maivs_dev {

constexpr uint32_t kKmThreads = 256;   // points per assignment workgroup (one per lane)
constexpr uint32_t kKmGroup = 8;       // centroids scored together per point
constexpr uint32_t kKmMaxDimPerThread = 8;  // update kernel: dims per thread (dim <= 2048)

struct KmJob {
    uint32_t first;  // first entry of this job's points in the row list
    uint32_t n;      // points
    uint32_t k;      // clusters, 1 <= k <= n
    uint32_t iters;
    uint32_t coff;   // first centroid (global cluster id) of this job
    uint32_t pad[3];
};

struct KmArgs {
    const float* x;         // n_rows x d
    const uint32_t* rows;   // n_points row ids, job-major (each job's points in its order)
    const KmJob* jobs;
    const uint32_t* blk_job;    // assignment workgroup -> job
    const uint32_t* blk_start;  // assignment workgroup -> first point within its job
    const uint32_t* c_job;      // global cluster -> job
    float* cents;           // sum_k x d
    uint32_t* best;         // n_points: cluster within the job, last iteration
    uint32_t* key;          // n_points: global cluster of the point (sort key)
    uint32_t* pos;          // n_points: global point position (sort value)
    uint32_t* cnt;          // sum_k
    uint32_t* start;        // sum_k: first sorted position of each non-empty cluster
    const uint32_t* skey;   // sorted keys
    const uint32_t* spos;   // sorted positions
    uint64_t* state;        // per job xorshift state
    uint32_t d, n_points, sum_k, n_jobs;
};

// Centroid c of every job starts as the job's point min(c * stride, n - 1), stride = max(n / k, 1).
__global__ void km_init_kernel(KmArgs a) {
    const uint32_t c = blockIdx.x;
    if (c >= a.sum_k) return;
    const KmJob J = a.jobs[a.c_job[c]];
    const uint32_t local = c - J.coff;
    const uint32_t stride = max(J.n / J.k, 1u);
    const uint32_t src = min(local * stride, J.n - 1);
    const float* xr = a.x + static_cast<uint64_t>(a.rows[J.first + src]) * a.d;
    for (uint32_t i = threadIdx.x; i < a.d; i += blockDim.x) a.cents[static_cast<uint64_t>(c) * a.d + i] = xr[i];
}

__global__ void km_zero_kernel(uint32_t* p, uint32_t n) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

// One lane per point: the first best centroid by the exact dot, kKmGroup centroids per pass.
// Every workgroup lies inside one job, so the centroid rows are read at wave-uniform addresses.
// V4: d % 4 == 0, so every row starts 16-byte aligned and the point is read 16 bytes at a time.
template <bool V4>
__global__ void __launch_bounds__(kKmThreads) km_assign_kernel(KmArgs a, uint32_t it) {
    const uint32_t jb = __builtin_amdgcn_readfirstlane(a.blk_job[blockIdx.x]);
    const KmJob J = a.jobs[jb];
    if (it >= J.iters) return;
    const uint32_t i = a.blk_start[blockIdx.x] + threadIdx.x;
    const bool valid = i < J.n;
    const uint32_t d = a.d, d8 = d & ~7u;
    const float* __restrict__ xr = a.x + static_cast<uint64_t>(a.rows[J.first + (valid ? i : 0u)]) * d;
    const float* __restrict__ cb = a.cents + static_cast<uint64_t>(J.coff) * d;
    const uint32_t k = J.k;
    uint32_t best = 0;
    float best_s = -INFINITY;
    for (uint32_t c0 = 0; c0 < k; c0 += kKmGroup) {
        float acc[kKmGroup][8];
#pragma unroll
        for (uint32_t g = 0; g < kKmGroup; ++g)
#pragma unroll
            for (uint32_t l = 0; l < 8; ++l) acc[g][l] = 0.0f;
        for (uint32_t t = 0; t < d8; t += 8) {
            float xv[8];
            if constexpr (V4) {
                const float4 x0 = *reinterpret_cast<const float4*>(xr + t);
                const float4 x1 = *reinterpret_cast<const float4*>(xr + t + 4);
                xv[0] = x0.x, xv[1] = x0.y, xv[2] = x0.z, xv[3] = x0.w;
                xv[4] = x1.x, xv[5] = x1.y, xv[6] = x1.z, xv[7] = x1.w;
            } else {  // a row of another dimension is only 4-byte aligned
#pragma unroll
                for (uint32_t l = 0; l < 8; ++l) xv[l] = xr[t + l];
            }
#pragma unroll
            for (uint32_t g = 0; g < kKmGroup; ++g) {
                const uint32_t c = min(c0 + g, k - 1);
                const float* cr = cb + static_cast<uint64_t>(c) * d + t;
#pragma unroll
                for (uint32_t l = 0; l < 8; ++l) acc[g][l] = __builtin_fmaf(xv[l], cr[l], acc[g][l]);
            }
        }
#pragma unroll
        for (uint32_t g = 0; g < kKmGroup; ++g) {
            const uint32_t c = c0 + g;
            const float* a8 = acc[g];
            float s = ((a8[0] + a8[4]) + (a8[2] + a8[6])) + ((a8[1] + a8[5]) + (a8[3] + a8[7]));
            const float* cr = cb + static_cast<uint64_t>(min(c, k - 1)) * d;
            for (uint32_t e = d8; e < d; ++e) s += xr[e] * cr[e];
            if (c < k && s > best_s) {
                best_s = s;
                best = c;
            }
        }
    }
    if (valid) {
        const uint32_t p = J.first + i;
        a.best[p] = best;
        a.key[p] = J.coff + best;
        a.pos[p] = p;
        atomicAdd(&a.cnt[J.coff + best], 1u);
    }
}

// Sorted positions -> first position of each non-empty cluster.
__global__ void km_starts_kernel(KmArgs a, uint32_t n) {
    for (uint32_t p = blockIdx.x * blockDim.x + threadIdx.x; p < n; p += gridDim.x * blockDim.x) {
        const uint32_t k = a.skey[p];
        if (p == 0 || a.skey[p - 1] != k) a.start[k] = p;
    }
}

// One workgroup per non-empty cluster: the in-order sum of its points, then the normalisation.
__global__ void __launch_bounds__(256) km_update_kernel(KmArgs a, uint32_t it) {
    extern __shared__ float s_sum[];  // d floats, then the norm
    const uint32_t c = blockIdx.x;
    const KmJob J = a.jobs[a.c_job[c]];
    if (it >= J.iters) return;
    const uint32_t m = a.cnt[c];
    if (m == 0) return;  // reseeded by km_reseed_kernel
    const uint32_t s0 = a.start[c], d = a.d, tid = threadIdx.x;
    float s[kKmMaxDimPerThread];
#pragma unroll
    for (uint32_t r = 0; r < kKmMaxDimPerThread; ++r) s[r] = 0.0f;
    constexpr uint32_t kAhead = 8;
    for (uint32_t u = 0; u < m; u += kAhead) {
        float v[kAhead][kKmMaxDimPerThread];
#pragma unroll
        for (uint32_t q = 0; q < kAhead; ++q) {
            const uint32_t mm = min(u + q, m - 1);
            const float* xr = a.x + static_cast<uint64_t>(a.rows[a.spos[s0 + mm]]) * d;
#pragma unroll
            for (uint32_t r = 0; r < kKmMaxDimPerThread; ++r) {
                const uint32_t dd = tid + r * 256;
                v[q][r] = dd < d ? xr[dd] : 0.0f;
            }
        }
#pragma unroll
        for (uint32_t q = 0; q < kAhead; ++q)
            if (u + q < m)
#pragma unroll
                for (uint32_t r = 0; r < kKmMaxDimPerThread; ++r) s[r] += v[q][r];
    }
#pragma unroll
    for (uint32_t r = 0; r < kKmMaxDimPerThread; ++r) {
        const uint32_t dd = tid + r * 256;
        if (dd < d) s_sum[dd] = s[r];
    }
    __syncthreads();
    if (tid == 0) {
        float nrm = -0.0f;
        for (uint32_t i = 0; i < d; ++i) {
            const float p = s_sum[i] * s_sum[i];
            nrm = nrm + p;
        }
        s_sum[d] = __builtin_sqrtf(nrm);
    }
    __syncthreads();
    const float nrm = s_sum[d];
    float* out = a.cents + static_cast<uint64_t>(c) * d;
    for (uint32_t dd = tid; dd < d; dd += blockDim.x) out[dd] = nrm > 1e-12f ? s_sum[dd] / nrm : s_sum[dd];
}

// One thread per job: empty clusters in ascending order take xorshift64 picks (src/tree.rs:230-236).
__global__ void km_reseed_kernel(KmArgs a, uint32_t it) {
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= a.n_jobs) return;
    const KmJob J = a.jobs[j];
    if (it >= J.iters) return;
    uint64_t st = a.state[j];
    for (uint32_t c = 0; c < J.k; ++c) {
        if (a.cnt[J.coff + c] != 0) continue;
        st ^= st << 13;
        st ^= st >> 7;
        st ^= st << 17;
        const uint32_t src = static_cast<uint32_t>(st % J.n);
        const float* xr = a.x + static_cast<uint64_t>(a.rows[J.first + src]) * a.d;
        float* out = a.cents + static_cast<uint64_t>(J.coff + c) * a.d;
        for (uint32_t i = 0; i < a.d; ++i) out[i] = xr[i];
    }
    a.state[j] = st;
}

}  // namespace maivs_dev
