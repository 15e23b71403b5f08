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
#include "wave_tree.h"

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

// ================================================================ placement (add_batch)

namespace maivs_dev {

// Placement of new vectors (src/index.rs:2442-2560 with the tree descent of src/tree.rs:120-159,
// 559-628), one wave per vector:
//   1. the rotation (2 x sign flip + FWHT, as the search's query prep) and the 1-bit code;
//   2. with a centroid tree: Hamming beam descent, each level keeping its `beam` smallest
//      distances with ties in encounter order (keep_smallest), children of the kept nodes in
//      order; the leaves keep `want`; no tree, or an empty result: every cell, in order;
//   3. exact 8-lane FMA dots against the candidates' f32 centroids;
//   4. the homes: max_assign 1 = the first best; else the top of (score desc, cell asc), either
//      cut at best - spill_margin or, with a polysemy strength, chosen greedily from the best 16
//      by 2 - 2 s_j + sum over chosen homes h of lam * p^2, p = (1 - s_h - s_j + <c_h, c_j>) /
//      sqrt(max(2 - 2 s_h, 1e-12)), first minimum;
//   5. the i8 / SQ8 code of the vector when the index keeps one.
constexpr uint32_t kPlaceWaves = 4;
constexpr uint32_t kPlacePool = 16;  // candidates the orthogonal choice considers (src/index.rs:2524)

struct PlaceArgs {
    const float* x;            // n x d
    const float* signs;        // 2 x P
    const float* cents;        // M x d
    TreeDev tree;              // n_levels == 0: no tree
    const uint32_t* beams;     // n_levels
    const float* sq_min;
    const float* sq_step;
    uint32_t* homes;           // n x ma, UINT32_MAX padded
    uint64_t* bits;            // n x W
    int8_t* codes;             // n x d when code_mode != 0
    float fht_scale, spill_lambda, spill_margin, quant_scale;
    uint32_t n, d, P, W, M, want, ma, kept_cap, code_mode, lds_per_wave;
};

// Per-wave LDS of the placement kernel, in order: qb[W] u64 | xs[P] | vs[d4] | hist[bits + 1, to 4]
// | rbase[cap + 1] | rpre[cap + 2] | knodes[cap] | outc[want] | hcache[kTreeHCache] u16
struct PlaceLds {
    uint64_t* qb;
    float *xs, *vs;
    uint32_t *hist, *rbase, *rpre, *knodes, *outc;
    uint16_t* hcache;
};

__host__ __device__ inline uint32_t place_lds_words(uint32_t P, uint32_t d, uint32_t W, uint32_t cap, uint32_t want) {
    const uint32_t d4 = (d + 3) & ~3u, hb = (W * 64 + 1 + 3) & ~3u;
    return 2 * W + P + d4 + hb + (cap + 1) + (cap + 2) + cap + want + kTreeHCache / 2;
}

__device__ __forceinline__ PlaceLds place_lds(uint8_t* base, const PlaceArgs& a) {
    PlaceLds L;
    L.qb = reinterpret_cast<uint64_t*>(base);
    L.xs = reinterpret_cast<float*>(L.qb + a.W);
    L.vs = L.xs + a.P;
    L.hist = reinterpret_cast<uint32_t*>(L.vs + ((a.d + 3) & ~3u));
    L.rbase = L.hist + ((a.W * 64 + 1 + 3) & ~3u);
    L.rpre = L.rbase + a.kept_cap + 1;
    L.knodes = L.rpre + a.kept_cap + 2;
    L.outc = L.knodes + a.kept_cap;
    L.hcache = reinterpret_cast<uint16_t*>(L.outc + a.want);
    return L;
}

template <int EPL>
__global__ void __launch_bounds__(kPlaceWaves * kWave) place_kernel(PlaceArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t lane = lane_id(), wv = threadIdx.x / kWave;
    const PlaceLds L = place_lds(smem + static_cast<size_t>(wv) * a.lds_per_wave, a);
    const uint32_t d = a.d, P = a.P, W = a.W, bits = W * 64, ma = a.ma;
    for (uint32_t i = blockIdx.x * kPlaceWaves + wv; i < a.n; i += gridDim.x * kPlaceWaves) {
        const float* v = a.x + static_cast<uint64_t>(i) * d;
        for (uint32_t j = lane; j < d; j += kWave) L.vs[j] = v[j];
        wave_sync();
        // ---- the i8 / SQ8 copy (src/index.rs:2582-2610, 3083-3123)
        if (a.code_mode) {
            int8_t* out = a.codes + static_cast<uint64_t>(i) * d;
            for (uint32_t j = lane; j < d; j += kWave) {
                const float x = L.vs[j];
                float c;
                if (a.code_mode == 1) {
                    c = roundf((x - a.sq_min[j]) / a.sq_step[j]);
                    c = fminf(fmaxf(c, 0.0f), 255.0f);
                    out[j] = static_cast<int8_t>(static_cast<uint8_t>(c));
                } else {
                    c = roundf(x * a.quant_scale);
                    c = fminf(fmaxf(c, -127.0f), 127.0f);
                    out[j] = static_cast<int8_t>(c);
                }
            }
        }
        // ---- rotation: element lane*EPL + e in x[e]; levels ascending, in-lane then cross-lane
        float x[EPL];
        const uint32_t base = lane * EPL;
#pragma unroll
        for (int e = 0; e < EPL; ++e) x[e] = base + e < d ? L.vs[base + e] : 0.0f;
        for (int r = 0; r < 2; ++r) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) x[e] *= a.signs[r * P + base + e];
#pragma unroll
            for (int h = 1; h < EPL; h <<= 1) {
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    if ((e & h) == 0) {
                        const float u = x[e], w = x[e + h];
                        x[e] = u + w;
                        x[e + h] = u - w;
                    }
                }
            }
#pragma unroll
            for (uint32_t m = 1; m < kWave; m <<= 1) {
                const bool upper = (lane & m) != 0;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const float w = __shfl_xor(x[e], static_cast<int>(m), kWave);
                    x[e] = upper ? w - x[e] : x[e] + w;
                }
            }
#pragma unroll
            for (int e = 0; e < EPL; ++e) x[e] *= a.fht_scale;
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) L.xs[base + e] = x[e];
        wave_sync();
        for (uint32_t w = 0; w < W; ++w) {
            const uint64_t m = __ballot(L.xs[64 * w + lane] < 0.0f);
            if (lane == 0) {
                L.qb[w] = m;
                a.bits[static_cast<uint64_t>(i) * W + w] = m;
            }
        }
        wave_sync();
        // ---- tree descent (src/tree.rs:574-628); no tree or no result: every cell
        uint32_t nout = tree_descent(a.tree, a.beams, a.want, L.qb, W, L.hist, L.rbase, L.rpre, L.knodes, L.outc,
                                     L.hcache, kTreeHCache);
        const bool use_tree = nout > 0;
        if (!use_tree) nout = a.M;  // every cell, in order (src/index.rs:2480-2509)
        // ---- exact scores and the running selection
        uint64_t kmin = kKeyMax;  // ma == 1: (score desc, position asc)
        uint64_t top = kKeyMax;   // ma > 1: the 64 best (score desc, cell asc), ascending over lanes
        for (uint32_t c0 = 0; c0 < nout; c0 += kWave) {
            const uint32_t j = c0 + lane;
            const bool valid = j < nout;
            const uint32_t cell = valid ? (use_tree ? L.outc[j] : j) : 0u;
            float s = 0.0f;
            if (valid) {
                const float* cr = a.cents + static_cast<uint64_t>(cell) * d;
                s = dot_lane(d, [&](uint32_t e) { return L.vs[e]; }, [&](uint32_t e) { return cr[e]; });
            }
            if (ma <= 1) {
                if (valid) kmin = min(kmin, desc_score_key(s, j));
            } else {
                uint64_t ck[1] = {valid ? desc_score_key(s, cell) : kKeyMax};
                wave_sort_u64<1>(ck);
                const uint64_t other = __shfl(ck[0], kWave - 1 - lane, kWave);
                uint64_t m[1] = {min(top, other)};
                wave_sort_u64<1>(m);
                top = m[0];
            }
        }
        uint32_t* hout = a.homes + static_cast<uint64_t>(i) * ma;
        if (ma <= 1) {
            const uint64_t best = [&] {
                uint64_t b = kmin;
                for (int o = 32; o > 0; o >>= 1) {
                    const uint64_t y = __shfl_xor(b, o, kWave);
                    b = y < b ? y : b;
                }
                return b;
            }();
            const uint32_t pos = best == kKeyMax ? 0u : static_cast<uint32_t>(best);
            if (lane == 0) hout[0] = use_tree ? L.outc[pos] : pos;
            continue;
        }
        const uint32_t ncand = min(nout, static_cast<uint32_t>(kWave));
        const float my_s = key_score(top);
        const uint32_t my_cell = static_cast<uint32_t>(top);
        if (a.spill_lambda > 0.0f) {
            // pick_orthogonal (src/index.rs:2523-2560) over the best min(16, n) candidates
            const uint32_t pool = min(kPlacePool, nout);
            const uint32_t r = min(ma, pool);
            const bool in_pool = lane < pool;
            float loss = 2.0f - 2.0f * my_s;
            bool taken = lane == 0;
            uint32_t nh = 1;
            uint32_t h_cell = __shfl(my_cell, 0, kWave);
            float h_s = __shfl(my_s, 0, kWave);
            if (lane == 0) hout[0] = h_cell;
            while (nh < r) {
                // add the newest home's term to every open candidate's loss
                if (in_pool && !taken) {
                    const float rn = __builtin_sqrtf(fmaxf(2.0f - 2.0f * h_s, 1e-12f));
                    const float* ch = a.cents + static_cast<uint64_t>(h_cell) * d;
                    const float* cj = a.cents + static_cast<uint64_t>(my_cell) * d;
                    const float g = dot_lane(d, [&](uint32_t e) { return ch[e]; }, [&](uint32_t e) { return cj[e]; });
                    const float p = (((1.0f - h_s) - my_s) + g) / rn;
                    loss = loss + (a.spill_lambda * p) * p;
                }
                const bool ok = in_pool && !taken && loss < INFINITY;
                uint64_t k = ok ? ((static_cast<uint64_t>(asc_f32_key(loss)) << 32) | lane) : kKeyMax;
                for (int o = 32; o > 0; o >>= 1) {
                    const uint64_t y = __shfl_xor(k, o, kWave);
                    k = y < k ? y : k;
                }
                if (k == kKeyMax) break;
                const uint32_t pick = static_cast<uint32_t>(k);
                if (lane == pick) taken = true;
                h_cell = __shfl(my_cell, static_cast<int>(pick), kWave);
                h_s = __shfl(my_s, static_cast<int>(pick), kWave);
                if (lane == 0) hout[nh] = h_cell;
                ++nh;
            }
            for (uint32_t j = nh + lane; j < ma; j += kWave) hout[j] = 0xFFFFFFFFu;
        } else {
            // the best r, cut at best - spill_margin (src/index.rs:2496-2508)
            const uint32_t r = min(ma, ncand);
            const float cutoff = __shfl(my_s, 0, kWave) - a.spill_margin;
            const bool take = lane < r && my_s >= cutoff;
            const uint64_t tm = __ballot(take);
            if (take) hout[lanes_below(tm)] = my_cell;
            for (uint32_t j = __popcll(tm) + lane; j < ma; j += kWave) hout[j] = 0xFFFFFFFFu;
        }
    }
}

}  // namespace maivs_dev
