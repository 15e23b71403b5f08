// libmaivs_gpu.so, index build: the batched spherical k-means behind train_centroids and the
// centroid tree (src/tree.rs:179-348, 354-460), bit-identical to the reference's CPU arithmetic.
//
// One call runs every job of a batch together, iteration by iteration (jobs with fewer
// iterations drop out):
//   km_zero      clear the cluster counts
//   km_assign    one lane per point: first best centroid by the exact 8-lane FMA dot; counts
//   radix sort   stable sort of (cluster, point position) -> each cluster's points in point order
//   km_starts    first sorted position of each cluster
//   km_update    one workgroup per non-empty cluster: in-order sum, norm, division
//   km_reseed    one thread per job: empty clusters take xorshift64 picks, in cluster order
#include <hip/hip_runtime.h>

#include <rocprim/device/device_radix_sort.hpp>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "build_kernels.h"
#include "ctx.h"
#include "store.h"

using namespace maivs_host;

namespace {

// Device buffers of one k-means call, freed when it returns.
struct Scratch {
    maivs_gpu_ctx* ctx;
    std::vector<void*> allocs;
    explicit Scratch(maivs_gpu_ctx* c) : ctx(c) {}
    ~Scratch() {
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

__global__ void km_iota_kernel(uint32_t* p, uint32_t n) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = i;
}

// best = 0, key = the job's first cluster, pos = the point itself: valid sort input before any
// assignment (jobs with zero iterations keep it).
__global__ void km_prime_kernel(KmArgs a) {
    for (uint32_t b = blockIdx.x; b < a.n_jobs; b += gridDim.x) {
        const KmJob J = a.jobs[b];
        for (uint32_t i = threadIdx.x; i < J.n; i += blockDim.x) {
            const uint32_t p = J.first + i;
            a.best[p] = 0;
            a.key[p] = J.coff;
            a.pos[p] = p;
        }
    }
}

uint32_t grid_for(uint64_t n, uint32_t threads) {
    return static_cast<uint32_t>(std::min<uint64_t>((n + threads - 1) / threads, 65535u));
}

}  // namespace

extern "C" int maivs_gpu_kmeans(maivs_gpu_ctx* ctx, const float* x, uint64_t n_rows, uint32_t dim,
                                const uint32_t* rows, const maivs_kmeans_job* jobs, uint32_t n_jobs,
                                uint32_t* assign, float* cents) {
    if (!ctx) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    if (!x || !jobs || !assign || !cents || n_jobs == 0 || n_rows == 0)
        return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_kmeans: null buffer or empty batch");
    if (dim == 0 || dim > 256 * kKmMaxDimPerThread)
        return fail(ctx, MAIVS_ERR_UNSUPPORTED, "maivs_gpu_kmeans: dim %u outside [1, %u]", dim, 256 * kKmMaxDimPerThread);
    std::vector<KmJob> hj(n_jobs);
    uint64_t n_points = 0, sum_k = 0;
    uint32_t max_iters = 0;
    for (uint32_t j = 0; j < n_jobs; ++j) {
        const maivs_kmeans_job& J = jobs[j];
        if (J.first != n_points || J.n == 0 || J.k == 0 || J.k > J.n)
            return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_kmeans: job %u (first %u, n %u, k %u) does not tile the rows",
                        j, J.first, J.n, J.k);
        hj[j] = KmJob{J.first, J.n, J.k, J.iters, static_cast<uint32_t>(sum_k), {0, 0, 0}};
        n_points += J.n;
        sum_k += J.k;
        max_iters = std::max(max_iters, J.iters);
    }
    if (n_points >= (1ull << 31) || sum_k >= (1ull << 31))
        return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_kmeans: batch too large");
    if (rows) {
        for (uint64_t p = 0; p < n_points; ++p)
            if (rows[p] >= n_rows) return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_kmeans: row id %u >= n_rows", rows[p]);
    } else if (n_points > n_rows) {
        return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_kmeans: more points than rows");
    }
    const uint32_t np = static_cast<uint32_t>(n_points), sk = static_cast<uint32_t>(sum_k);
    // assignment workgroups never straddle two jobs
    std::vector<uint32_t> blk_job, blk_start, c_job(sk);
    for (uint32_t j = 0; j < n_jobs; ++j) {
        for (uint32_t s = 0; s < hj[j].n; s += kKmThreads) {
            blk_job.push_back(j);
            blk_start.push_back(s);
        }
        for (uint32_t c = 0; c < hj[j].k; ++c) c_job[hj[j].coff + c] = j;
    }
    std::vector<uint64_t> state(n_jobs);
    for (uint32_t j = 0; j < n_jobs; ++j) state[j] = jobs[j].seed | 1ull;

    HIP_TRY(ctx, hipSetDevice(ctx->device));
    Scratch S(ctx);
    KmArgs a{};
    a.d = dim;
    a.n_points = np;
    a.sum_k = sk;
    a.n_jobs = n_jobs;
    float *d_x = nullptr, *d_cents = nullptr;
    uint32_t *d_rows = nullptr, *d_best, *d_key, *d_pos, *d_cnt, *d_start, *d_skey, *d_spos, *d_bj, *d_bs, *d_cj;
    KmJob* d_jobs = nullptr;
    uint64_t* d_state = nullptr;
    int rc = 0;
    if ((rc = S.upload(&d_x, x, n_rows * dim)) || (rc = S.upload(&d_jobs, hj.data(), n_jobs)) ||
        (rc = S.upload(&d_bj, blk_job.data(), blk_job.size())) || (rc = S.upload(&d_bs, blk_start.data(), blk_start.size())) ||
        (rc = S.upload(&d_cj, c_job.data(), sk)) || (rc = S.upload(&d_state, state.data(), n_jobs)) ||
        (rc = S.alloc(&d_cents, static_cast<size_t>(sk) * dim)) || (rc = S.alloc(&d_best, np)) ||
        (rc = S.alloc(&d_key, np)) || (rc = S.alloc(&d_pos, np)) || (rc = S.alloc(&d_cnt, sk)) ||
        (rc = S.alloc(&d_start, sk)) || (rc = S.alloc(&d_skey, np)) || (rc = S.alloc(&d_spos, np)))
        return rc;
    if (rows) {
        if ((rc = S.upload(&d_rows, rows, np))) return rc;
    } else {
        if ((rc = S.alloc(&d_rows, np))) return rc;
        km_iota_kernel<<<grid_for(np, 256), 256, 0, ctx->stream>>>(d_rows, np);
    }
    a.x = d_x;
    a.rows = d_rows;
    a.jobs = d_jobs;
    a.blk_job = d_bj;
    a.blk_start = d_bs;
    a.c_job = d_cj;
    a.cents = d_cents;
    a.best = d_best;
    a.key = d_key;
    a.pos = d_pos;
    a.cnt = d_cnt;
    a.start = d_start;
    a.skey = d_skey;
    a.spos = d_spos;
    a.state = d_state;

    unsigned end_bit = 1;
    while (end_bit < 32 && (1ull << end_bit) < sum_k) ++end_bit;
    size_t tmp_bytes = 0;
    HIP_TRY(ctx, rocprim::radix_sort_pairs(nullptr, tmp_bytes, d_key, d_skey, d_pos, d_spos, np, 0u, end_bit,
                                           ctx->stream));
    void* d_tmp = nullptr;
    if ((rc = S.alloc(reinterpret_cast<uint8_t**>(&d_tmp), tmp_bytes))) return rc;

    km_init_kernel<<<sk, 256, 0, ctx->stream>>>(a);
    km_prime_kernel<<<std::min<uint32_t>(n_jobs, 4096), 256, 0, ctx->stream>>>(a);
    const size_t upd_lds = (static_cast<size_t>(dim) + 1) * sizeof(float);
    for (uint32_t it = 0; it < max_iters; ++it) {
        km_zero_kernel<<<grid_for(sk, 256), 256, 0, ctx->stream>>>(d_cnt, sk);
        if (dim % 4 == 0)
            km_assign_kernel<true><<<static_cast<uint32_t>(blk_job.size()), kKmThreads, 0, ctx->stream>>>(a, it);
        else
            km_assign_kernel<false><<<static_cast<uint32_t>(blk_job.size()), kKmThreads, 0, ctx->stream>>>(a, it);
        HIP_TRY(ctx, rocprim::radix_sort_pairs(d_tmp, tmp_bytes, d_key, d_skey, d_pos, d_spos, np, 0u, end_bit,
                                               ctx->stream));
        km_starts_kernel<<<grid_for(np, 256), 256, 0, ctx->stream>>>(a, np);
        km_update_kernel<<<sk, 256, upd_lds, ctx->stream>>>(a, it);
        km_reseed_kernel<<<(n_jobs + 63) / 64, 64, 0, ctx->stream>>>(a, it);
    }
    HIP_TRY(ctx, hipGetLastError());
    HIP_TRY(ctx, hipMemcpyAsync(assign, d_best, static_cast<size_t>(np) * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(cents, d_cents, static_cast<size_t>(sk) * dim * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

extern "C" int maivs_gpu_place(maivs_gpu_ctx* ctx, const maivs_place_desc* pd, const float* x, uint32_t n,
                               uint32_t* homes, uint64_t* bits, int8_t* codes) {
    if (!ctx) return MAIVS_ERR_ARG;
    std::lock_guard<std::mutex> lk(ctx->mu);
    if (!pd || !x || !homes || !bits || !pd->rot_signs || !pd->centroids)
        return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_place: null buffer");
    if (n == 0) return 0;
    const maivs_place_desc& D = *pd;
    const maivs_tree_desc& T = D.tree;
    const uint32_t d = D.dim, P = D.dim_pad, W = D.n_words, M = D.n_cells, ma = D.max_assign;
    if (d == 0 || P < 64 || P > 2048 || (P & (P - 1)) != 0 || d > P || W == 0 || W * 64 > P || M == 0)
        return fail(ctx, MAIVS_ERR_UNSUPPORTED, "maivs_gpu_place: dim %u / dim_pad %u / words %u / cells %u", d, P, W, M);
    if (ma == 0 || ma > 64) return fail(ctx, MAIVS_ERR_UNSUPPORTED, "maivs_gpu_place: max_assign %u outside [1, 64]", ma);
    if (D.code_mode > 2 || (D.code_mode && !codes) || (D.code_mode == 1 && (!D.sq_min || !D.sq_step)))
        return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_place: bad code mode");
    const bool has_tree = T.n_levels > 0;
    const uint32_t want = has_tree ? std::max(D.tree_want, 1u) : 1u;
    std::vector<uint32_t> beams(T.n_levels, 0);
    if (has_tree) {
        if (!T.level_n) return fail(ctx, MAIVS_ERR_ARG, "maivs_gpu_place: incomplete tree");
        tree_beams(T.level_n, T.n_levels, T.beam_frac, T.min_beam, want, beams.data());
    }
    uint32_t cap = 1;
    for (uint32_t b : beams) cap = std::max(cap, b);
    const uint32_t words = place_lds_words(P, d, W, cap, want);
    const uint32_t lds_per_wave = (words * 4 + 15) & ~15u;
    if (static_cast<size_t>(lds_per_wave) * kPlaceWaves > 160 * 1024)
        return fail(ctx, MAIVS_ERR_UNSUPPORTED, "maivs_gpu_place: %u bytes of LDS per wave", lds_per_wave);

    HIP_TRY(ctx, hipSetDevice(ctx->device));
    Scratch S(ctx);
    PlaceArgs a{};
    float *d_x, *d_signs, *d_cents, *d_sqmin = nullptr, *d_sqstep = nullptr;
    uint32_t *d_homes, *d_beams = nullptr;
    uint64_t* d_bits;
    int8_t* d_codes = nullptr;
    int rc = 0;
    if ((rc = S.upload(&d_x, x, static_cast<size_t>(n) * d)) || (rc = S.upload(&d_signs, D.rot_signs, 2 * static_cast<size_t>(P))) ||
        (rc = S.upload(&d_cents, D.centroids, static_cast<size_t>(M) * d)) || (rc = S.alloc(&d_homes, static_cast<size_t>(n) * ma)) ||
        (rc = S.alloc(&d_bits, static_cast<size_t>(n) * W)))
        return rc;
    if (D.code_mode) {
        if ((rc = S.alloc(&d_codes, static_cast<size_t>(n) * d))) return rc;
        if (D.code_mode == 1 && ((rc = S.upload(&d_sqmin, D.sq_min, d)) || (rc = S.upload(&d_sqstep, D.sq_step, d)))) return rc;
    }
    if (has_tree) {
        if ((rc = upload_tree(ctx, S.allocs, &T, W, M, &a.tree, nullptr)) || (rc = S.upload(&d_beams, beams.data(), beams.size())))
            return rc;
    }
    a.x = d_x;
    a.signs = d_signs;
    a.cents = d_cents;
    a.beams = d_beams;
    a.sq_min = d_sqmin;
    a.sq_step = d_sqstep;
    a.homes = d_homes;
    a.bits = d_bits;
    a.codes = d_codes;
    a.fht_scale = 1.0f / std::sqrt(static_cast<float>(P));
    a.spill_lambda = D.spill_lambda;
    a.spill_margin = D.spill_margin;
    a.quant_scale = D.quant_scale;
    a.n = n;
    a.d = d;
    a.P = P;
    a.W = W;
    a.M = M;
    a.want = want;
    a.ma = ma;
    a.kept_cap = cap;
    a.code_mode = D.code_mode;
    a.lds_per_wave = lds_per_wave;
    const uint32_t blocks = static_cast<uint32_t>(std::min<uint64_t>((n + kPlaceWaves - 1) / kPlaceWaves, 4096));
    const size_t lds = static_cast<size_t>(lds_per_wave) * kPlaceWaves;
    switch (P / 64) {
        case 1: place_kernel<1><<<blocks, kPlaceWaves * kWave, lds, ctx->stream>>>(a); break;
        case 2: place_kernel<2><<<blocks, kPlaceWaves * kWave, lds, ctx->stream>>>(a); break;
        case 4: place_kernel<4><<<blocks, kPlaceWaves * kWave, lds, ctx->stream>>>(a); break;
        case 8: place_kernel<8><<<blocks, kPlaceWaves * kWave, lds, ctx->stream>>>(a); break;
        case 16: place_kernel<16><<<blocks, kPlaceWaves * kWave, lds, ctx->stream>>>(a); break;
        default: place_kernel<32><<<blocks, kPlaceWaves * kWave, lds, ctx->stream>>>(a); break;
    }
    HIP_TRY(ctx, hipGetLastError());
    HIP_TRY(ctx, hipMemcpyAsync(homes, d_homes, static_cast<size_t>(n) * ma * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipMemcpyAsync(bits, d_bits, static_cast<size_t>(n) * W * 8, hipMemcpyDeviceToHost, ctx->stream));
    if (D.code_mode)
        HIP_TRY(ctx, hipMemcpyAsync(codes, d_codes, static_cast<size_t>(n) * d, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    // the rows into the row store, and the primary sums, while the batch is on the device
    if (D.store_slots && (rc = store_write(ctx, D.store_slots, n, d_x, d_bits, d_codes, D.code_mode != 0))) return rc;
    if (D.sums) {
        for (uint32_t i = 0; i < n; ++i)
            if (homes[static_cast<size_t>(i) * ma] >= M) return fail(ctx, MAIVS_ERR_HIP, "maivs_gpu_place: vector %u has no home", i);
        if ((rc = cell_sums(ctx, d_x, d_homes, ma, n, M, d, D.sums))) return rc;
    }
    return 0;
}
