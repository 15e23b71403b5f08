/*
 * The oracle: a CPU restatement of MAIVS's batched cell-major search, used only by the tests,
 * by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, to check the GPU's results and as
 * the timed CPU baseline. Never linked into or called by the product library.
 *
 * Every function cites the reference file:line (V47VANSH/MAIVS) it restates. The arena and
 * parameters are the same POD structs the GPU library takes (include/maivs_gpu.h).
 */
#ifndef MAIVS_ORACLE_H
#define MAIVS_ORACLE_H

#include <stdint.h>

#include "../include/maivs_gpu.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- kernels (src/quantize.rs, src/index.rs:41-343) ---- */
void orc_make_signs(uint32_t dim_pad, uint64_t seed, float* out /* 2*dim_pad */);
void orc_fht(float* a, uint32_t n);
void orc_rotate(const float* v, uint32_t dim, const float* signs, uint32_t dim_pad, float* out);
void orc_pack_signs(const float* rot, uint32_t n, uint64_t* out, uint32_t nw);
uint32_t orc_hamming(const uint64_t* a, const uint64_t* b, uint32_t nw);
void orc_fs_query(const float* rq, uint32_t n_rq, uint32_t nw, uint8_t* lut, float* delta, float* bias);
float orc_fs_estimate(float delta, float bias, uint32_t sum);
void orc_fs_pack_block(const uint64_t* codes, uint32_t ncodes, uint32_t nw, uint8_t* out);
void orc_fs_unpack(const uint8_t* block, uint32_t lane, uint32_t nw, uint64_t* out);
void orc_fs_block_sums(const uint8_t* block, const uint8_t* lut, uint32_t npairs, uint16_t* out);
void orc_fs_block_sums_scalar(const uint8_t* block, const uint8_t* lut, uint32_t npairs, uint16_t* out);
float orc_dot_f32(const float* a, const float* b, uint32_t n);
float orc_dot_f32_u8(const float* qs, const uint8_t* v, uint32_t n);
uint32_t orc_hamming_cutoff(const uint16_t* hs, const uint8_t* keep, uint32_t n, uint32_t want, uint32_t bits);

/* ---- the path ---- */
/* route_batch, src/index.rs:1873-1980. chosen/cscore nq x nprobe (tail UINT32_MAX / NaN). */
int orc_route_batch(const maivs_arena_desc* a, const float* q, uint32_t nq, const maivs_search_params* p,
                    uint32_t nthreads, uint64_t* qbits, uint32_t* chosen, float* cscore, uint32_t* nchosen);

/* search_batch_cellmajor + rerank_exact, src/index.rs:1999-2311, 1309-1378.
 * out nq x k slots / scores, best first, ties by ascending slot, padded UINT32_MAX / -inf.
 * p->route_mode 0 routes with route_batch; 1 routes each query with route_query (tree, else every
 * live cell), as the reference does when route_batch returns None (:2105-2124). */
int orc_search_batch(const maivs_arena_desc* a, const float* q, uint32_t nq, const maivs_search_params* p,
                     uint32_t nthreads, uint32_t* out_slots, float* out_scores);

/* The per-query path: route_query + search_one + rerank_exact (src/index.rs:1168-1305,
 * 1381-1864, 1309-1378) for the binary FastScan configuration, every query on its own. Routing
 * uses a->tree when it has levels (src/tree.rs:559-628), else (p->route_mode 0 with a->cent_bits)
 * the two-stage shortlist with want = nprobe * shortlist_mult, else every live cell. out nq x k as
 * orc_search_batch. */
int orc_search_one(const maivs_arena_desc* a, const float* q, uint32_t nq, const maivs_search_params* p,
                   uint32_t nthreads, uint32_t* out_slots, float* out_scores);

/* route_query alone: chosen / cscore nq x nprobe (tail UINT32_MAX / NaN), nchosen nq. */
int orc_route_query(const maivs_arena_desc* a, const float* q, uint32_t nq, const maivs_search_params* p,
                    uint32_t nthreads, uint32_t* chosen, float* cscore, uint32_t* nchosen);

/* Intermediates of the last orc_search_batch (same layout as maivs_gpu_last_candidates). */
int orc_last_candidates(uint32_t* tau, uint32_t* rest_end, uint32_t* cut, uint32_t* ncand, uint32_t* cand_slots,
                        uint32_t* cand_d, uint64_t cap);

/* Total candidates of the last call (to size the arrays above). */
uint64_t orc_last_total_candidates(void);

/* Not a restatement: checks the host libm that the GPU build's radii rely on. Number of f32 x in
 * [-1, 1) whose successor y has acosf(y) > acosf(x) (0: acosf is non-increasing there);
 * *first_bad_bits = the first such x's bit pattern, or UINT64_MAX. */
uint64_t orc_acosf_violations(uint32_t nthreads, uint64_t* first_bad_bits);

#ifdef __cplusplus
}
#endif
#endif
