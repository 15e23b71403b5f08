// What the placement (build.hip) calls in the row store (store.hip).
#pragma once

#include <stdint.h>

struct maivs_gpu_ctx;

namespace maivs_host {

// Writes rows i < n of the placed batch (device buffers: f32 rows, sign codes, i8 / SQ8 rows) to
// the store at h_slots[i], growing it as needed.
int store_write(maivs_gpu_ctx* ctx, const uint32_t* h_slots, uint32_t n, const float* d_x, const uint64_t* d_bits,
                const int8_t* d_codes, bool has_codes);

// Adds each row of d_x (n x d, device) to h_sums (M x d, host, in and out) at its primary home
// d_homes[i * ma], the rows of a cell in input order.
int cell_sums(maivs_gpu_ctx* ctx, const float* d_x, const uint32_t* d_homes, uint32_t ma, uint32_t n, uint32_t M,
              uint32_t d, float* h_sums);

}  // namespace maivs_host
