// The oracle (test infrastructure; see oracle.h): CPU restatement of MAIVS's batched
// cell-major search path. Compiled with -O2 -mavx2 -mfma -ffp-contract=off so that an FMA
// appears exactly where the reference uses _mm256_fmadd_ps, and libm's acosf / cosf / expf are
// the ones the reference's f32::acos / cos / exp reach on Linux.
//
// Parity status (also in the repository's design notes): every function here is pinned by
// the tests under tests/ (closed forms, brute force, invariants); the one boundary no check
// can pin is the reference's unstable-sort order among exactly equal f32 scores, which this
// restatement fixes to (score desc, id asc).
#include "oracle.h"

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

constexpr uint32_t kSeedCells = 8;   // SEED_CELLS, src/index.rs:2018
constexpr uint32_t kQB = 32;         // route tile, src/index.rs:1878

template <class F>
void par_for(uint32_t nthreads, size_t n, F&& f, size_t grain = 1) {
    if (n == 0) return;
    size_t nt = std::min<size_t>(std::max<uint32_t>(nthreads, 1), (n + grain - 1) / grain);
    if (nt <= 1) {
        for (size_t i = 0; i < n; ++i) f(i);
        return;
    }
    std::atomic<size_t> next{0};
    auto run = [&]() {
        for (;;) {
            size_t s = next.fetch_add(grain);
            if (s >= n) return;
            size_t e = std::min(n, s + grain);
            for (size_t i = s; i < e; ++i) f(i);
        }
    };
    std::vector<std::thread> th;
    for (size_t t = 1; t < nt; ++t) th.emplace_back(run);
    run();
    for (auto& t : th) t.join();
}

inline float hsum8(__m256 v) {  // hsum_ps, src/index.rs:58-65
    __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 0x55));
    return _mm_cvtss_f32(s);
}

struct Cand {
    uint32_t d, slot;
};

struct LastRun {
    std::vector<uint32_t> tau, rest_end, cut;
    std::vector<std::vector<Cand>> cands;
} g_last;
// whether orc_search_batch keeps each query's candidates for orc_last_candidates (the timing
// runs of the CPU baseline switch it off: the reference keeps nothing of the kind)
bool g_record = true;

}  // namespace

extern "C" {

// src/quantize.rs:132-148: splitmix64, +1 when the low bit is 0.
void orc_make_signs(uint32_t dim_pad, uint64_t seed, float* out) {
    uint64_t st = seed;
    for (uint32_t i = 0; i < 2 * dim_pad; ++i) {
        st += 0x9E3779B97F4A7C15ull;
        uint64_t z = st;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z = z ^ (z >> 31);
        out[i] = (z & 1ull) ? -1.0f : 1.0f;
    }
}

// src/quantize.rs:71-126. Levels 1, 2, 4 inside 8-blocks, then contiguous halves h = 8 .. n/2,
// then the multiply by 1/sqrt(n) (f32).
void orc_fht(float* a, uint32_t n) {
    uint32_t h = 1;
    if (n >= 8 && n % 8 == 0) {
        for (uint32_t b = 0; b < n; b += 8) {
            float x[8];
            for (int i = 0; i < 8; ++i) x[i] = a[b + i];
            for (uint32_t hh : {1u, 2u, 4u})
                for (uint32_t i = 0; i < 8; i += hh << 1)
                    for (uint32_t j = i; j < i + hh; ++j) {
                        float u = x[j], v = x[j + hh];
                        x[j] = u + v;
                        x[j + hh] = u - v;
                    }
            for (int i = 0; i < 8; ++i) a[b + i] = x[i];
        }
        h = 8;
        for (; h < n; h <<= 1)
            for (uint32_t b = 0; b < n; b += h << 1)
                for (uint32_t j = 0; j < h; ++j) {
                    float x = a[b + j], y = a[b + h + j];
                    a[b + j] = x + y;
                    a[b + h + j] = x - y;
                }
    }
    for (; h < n; h <<= 1)
        for (uint32_t i = 0; i < n; i += h << 1)
            for (uint32_t j = i; j < i + h; ++j) {
                float x = a[j], y = a[j + h];
                a[j] = x + y;
                a[j + h] = x - y;
            }
    float s = 1.0f / std::sqrt(static_cast<float>(n));
    for (uint32_t i = 0; i < n; ++i) a[i] *= s;
}

// src/quantize.rs:152-163
void orc_rotate(const float* v, uint32_t dim, const float* signs, uint32_t dim_pad, float* out) {
    std::memcpy(out, v, dim * sizeof(float));
    std::fill(out + dim, out + dim_pad, 0.0f);
    for (int r = 0; r < 2; ++r) {
        for (uint32_t i = 0; i < dim_pad; ++i) out[i] *= signs[r * dim_pad + i];
        orc_fht(out, dim_pad);
    }
}

// src/quantize.rs:57-67
void orc_pack_signs(const float* rot, uint32_t n, uint64_t* out, uint32_t nw) {
    std::fill(out, out + nw, 0ull);
    uint32_t bits = std::min(nw * 64u, n);
    for (uint32_t i = 0; i < bits; ++i)
        if (rot[i] < 0.0f) out[i >> 6] |= 1ull << (i & 63);
}

// src/quantize.rs:183-201
uint32_t orc_hamming(const uint64_t* a, const uint64_t* b, uint32_t nw) {
    uint32_t s = 0;
    for (uint32_t i = 0; i < nw; ++i) s += static_cast<uint32_t>(_mm_popcnt_u64(a[i] ^ b[i]));
    return s;
}

// FsQuery::new, src/quantize.rs:279-313
void orc_fs_query(const float* rq, uint32_t n_rq, uint32_t nw, uint8_t* lut, float* delta_out, float* bias_out) {
    const uint32_t npos = nw * 16;
    std::vector<float> raw(npos * 16), mins(npos);
    float range = 0.0f;
    for (uint32_t j = 0; j < npos; ++j) {
        float lo = INFINITY, hi = -INFINITY;
        for (uint32_t e = 0; e < 16; ++e) {
            float v = 0.0f;
            for (uint32_t t = 0; t < 4; ++t) {
                uint32_t d = 4 * j + t;
                float x = d < n_rq ? rq[d] : 0.0f;
                v += ((e >> t) & 1u) ? -x : x;
            }
            raw[j * 16 + e] = v;
            lo = std::fmin(lo, v);
            hi = std::fmax(hi, v);
        }
        mins[j] = lo;
        range = std::fmax(range, hi - lo);
    }
    float delta = std::fmax(range / 255.0f, 1e-12f);
    for (uint32_t p = 0; p < npos / 2; ++p)
        for (uint32_t half = 0; half < 2; ++half) {
            uint32_t j = 2 * p + half;
            for (uint32_t e = 0; e < 16; ++e) {
                float q = std::round((raw[j * 16 + e] - mins[j]) / delta);
                q = std::fmin(std::fmax(q, 0.0f), 255.0f);
                lut[p * 32 + half * 16 + e] = static_cast<uint8_t>(q);
            }
        }
    float bias = -0.0f;  // Rust's f32 Sum folds from -0.0
    for (uint32_t j = 0; j < npos; ++j) bias += mins[j];
    *delta_out = delta;
    *bias_out = bias;
}

// FsQuery::estimate, src/quantize.rs:317-319
float orc_fs_estimate(float delta, float bias, uint32_t sum) { return delta * static_cast<float>(sum) + bias; }

// fs_pack_block, src/quantize.rs:238-250 (codes: ncodes x nw words)
void orc_fs_pack_block(const uint64_t* codes, uint32_t ncodes, uint32_t nw, uint8_t* out) {
    auto nibble = [&](uint32_t lane, uint32_t j) -> uint8_t {
        if (lane >= ncodes) return 0;
        return static_cast<uint8_t>((codes[lane * nw + (j >> 4)] >> ((j & 15) * 4)) & 0xF);
    };
    for (uint32_t p = 0; p < nw * 8; ++p)
        for (uint32_t half = 0; half < 2; ++half)
            for (uint32_t i = 0; i < 16; ++i) {
                uint32_t j = 2 * p + half;
                out[p * 32 + half * 16 + i] = static_cast<uint8_t>(nibble(i, j) | (nibble(i + 16, j) << 4));
            }
}

// fs_unpack, src/quantize.rs:254-265
void orc_fs_unpack(const uint8_t* block, uint32_t lane, uint32_t nw, uint64_t* out) {
    std::fill(out, out + nw, 0ull);
    uint32_t i = lane % 16;
    bool hi = lane >= 16;
    for (uint32_t j = 0; j < nw * 16; ++j) {
        uint8_t byte = block[(j / 2) * 32 + (j % 2) * 16 + i];
        uint64_t n = hi ? (byte >> 4) : (byte & 0xF);
        out[j >> 4] |= n << ((j & 15) * 4);
    }
}

// fs_block_sums_scalar, src/quantize.rs:335-349
void orc_fs_block_sums_scalar(const uint8_t* block, const uint8_t* lut, uint32_t npairs, uint16_t* out) {
    std::fill(out, out + 32, static_cast<uint16_t>(0));
    for (uint32_t p = 0; p < npairs; ++p)
        for (uint32_t half = 0; half < 2; ++half) {
            uint32_t base = p * 32 + half * 16;
            for (uint32_t i = 0; i < 16; ++i) {
                uint8_t b = block[base + i];
                out[i] = static_cast<uint16_t>(out[i] + lut[base + (b & 0xF)]);
                out[i + 16] = static_cast<uint16_t>(out[i + 16] + lut[base + (b >> 4)]);
            }
        }
}

// fs_block_sums_avx2, src/quantize.rs:351-386: pshufb per half, u8 results folded into u16
// lanes as even + 256*odd and odd, then un-mixed.
void orc_fs_block_sums(const uint8_t* block, const uint8_t* lut, uint32_t npairs, uint16_t* out) {
    const __m256i mask = _mm256_set1_epi8(0x0F);
    __m256i a0l = _mm256_setzero_si256(), a1l = _mm256_setzero_si256();
    __m256i a0h = _mm256_setzero_si256(), a1h = _mm256_setzero_si256();
    for (uint32_t p = 0; p < npairs; ++p) {
        __m256i c = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(block + p * 32));
        __m256i l = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(lut + p * 32));
        __m256i rl = _mm256_shuffle_epi8(l, _mm256_and_si256(c, mask));
        __m256i rh = _mm256_shuffle_epi8(l, _mm256_and_si256(_mm256_srli_epi16(c, 4), mask));
        a0l = _mm256_add_epi16(a0l, rl);
        a1l = _mm256_add_epi16(a1l, _mm256_srli_epi16(rl, 8));
        a0h = _mm256_add_epi16(a0h, rh);
        a1h = _mm256_add_epi16(a1h, _mm256_srli_epi16(rh, 8));
    }
    auto fold = [](__m256i a0, __m256i a1, uint16_t* dst) {
        __m256i even = _mm256_sub_epi16(a0, _mm256_slli_epi16(a1, 8));
        __m128i e = _mm_add_epi16(_mm256_castsi256_si128(even), _mm256_extracti128_si256(even, 1));
        __m128i o = _mm_add_epi16(_mm256_castsi256_si128(a1), _mm256_extracti128_si256(a1, 1));
        _mm_storeu_si128(reinterpret_cast<__m128i*>(dst), _mm_unpacklo_epi16(e, o));
        _mm_storeu_si128(reinterpret_cast<__m128i*>(dst + 8), _mm_unpackhi_epi16(e, o));
    };
    fold(a0l, a1l, out);
    fold(a0h, a1h, out + 16);
}

// dot_f32_avx2, src/index.rs:136-152
float orc_dot_f32(const float* a, const float* b, uint32_t n) {
    __m256 acc = _mm256_setzero_ps();
    uint32_t i = 0;
    for (; i + 8 <= n; i += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc);
    float s = hsum8(acc);
    for (; i < n; ++i) s += a[i] * b[i];
    return s;
}

// dot_f32_u8_avx2, src/index.rs:278-294
float orc_dot_f32_u8(const float* qs, const uint8_t* v, uint32_t n) {
    __m256 acc = _mm256_setzero_ps();
    uint32_t i = 0;
    for (; i + 8 <= n; i += 8) {
        __m256 vf = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_loadl_epi64(reinterpret_cast<const __m128i*>(v + i))));
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(qs + i), vf, acc);
    }
    float s = hsum8(acc);
    for (; i < n; ++i) s += qs[i] * static_cast<float>(v[i]);
    return s;
}

// hamming_cutoff, src/index.rs:86-104
uint32_t orc_hamming_cutoff(const uint16_t* hs, const uint8_t* keep, uint32_t n, uint32_t want, uint32_t bits) {
    if (want == 0) return 0;
    std::vector<uint32_t> hist(bits + 1, 0);
    for (uint32_t i = 0; i < n; ++i)
        if (keep[i]) hist[hs[i]] += 1;
    size_t cum = 0;
    for (uint32_t t = 0; t <= bits; ++t) {
        cum += hist[t];
        if (cum >= want) return t;
    }
    return bits;
}

}  // extern "C"

namespace {

struct Arena {
    const maivs_arena_desc* a;
    uint32_t d, P, nw, M, npos, maxk, bb;
    std::vector<uint8_t> live;
    uint32_t n_live = 0;
    explicit Arena(const maivs_arena_desc* ad) : a(ad) {
        d = ad->dim;
        P = ad->dim_pad;
        nw = ad->n_words;
        M = ad->n_cells;
        npos = nw * 16;
        maxk = 255 * npos;
        bb = nw * 256;
        live.resize(M);
        for (uint32_t c = 0; c < M; ++c) {
            live[c] = ad->mem_off[c + 1] > ad->mem_off[c];
            n_live += live[c];
        }
    }
    uint32_t mem_len(uint32_t c) const { return a->mem_off[c + 1] - a->mem_off[c]; }
};

inline bool score_before(const std::pair<uint32_t, float>& x, const std::pair<uint32_t, float>& y) {
    if (x.second != y.second) return x.second > y.second;
    return x.first < y.first;
}

// cent_score (src/index.rs:777-800): SQ8 copy when present, else the f32 centroid.
float cent_score(const Arena& A, uint32_t c, const float* q, const float* cqs, float cqbase) {
    if (A.a->cent_sq8) return orc_dot_f32_u8(cqs, A.a->cent_sq8 + static_cast<size_t>(c) * A.d, A.d) + cqbase;
    return orc_dot_f32(q, A.a->centroids + static_cast<size_t>(c) * A.d, A.d);
}

struct Routed {
    std::vector<uint64_t> bits;
    std::vector<uint32_t> chosen;
    std::vector<float> cscore;
};

struct QRoute {
    std::vector<uint64_t> bits;
    std::vector<float> rot;
    std::vector<uint32_t> chosen;
    std::vector<float> cscore;
};

QRoute route_query(const Arena& A, const float* q, const maivs_search_params* p);

// route_batch, src/index.rs:1873-1980
std::vector<Routed> route_batch(const Arena& A, const float* data, uint32_t nq, const maivs_search_params* p,
                                uint32_t nthreads) {
    const uint32_t d = A.d, nw = A.nw, M = A.M, cl = nw * 64;
    std::vector<Routed> out(nq);
    uint32_t want_c = std::min<uint32_t>(p->nprobe * std::max<uint32_t>(p->shortlist_mult, 2), A.n_live);
    if (want_c == 0) {
        for (auto& r : out) r.bits.assign(nw, 0);
        return out;
    }
    std::vector<uint64_t> qbits(static_cast<size_t>(nq) * nw);
    par_for(nthreads, nq, [&](size_t qi) {
        std::vector<float> rot(A.P);
        orc_rotate(data + qi * d, d, A.a->rot_signs, A.P, rot.data());
        orc_pack_signs(rot.data(), A.P, &qbits[qi * nw], nw);
    }, 16);
    std::vector<std::vector<uint32_t>> shortlists(nq);
    uint32_t ntile = (nq + kQB - 1) / kQB;
    par_for(nthreads, ntile, [&](size_t ti) {
        uint32_t q0 = static_cast<uint32_t>(ti) * kQB, b = std::min(kQB, nq - q0);
        std::vector<uint16_t> hs(static_cast<size_t>(b) * M);
        for (uint32_t c = 0; c < M; ++c) {
            const uint64_t* cc = A.a->cent_bits + static_cast<size_t>(c) * nw;
            for (uint32_t bi = 0; bi < b; ++bi)
                hs[static_cast<size_t>(bi) * M + c] =
                    static_cast<uint16_t>(orc_hamming(&qbits[static_cast<size_t>(q0 + bi) * nw], cc, nw));
        }
        for (uint32_t bi = 0; bi < b; ++bi) {
            const uint16_t* row = &hs[static_cast<size_t>(bi) * M];
            uint32_t cut = orc_hamming_cutoff(row, A.live.data(), M, want_c, cl);
            auto& sl = shortlists[q0 + bi];
            for (uint32_t c = 0; c < M; ++c)
                if (A.live[c] && row[c] <= cut) sl.push_back(c);
        }
    });
    par_for(nthreads, nq, [&](size_t qi) {
        const float* q = data + qi * d;
        std::vector<float> cqs(d, 0.0f);
        float cqbase = 0.0f;
        if (A.a->cent_sq8) {
            for (uint32_t j = 0; j < d; ++j) {
                cqs[j] = q[j] * A.a->csq_step[j];
                cqbase += q[j] * A.a->csq_min[j];
            }
        }
        std::vector<std::pair<uint32_t, float>> cs;
        for (uint32_t c : shortlists[qi]) cs.emplace_back(c, cent_score(A, c, q, cqs.data(), cqbase));
        uint32_t cap = std::min<uint32_t>(p->nprobe, static_cast<uint32_t>(cs.size()));
        Routed& r = out[qi];
        r.bits.assign(&qbits[qi * nw], &qbits[qi * nw] + nw);
        if (cap == 0) return;
        if (cap < cs.size()) {
            std::nth_element(cs.begin(), cs.begin() + (cap - 1), cs.end(), score_before);
            cs.resize(cap);
        }
        std::sort(cs.begin(), cs.end(), score_before);
        if (p->target_confidence >= 1.0f) {
            for (auto& e : cs) r.chosen.push_back(e.first);
        } else {
            float max_s = cs[0].second;
            float z = -0.0f;  // f32 Sum
            for (auto& e : cs) z += std::exp((e.second - max_s) * p->beta);
            float cum = 0.0f;
            for (auto& e : cs) {
                r.chosen.push_back(e.first);
                cum += std::exp((e.second - max_s) * p->beta) / (z + 1e-9f);
                if (cum >= p->target_confidence) break;
            }
        }
        for (size_t i = 0; i < r.chosen.size(); ++i) r.cscore.push_back(cs[i].second);
    }, 8);
    return out;
}

struct QState {
    std::vector<uint32_t> rest;
    std::vector<Cand> seed;
    uint32_t tau;
    uint32_t rest_end;
    std::vector<uint8_t> lut;
    float delta, bias;
    std::vector<uint64_t> probed;
};

}  // namespace

extern "C" {

int orc_route_batch(const maivs_arena_desc* a, const float* q, uint32_t nq, const maivs_search_params* p,
                    uint32_t nthreads, uint64_t* qbits, uint32_t* chosen, float* cscore, uint32_t* nchosen) {
    if (!a || !p || (!q && nq) || !a->cent_bits) return MAIVS_ERR_ARG;
    Arena A(a);
    std::vector<Routed> r = route_batch(A, q, nq, p, nthreads);
    for (uint32_t i = 0; i < nq; ++i) {
        if (qbits) std::memcpy(qbits + static_cast<size_t>(i) * A.nw, r[i].bits.data(), A.nw * 8);
        if (nchosen) nchosen[i] = static_cast<uint32_t>(r[i].chosen.size());
        for (uint32_t j = 0; j < p->nprobe; ++j) {
            bool ok = j < r[i].chosen.size();
            if (chosen) chosen[static_cast<size_t>(i) * p->nprobe + j] = ok ? r[i].chosen[j] : UINT32_MAX;
            if (cscore) cscore[static_cast<size_t>(i) * p->nprobe + j] = ok ? r[i].cscore[j] : NAN;
        }
    }
    return 0;
}

// search_batch_cellmajor (src/index.rs:1999-2311) with the FastScan scan and rerank_exact.
int orc_search_batch(const maivs_arena_desc* a, const float* data, uint32_t nq, const maivs_search_params* p,
                     uint32_t nthreads, uint32_t* out_slots, float* out_scores) {
    if (!a || !p || (!data && nq) || (p->route_mode == 0 && !a->cent_bits) || !a->fs_codes || !a->fs_off || p->k == 0)
        return MAIVS_ERR_ARG;
    Arena A(a);
    const uint32_t d = A.d, nw = A.nw, M = A.M, dp = A.maxk, k = p->k;
    const uint32_t target = std::max<uint32_t>(k * std::max<uint32_t>(p->rerank_factor, 1), 1);
    const uint32_t ma = a->max_assign;
    const bool poly = ma > 1;
    const uint32_t mwords = (M + 63) / 64;
    const uint32_t npairs = A.npos / 2;

    auto canonical = [&](uint32_t slot, uint32_t ci, const std::vector<uint64_t>& probed) {
        const uint32_t* h = a->slot_cells + static_cast<size_t>(slot) * ma;
        for (uint32_t j = 0; j < ma; ++j)
            if (h[j] != UINT32_MAX && h[j] < ci && ((probed[h[j] >> 6] >> (h[j] & 63)) & 1)) return false;
        return true;
    };
    // keep!: the tag-range predicate of src/index.rs:1428-1439 (filtering = a filter is set and
    // tags exist, :1430-1431). The reference applies it on its per-query path only; here it sits
    // beside the canonical test in the cell-major scan, as the GPU path applies it.
    const bool filtering = p->filter && a->tags;
    auto keep = [&](uint32_t slot) {
        if (!filtering) return true;
        const uint32_t tg = a->tags[slot];
        return tg >= p->tag_lo && tg <= p->tag_hi;
    };
    // scan_cell, FastScan branch, src/index.rs:2048-2074
    auto scan_cell = [&](uint32_t c, const QState& s, uint32_t t, std::vector<Cand>& out) {
        uint32_t len = A.mem_len(c);
        if (len == 0) return;
        const uint32_t* mem = a->members + a->mem_off[c];
        uint32_t b0 = a->fs_off[c], b1 = a->fs_off[c + 1];
        uint16_t sums[32];
        for (uint32_t b = b0; b < b1; ++b) {
            orc_fs_block_sums(a->fs_codes + static_cast<size_t>(b) * A.bb, s.lut.data(), npairs, sums);
            uint32_t base = (b - b0) * 32, nv = std::min<uint32_t>(32, len - base);
            for (uint32_t i = 0; i < nv; ++i) {
                uint32_t dd = dp - sums[i];
                if (dd <= t) {
                    uint32_t slot = mem[base + i];
                    if (keep(slot) && (!poly || canonical(slot, c, s.probed))) out.push_back({dd, slot});
                }
            }
        }
    };
    auto kth_d = [](std::vector<Cand>& v, uint32_t kk) {
        std::nth_element(v.begin(), v.begin() + (kk - 1), v.end(), [](const Cand& x, const Cand& y) { return x.d < y.d; });
        return v[kk - 1].d;
    };

    // 1. route, then per query: FastScan table, seed scan, tau, adaptive cut (src/index.rs:2126-2191)
    // route_batch returns None without two-stage routing: each query routed by route_query instead
    // (src/index.rs:2105-2124)
    std::vector<Routed> probes;
    if (p->route_mode == 0) {
        probes = route_batch(A, data, nq, p, nthreads);
    } else {
        probes.resize(nq);
        par_for(nthreads, nq, [&](size_t qi) {
            QRoute r = route_query(A, data + qi * d, p);
            probes[qi].bits = std::move(r.bits);
            probes[qi].chosen = std::move(r.chosen);
            probes[qi].cscore = std::move(r.cscore);
        }, 4);
    }
    std::vector<QState> st(nq);
    const float norm = std::sqrt(2.0f * static_cast<float>(A.P) / static_cast<float>(M_PI));
    par_for(nthreads, nq, [&](size_t qi) {
        QState& s = st[qi];
        const Routed& r = probes[qi];
        uint32_t nchosen = static_cast<uint32_t>(r.chosen.size());
        uint32_t ns = std::min(kSeedCells, nchosen);
        if (poly) {
            s.probed.assign(mwords, 0);
            for (uint32_t c : r.chosen) s.probed[c >> 6] |= 1ull << (c & 63);
        }
        std::vector<float> rot(A.P);
        orc_rotate(data + qi * d, d, a->rot_signs, A.P, rot.data());
        s.lut.resize(A.npos * 16);
        orc_fs_query(rot.data(), A.P, nw, s.lut.data(), &s.delta, &s.bias);
        for (uint32_t i = 0; i < ns; ++i) scan_cell(r.chosen[i], s, dp, s.seed);
        s.tau = dp;
        if (s.seed.size() >= target) {
            s.tau = kth_d(s.seed, target);
            uint32_t tau = s.tau;
            s.seed.erase(std::remove_if(s.seed.begin(), s.seed.end(), [&](const Cand& e) { return e.d > tau; }),
                         s.seed.end());
        }
        uint32_t rest_end = nchosen;
        if (p->adaptive && s.seed.size() >= target && ns < nchosen) {
            float est = orc_fs_estimate(s.delta, s.bias, dp - s.tau);
            float thr = std::fmin(std::fmax(est / norm, -1.0f), 1.0f);
            std::vector<float> suffix(nchosen + 1, -INFINITY);
            for (uint32_t i = nchosen; i-- > ns;) {
                float cs = std::fmin(std::fmax(r.cscore[i], -1.0f), 1.0f);
                float ang = std::acos(cs);
                float b = std::cos(std::fmax(ang - a->r_bound[r.chosen[i]], 0.0f));
                suffix[i] = std::fmax(b, suffix[i + 1]);
            }
            for (uint32_t i = ns; i < nchosen; ++i)
                if (suffix[i] < thr - p->at_margin) {
                    rest_end = i;
                    break;
                }
        }
        s.rest_end = rest_end;
        s.rest.assign(r.chosen.begin() + ns, r.chosen.begin() + rest_end);
    }, 4);

    // 2. invert: cell -> queries (counting sort, queries ascending), src/index.rs:2193-2213
    std::vector<size_t> start(M + 1, 0);
    for (auto& s : st)
        for (uint32_t c : s.rest) start[c + 1] += 1;
    for (uint32_t c = 0; c < M; ++c) start[c + 1] += start[c];
    std::vector<uint32_t> qof(start[M]);
    {
        std::vector<size_t> pos(start.begin(), start.end() - 1);
        for (uint32_t qi = 0; qi < nq; ++qi)
            for (uint32_t c : st[qi].rest) qof[pos[c]++] = qi;
    }
    // 3. balanced contiguous cell ranges, src/index.rs:2215-2229
    size_t ntask = static_cast<size_t>(std::max<uint32_t>(nthreads, 1)) * 4;
    size_t total = 0;
    std::vector<size_t> work(M);
    for (uint32_t c = 0; c < M; ++c) {
        work[c] = static_cast<size_t>(A.mem_len(c)) * (start[c + 1] - start[c]);
        total += work[c];
    }
    total = std::max<size_t>(total, 1);
    std::vector<std::pair<uint32_t, uint32_t>> ranges;
    {
        size_t acc = 0;
        uint32_t c0 = 0;
        for (uint32_t c = 0; c < M; ++c) {
            acc += work[c];
            if (acc * ntask >= total * (ranges.size() + 1) || c + 1 == M) {
                ranges.emplace_back(c0, c + 1);
                c0 = c + 1;
            }
        }
    }
    // 4. scan with per-worker top-target buffers and a shared per-query cut-off, :2231-2275
    std::vector<std::atomic<uint32_t>> gtau(nq);
    for (uint32_t qi = 0; qi < nq; ++qi) gtau[qi].store(st[qi].tau, std::memory_order_relaxed);
    std::vector<std::vector<std::vector<Cand>>> partials(ranges.size());
    par_for(nthreads, ranges.size(), [&](size_t ri) {
        auto& bufs = partials[ri];
        bufs.assign(nq, {});
        std::vector<uint32_t> ltau(nq, dp);
        for (uint32_t c = ranges[ri].first; c < ranges[ri].second; ++c) {
            if (start[c + 1] == start[c] || A.mem_len(c) == 0) continue;
            for (size_t t = start[c]; t < start[c + 1]; ++t) {
                uint32_t qi = qof[t];
                auto& bq = bufs[qi];
                uint32_t cut = std::min(ltau[qi], gtau[qi].load(std::memory_order_relaxed));
                size_t before = bq.size();
                scan_cell(c, st[qi], cut, bq);
                if (bq.size() > before && (bq.size() >= 2 * static_cast<size_t>(target) ||
                                           (bq.size() >= target && cut == dp))) {
                    cut = std::min(cut, kth_d(bq, target));
                    uint32_t tt = cut;
                    bq.erase(std::remove_if(bq.begin(), bq.end(), [&](const Cand& e) { return e.d > tt; }), bq.end());
                }
                if (bq.size() >= target) {
                    uint32_t cur = gtau[qi].load(std::memory_order_relaxed);
                    while (cut < cur && !gtau[qi].compare_exchange_weak(cur, cut, std::memory_order_relaxed)) {
                    }
                }
                ltau[qi] = cut;
            }
        }
    });
    // 5. merge, exact tie-inclusive cut at target, rerank (src/index.rs:2277-2311, 1309-1378)
    const bool record = g_record;
    g_last.tau.assign(record ? nq : 0, 0);
    g_last.rest_end.assign(record ? nq : 0, 0);
    g_last.cut.assign(record ? nq : 0, 0);
    g_last.cands.assign(record ? nq : 0, {});
    par_for(nthreads, nq, [&](size_t qi) {
        uint32_t t = gtau[qi].load(std::memory_order_relaxed);
        std::vector<Cand> v;
        for (auto& e : st[qi].seed)
            if (e.d <= t) v.push_back(e);
        for (auto& part : partials)
            for (auto& e : part[qi])
                if (e.d <= t) v.push_back(e);
        // reported cut-off: the target-th smallest d of the candidates (the reference's
        // merge only cuts when more than target remain; the set is the same either way)
        uint32_t cut = v.size() >= target ? kth_d(v, target) : dp;
        if (v.size() > target)
            v.erase(std::remove_if(v.begin(), v.end(), [&](const Cand& e) { return e.d > cut; }), v.end());
        const float* q = data + qi * d;
        std::vector<std::pair<uint32_t, float>> scored;
        scored.reserve(v.size());
        if (a->rerank_mode == MAIVS_RERANK_SQ8) {
            std::vector<float> qs(d);
            float base = 0.0f;
            for (uint32_t j = 0; j < d; ++j) {
                qs[j] = q[j] * a->sq_step[j];
                base += q[j] * a->sq_min[j];
            }
            for (auto& e : v)
                scored.emplace_back(e.slot, base + orc_dot_f32_u8(qs.data(), a->sq8_codes + static_cast<size_t>(e.slot) * d, d));
        } else {
            for (auto& e : v)
                scored.emplace_back(e.slot, orc_dot_f32(q, a->vecs_f32 + static_cast<size_t>(e.slot) * d, d));
        }
        uint32_t kk = std::min<uint32_t>(k, static_cast<uint32_t>(scored.size()));
        if (kk > 0) {
            std::partial_sort(scored.begin(), scored.begin() + kk, scored.end(), score_before);
        }
        for (uint32_t i = 0; i < k; ++i) {
            out_slots[qi * k + i] = i < kk ? scored[i].first : UINT32_MAX;
            out_scores[qi * k + i] = i < kk ? scored[i].second : -INFINITY;
        }
        if (!record) return;
        std::sort(v.begin(), v.end(), [](const Cand& x, const Cand& y) { return x.d != y.d ? x.d < y.d : x.slot < y.slot; });
        g_last.tau[qi] = st[qi].tau;
        g_last.rest_end[qi] = st[qi].rest_end;
        g_last.cut[qi] = cut;
        g_last.cands[qi] = std::move(v);
    }, 4);
    return 0;
}

void orc_set_record(int on) { g_record = on != 0; }

uint64_t orc_last_total_candidates(void) {
    uint64_t n = 0;
    for (auto& v : g_last.cands) n += v.size();
    return n;
}

int orc_last_candidates(uint32_t* tau, uint32_t* rest_end, uint32_t* cut, uint32_t* ncand, uint32_t* cand_slots,
                        uint32_t* cand_d, uint64_t cap) {
    uint64_t pos = 0;
    for (size_t qi = 0; qi < g_last.cands.size(); ++qi) {
        if (tau) tau[qi] = g_last.tau[qi];
        if (rest_end) rest_end[qi] = g_last.rest_end[qi];
        if (cut) cut[qi] = g_last.cut[qi];
        if (ncand) ncand[qi] = static_cast<uint32_t>(g_last.cands[qi].size());
        for (auto& e : g_last.cands[qi]) {
            if (pos >= cap) {
                if (cand_slots || cand_d) return MAIVS_ERR_ARG;
                break;
            }
            if (cand_slots) cand_slots[pos] = e.slot;
            if (cand_d) cand_d[pos] = e.d;
            ++pos;
        }
    }
    return 0;
}

}  // extern "C"

// ================================================================ the per-query path

namespace {

// keep_smallest, src/tree.rs:120-159: the `keep` smallest distances, ties at the cut-off in
// encounter order, order preserved.
void keep_smallest(std::vector<std::pair<uint32_t, uint32_t>>& v, size_t keep, uint32_t bits) {
    if (keep >= v.size()) return;
    std::vector<uint32_t> hist(bits + 1, 0);
    for (auto& e : v) hist[e.first] += 1;
    size_t cum = 0, t = 0;
    while (t < bits) {
        cum += hist[t];
        if (cum >= keep) break;
        ++t;
    }
    if (t == bits) cum += hist[t];
    size_t need_eq = keep - (cum - hist[t]);
    size_t w = 0;
    for (size_t r = 0; r < v.size(); ++r) {
        auto e = v[r];
        if (e.first < t || (e.first == t && need_eq > 0)) {
            if (e.first == t) --need_eq;
            v[w++] = e;
        }
    }
    v.resize(w);
}

// CentroidTree::search, src/tree.rs:559-628 (beams :559-570), over the arena's tree description.
std::vector<uint32_t> tree_search(const maivs_tree_desc& T, uint32_t nw, const uint64_t* qb, size_t want) {
    std::vector<uint32_t> out;
    const uint32_t L = T.n_levels, bits = nw * 64;
    if (L == 0) return out;
    std::vector<size_t> off(L + 1, 0);
    for (uint32_t l = 0; l < L; ++l) off[l + 1] = off[l] + T.level_n[l];
    std::vector<size_t> beams(L);
    size_t need = std::max<size_t>(want, 1);
    for (uint32_t i = L; i-- > 0;) {
        size_t raw = static_cast<size_t>(std::ceil(static_cast<float>(need) * T.beam_frac));
        size_t b = std::min<size_t>(std::max<size_t>(raw, T.min_beam), T.level_n[i]);
        beams[i] = b;
        need = b;
    }
    std::vector<uint32_t> frontier(T.level_n[0]);
    for (uint32_t i = 0; i < T.level_n[0]; ++i) frontier[i] = i;
    std::vector<std::pair<uint32_t, uint32_t>> scored;
    for (uint32_t li = 0; li < L; ++li) {
        scored.clear();
        for (uint32_t node : frontier)
            scored.emplace_back(orc_hamming(qb, T.level_codes + (off[li] + node) * nw, nw), node);
        size_t keep = std::min(beams[li], scored.size());
        if (keep == 0) return out;
        keep_smallest(scored, keep, bits);
        std::vector<uint32_t> expand;
        for (auto& e : scored) {
            uint32_t st = T.child_start[off[li] + e.second], ln = T.child_len[off[li] + e.second];
            for (uint32_t c = 0; c < ln; ++c) expand.push_back(st + c);  // compacted layout: contiguous
        }
        frontier.swap(expand);
    }
    scored.clear();
    for (uint32_t leaf : frontier) scored.emplace_back(orc_hamming(qb, T.leaf_codes + static_cast<size_t>(leaf) * nw, nw), leaf);
    size_t keep = std::min(want, scored.size());
    if (keep == 0) return out;
    keep_smallest(scored, keep, bits);
    for (auto& e : scored) out.push_back(T.leaf_cells[e.second]);
    return out;
}

// route_query, src/index.rs:1168-1305 (the tree, two-stage and flat branches; no graph router)
QRoute route_query(const Arena& A, const float* q, const maivs_search_params* p) {
    const maivs_arena_desc* a = A.a;
    const uint32_t d = A.d, nw = A.nw, M = A.M, cl = nw * 64;
    QRoute r;
    std::vector<float> cqs(d, 0.0f);
    float cqbase = 0.0f;
    if (a->cent_sq8) {
        for (uint32_t j = 0; j < d; ++j) {
            cqs[j] = q[j] * a->csq_step[j];
            cqbase += q[j] * a->csq_min[j];
        }
    }
    r.rot.assign(A.P, 0.0f);
    r.bits.assign(nw, 0);
    orc_rotate(q, d, a->rot_signs, A.P, r.rot.data());
    orc_pack_signs(r.rot.data(), A.P, r.bits.data(), nw);
    std::vector<std::pair<uint32_t, float>> cs;
    const maivs_tree_desc* T = a->tree;
    if (T && T->n_levels > 0) {
        size_t want_c = std::min<size_t>(static_cast<size_t>(p->nprobe) * std::max<uint32_t>(p->shortlist_mult, 2), T->n_leaf);
        for (uint32_t ci : tree_search(*T, nw, r.bits.data(), want_c))
            if (A.live[ci]) cs.emplace_back(ci, cent_score(A, ci, q, cqs.data(), cqbase));
    } else if (p->route_mode == 0 && a->cent_bits) {
        // the two-stage branch runs only with two_stage on and centroid codes present (:1241)
        std::vector<uint16_t> hs(M);
        for (uint32_t c = 0; c < M; ++c)
            hs[c] = static_cast<uint16_t>(orc_hamming(r.bits.data(), a->cent_bits + static_cast<size_t>(c) * nw, nw));
        uint32_t want_c = std::min<uint32_t>(p->nprobe * p->shortlist_mult, A.n_live);
        uint32_t cut = orc_hamming_cutoff(hs.data(), A.live.data(), M, want_c, cl);
        for (uint32_t c = 0; c < M; ++c)
            if (hs[c] <= cut && A.live[c]) cs.emplace_back(c, cent_score(A, c, q, cqs.data(), cqbase));
    } else {
        for (uint32_t c = 0; c < M; ++c)
            if (A.live[c]) cs.emplace_back(c, cent_score(A, c, q, cqs.data(), cqbase));
    }
    uint32_t cap = std::min<uint32_t>(p->nprobe, static_cast<uint32_t>(cs.size()));
    if (cap == 0) return r;
    if (cap < cs.size()) {
        std::nth_element(cs.begin(), cs.begin() + (cap - 1), cs.end(), score_before);
        cs.resize(cap);
    }
    std::sort(cs.begin(), cs.end(), score_before);
    if (p->target_confidence >= 1.0f) {
        for (auto& e : cs) r.chosen.push_back(e.first);
    } else {
        float max_s = cs[0].second;
        float z = 0.0f;
        for (auto& e : cs) z += std::exp((e.second - max_s) * p->beta);
        float cum = 0.0f;
        for (auto& e : cs) {
            r.chosen.push_back(e.first);
            cum += std::exp((e.second - max_s) * p->beta) / (z + 1e-9f);
            if (cum >= p->target_confidence) break;
        }
    }
    for (size_t i = 0; i < r.chosen.size(); ++i) r.cscore.push_back(cs[i].second);
    return r;
}

// rerank_exact, src/index.rs:1309-1378: exact scores of the candidates, top k (score desc, slot asc).
void rerank_top(const Arena& A, const float* q, const std::vector<uint32_t>& slots, uint32_t k, uint32_t* out_slots,
                float* out_scores) {
    const maivs_arena_desc* a = A.a;
    const uint32_t d = A.d;
    std::vector<std::pair<uint32_t, float>> scored;
    scored.reserve(slots.size());
    if (a->rerank_mode == MAIVS_RERANK_SQ8) {
        std::vector<float> qs(d);
        float base = 0.0f;
        for (uint32_t j = 0; j < d; ++j) {
            qs[j] = q[j] * a->sq_step[j];
            base += q[j] * a->sq_min[j];
        }
        for (uint32_t s : slots)
            scored.emplace_back(s, base + orc_dot_f32_u8(qs.data(), a->sq8_codes + static_cast<size_t>(s) * d, d));
    } else {
        for (uint32_t s : slots) scored.emplace_back(s, orc_dot_f32(q, a->vecs_f32 + static_cast<size_t>(s) * d, d));
    }
    uint32_t kk = std::min<uint32_t>(k, static_cast<uint32_t>(scored.size()));
    if (kk > 0) std::partial_sort(scored.begin(), scored.begin() + kk, scored.end(), score_before);
    for (uint32_t i = 0; i < k; ++i) {
        out_slots[i] = i < kk ? scored[i].first : UINT32_MAX;
        out_scores[i] = i < kk ? scored[i].second : -INFINITY;
    }
}

}  // namespace

extern "C" {

int orc_route_query(const maivs_arena_desc* a, const float* q, uint32_t nq, const maivs_search_params* p,
                    uint32_t nthreads, uint32_t* chosen, float* cscore, uint32_t* nchosen) {
    if (!a || !p || (!q && nq)) return MAIVS_ERR_ARG;
    Arena A(a);
    par_for(nthreads, nq, [&](size_t qi) {
        QRoute r = route_query(A, q + qi * A.d, p);
        if (nchosen) nchosen[qi] = static_cast<uint32_t>(r.chosen.size());
        for (uint32_t j = 0; j < p->nprobe; ++j) {
            bool ok = j < r.chosen.size();
            if (chosen) chosen[qi * p->nprobe + j] = ok ? r.chosen[j] : UINT32_MAX;
            if (cscore) cscore[qi * p->nprobe + j] = ok ? r.cscore[j] : NAN;
        }
    }, 4);
    return 0;
}

// search_one, src/index.rs:1381-1864, binary mode: the FastScan branch on a compacted index with
// FastScan blocks (:1689-1742), else the Hamming branch over per-slot codes (:1694-1760).
int orc_search_one(const maivs_arena_desc* a, const float* data, uint32_t nq, const maivs_search_params* p,
                   uint32_t nthreads, uint32_t* out_slots, float* out_scores) {
    if (!a || !p || (!data && nq) || p->k == 0) return MAIVS_ERR_ARG;
    const bool fs_on = a->fs_codes && a->fs_off;
    if (!fs_on && !a->slot_codes) return MAIVS_ERR_ARG;
    Arena A(a);
    const uint32_t d = A.d, nw = A.nw, M = A.M, maxk = A.maxk, k = p->k;
    const uint32_t ma = a->max_assign;
    const bool dedup = ma > 1;
    const uint32_t want0 = k * std::max<uint32_t>(p->rerank_factor, 1);
    const uint32_t target = std::max<uint32_t>(want0, 1);
    const uint32_t npairs = A.npos / 2;
    const bool filtering = p->filter && a->tags;
    const float norm = std::sqrt(2.0f * static_cast<float>(A.P) / static_cast<float>(M_PI));
    par_for(nthreads, nq, [&](size_t qi) {
        const float* q = data + qi * d;
        uint32_t* os = out_slots + qi * k;
        float* osc = out_scores + qi * k;
        for (uint32_t i = 0; i < k; ++i) {
            os[i] = UINT32_MAX;
            osc[i] = -INFINITY;
        }
        QRoute r = route_query(A, q, p);
        const size_t n = r.chosen.size();
        if (n == 0) return;
        // rank of every probed cell: a slot counts only at its first-ranked probed home (:1405-1447)
        std::vector<uint32_t> crank(M, UINT32_MAX);
        for (size_t i = 0; i < n; ++i) crank[r.chosen[i]] = static_cast<uint32_t>(i);
        auto seen = [&](uint32_t slot, uint32_t ci) {
            if (!dedup) return false;
            const uint32_t rc = crank[ci];
            for (uint32_t j = 0; j < ma; ++j) {
                uint32_t h = a->slot_cells[static_cast<size_t>(slot) * ma + j];
                if (h != UINT32_MAX && h != ci && crank[h] != UINT32_MAX && crank[h] < rc) return true;
            }
            return false;
        };
        auto keep = [&](uint32_t slot) {
            if (!filtering) return true;
            const uint32_t t = a->tags[slot];
            return t >= p->tag_lo && t <= p->tag_hi;
        };
        // reachability bounds and their suffix maxima (:1466-1489)
        std::vector<float> suffix;
        if (p->adaptive) {
            suffix.assign(n + 1, -INFINITY);
            std::vector<float> bounds(n);
            for (size_t i = 0; i < n; ++i) {
                float cs = std::fmin(std::fmax(r.cscore[i], -1.0f), 1.0f);
                float ang = std::acos(cs);
                bounds[i] = std::cos(std::fmax(ang - a->r_bound[r.chosen[i]], 0.0f));
            }
            for (size_t i = n; i-- > 0;) suffix[i] = std::fmax(bounds[i], suffix[i + 1]);
        }
        if (!fs_on) {
            // Hamming branch (:1694-1760), asymmetric cascade off: every member of the probed cells
            // in member order, keep! and the exactly-once rule, then the bucket queue on the
            // Hamming distance h in [0, dp]; after a cell, the adaptive stop on
            // score_to_cos(hamming_score(tau)) = cos(pi * tau / dp) in f32 (:1139-1158, quantize.rs:206).
            const uint32_t dp = nw * 64;
            std::vector<uint32_t> hist(dp + 1, 0);
            std::vector<std::pair<uint32_t, uint32_t>> hc;  // (h, slot)
            uint32_t tau = dp;
            size_t kept = 0;
            for (size_t ci_i = 0; ci_i < n; ++ci_i) {
                const uint32_t ci = r.chosen[ci_i];
                const uint32_t len = A.mem_len(ci);
                const uint32_t* mem = a->members + a->mem_off[ci];
                for (uint32_t i = 0; i < len; ++i) {
                    const uint32_t slot = mem[i];
                    if (!keep(slot) || seen(slot, ci)) continue;
                    const uint32_t h = orc_hamming(r.bits.data(), a->slot_codes + static_cast<size_t>(slot) * nw, nw);
                    if (h <= tau) {
                        hc.emplace_back(h, slot);
                        hist[h] += 1;
                        kept += 1;
                        while (tau > 0 && kept - hist[tau] >= target) {
                            kept -= hist[tau];
                            tau -= 1;
                        }
                    }
                }
                if (p->adaptive && kept >= target) {
                    const float dpf = static_cast<float>(dp);
                    const float sc = dpf - 2.0f * static_cast<float>(tau);  // hamming_score
                    const float hh = (dpf - sc) * 0.5f;
                    const float thr = std::cos(static_cast<float>(M_PI) * hh / dpf);
                    if (suffix[ci_i + 1] < thr - p->at_margin) break;
                }
            }
            // every survivor h <= tau, ties included, goes to the rerank (:1761-1775, 1840-1850)
            std::vector<uint32_t> slots;
            for (auto& e : hc)
                if (e.first <= tau) slots.push_back(e.second);
            rerank_top(A, q, slots, k, os, osc);
            return;
        }
        // FastScan scan with the bucket queue on d >> 6 (:1689-1742)
        std::vector<uint8_t> lut(A.npos * 16);
        float delta, bias;
        orc_fs_query(r.rot.data(), A.P, nw, lut.data(), &delta, &bias);
        std::vector<uint32_t> hist(nw * 64 + 1, 0);
        struct H {
            uint32_t hc, slot, d;
        };
        std::vector<H> hc;
        uint32_t tau = maxk >> 6;
        size_t kept = 0;
        uint16_t sums[32];
        for (size_t ci_i = 0; ci_i < n; ++ci_i) {
            const uint32_t ci = r.chosen[ci_i];
            const uint32_t len = A.mem_len(ci);
            const uint32_t* mem = a->members + a->mem_off[ci];
            for (uint32_t b = a->fs_off[ci]; b < a->fs_off[ci + 1]; ++b) {
                orc_fs_block_sums(a->fs_codes + static_cast<size_t>(b) * A.bb, lut.data(), npairs, sums);
                uint32_t base = (b - a->fs_off[ci]) * 32, nv = std::min<uint32_t>(32, len - base);
                for (uint32_t i = 0; i < nv; ++i) {
                    uint32_t dd = maxk - sums[i];
                    uint32_t h = dd >> 6;
                    if (h <= tau) {
                        uint32_t slot = mem[base + i];
                        if (!keep(slot) || seen(slot, ci)) continue;
                        hc.push_back({h, slot, dd});
                        hist[h] += 1;
                        kept += 1;
                        while (tau > 0 && kept - hist[tau] >= target) {
                            kept -= hist[tau];
                            tau -= 1;
                        }
                    }
                }
            }
            if (p->adaptive && kept >= target) {
                uint32_t top = ((tau + 1) << 6) - 1;
                uint32_t worst = maxk > top ? maxk - top : 0;
                float thr = std::fmin(std::fmax(orc_fs_estimate(delta, bias, worst) / norm, -1.0f), 1.0f);
                if (suffix[ci_i + 1] < thr - p->at_margin) break;
            }
        }
        // survivors h <= tau; the want0 smallest d (ties: ascending slot, the fixed order), :1743-1757
        std::vector<H> cands;
        for (auto& e : hc)
            if (e.hc <= tau) cands.push_back(e);
        if (want0 > 0 && cands.size() > want0) {
            std::nth_element(cands.begin(), cands.begin() + (want0 - 1), cands.end(),
                             [](const H& x, const H& y) { return x.d != y.d ? x.d < y.d : x.slot < y.slot; });
            cands.resize(want0);
        }
        std::vector<uint32_t> slots;
        for (auto& e : cands) slots.push_back(e.slot);
        rerank_top(A, q, slots, k, os, osc);
    }, 4);
    return 0;
}

}  // extern "C"

// ---- the host libm (not a restatement): what the GPU radii rely on ----

extern "C" uint64_t orc_acosf_violations(uint32_t nthreads, uint64_t* first_bad_bits) {
    // Every f32 in [-1, 1] in increasing order: -1 .. -0 (bit patterns 0xBF800000 down to
    // 0x80000000), then +0 .. 1 (0x00000000 up to 0x3F800000). Counts the x whose successor y has
    // acosf(y) > acosf(x), i.e. where acosf fails to be non-increasing.
    const uint64_t n_neg = 0xBF800000ull - 0x80000000ull + 1, N = 2 * n_neg;
    auto at = [&](uint64_t k) -> float {
        const uint32_t b = static_cast<uint32_t>(k < n_neg ? 0xBF800000ull - k : k - n_neg);
        float f;
        std::memcpy(&f, &b, 4);
        return f;
    };
    const size_t chunks = 4096;
    std::vector<uint64_t> bad(chunks, 0), first(chunks, UINT64_MAX);
    par_for(nthreads, chunks, [&](size_t ch) {
        const uint64_t lo = 1 + (N - 1) * ch / chunks, hi = 1 + (N - 1) * (ch + 1) / chunks;
        float prev = std::acos(at(lo - 1));
        for (uint64_t k = lo; k < hi; ++k) {
            const float cur = std::acos(at(k));
            if (cur > prev) {
                if (!bad[ch]) first[ch] = k - 1;
                ++bad[ch];
            }
            prev = cur;
        }
    });
    uint64_t total = 0, f = UINT64_MAX;
    for (size_t ch = 0; ch < chunks; ++ch) {
        total += bad[ch];
        f = std::min(f, first[ch]);
    }
    if (first_bad_bits) {
        float x = f == UINT64_MAX ? 0.0f : at(f);
        uint32_t b;
        std::memcpy(&b, &x, 4);
        *first_bad_bits = f == UINT64_MAX ? UINT64_MAX : b;
    }
    return total;
}
