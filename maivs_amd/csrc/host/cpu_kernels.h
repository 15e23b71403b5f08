// Host-side numeric kernels of the index build: rotation, sign codes, FastScan layout and the
// AVX2 dot products, with the reference's exact operation order so the arena the GPU searches
// is the arena the reference would build.
//
// Everything here is compiled with -ffp-contract=off: an FMA appears only where the reference
// uses _mm256_fmadd_ps.
#pragma once

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <thread>
#include <vector>

namespace maivs {

constexpr int kRounds = 2;       // (H*D) rounds, src/quantize.rs:34
constexpr int kFsBlock = 32;     // vectors per FastScan block, src/quantize.rs:222

// Next power of two >= n, at least 64 (src/quantize.rs:38-40).
inline size_t pad_dim(size_t n) {
    size_t p = 1;
    while (p < n) p <<= 1;
    return std::max<size_t>(p, 64);
}

// Whole 64-bit words of a code of `code_bits` bits (0 = full length), src/quantize.rs:50-53.
inline size_t code_words(size_t code_bits, size_t dim_pad) {
    size_t b = code_bits == 0 ? dim_pad : std::min(code_bits, dim_pad);
    return std::max<size_t>(b / 64, 1);
}

inline size_t fs_block_bytes(size_t nw) { return nw * 64 * kFsBlock / 8; }

// splitmix64 +-1 signs, ROUNDS x dim_pad, src/quantize.rs:132-148.
inline std::vector<float> make_signs(size_t dim_pad, uint64_t seed) {
    std::vector<float> out(kRounds * dim_pad);
    uint64_t state = seed;
    for (size_t i = 0; i < out.size(); ++i) {
        state += 0x9E3779B97F4A7C15ull;
        uint64_t z = state;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        out[i] = (z & 1) == 0 ? 1.0f : -1.0f;
    }
    return out;
}

// Normalised fast Walsh-Hadamard transform, butterfly levels h = 1, 2, 4, ..., n/2 in order,
// then a multiply by 1/sqrt(n) computed in f32 (src/quantize.rs:71-126). The order of the
// butterflies inside a level does not change any result; the order of the levels does.
inline void fht_inplace(float* a, size_t n) {
    for (size_t h = 1; h < n; h <<= 1) {
        for (size_t i = 0; i < n; i += h << 1) {
            for (size_t j = i; j < i + h; ++j) {
                float x = a[j], y = a[j + h];
                a[j] = x + y;
                a[j + h] = x - y;
            }
        }
    }
    const float s = 1.0f / std::sqrt(static_cast<float>(n));
    for (size_t i = 0; i < n; ++i) a[i] *= s;
}

// Copy v into out[0..dim), zero the rest of dim_pad, then ROUNDS x (sign flip, FWHT);
// src/quantize.rs:152-163.
inline void rotate(const float* v, size_t dim, const float* signs, size_t dim_pad, float* out) {
    for (size_t i = 0; i < dim; ++i) out[i] = v[i];
    for (size_t i = dim; i < dim_pad; ++i) out[i] = 0.0f;
    for (int r = 0; r < kRounds; ++r) {
        const float* s = signs + r * dim_pad;
        for (size_t i = 0; i < dim_pad; ++i) out[i] *= s[i];
        fht_inplace(out, dim_pad);
    }
}

// Bit i set iff rotated[i] < 0, over the first nw*64 coordinates; src/quantize.rs:57-67.
inline void pack_signs_trunc(const float* rot, size_t n, uint64_t* out, size_t nw) {
    for (size_t w = 0; w < nw; ++w) out[w] = 0;
    size_t bits = std::min(nw * 64, n);
    for (size_t i = 0; i < bits; ++i)
        if (rot[i] < 0.0f) out[i >> 6] |= 1ull << (i & 63);
}

inline uint32_t hamming(const uint64_t* a, const uint64_t* b, size_t nw) {
    uint32_t s = 0;
    for (size_t i = 0; i < nw; ++i) s += static_cast<uint32_t>(__builtin_popcountll(a[i] ^ b[i]));
    return s;
}

inline uint8_t nib(const uint64_t* code, size_t j) {
    return static_cast<uint8_t>((code[j >> 4] >> ((j & 15) * 4)) & 0xF);
}

// Interleave up to 32 codes into one FastScan block: byte [p*32 + half*16 + i] holds
// nibble 2p+half of lane i (low) and of lane i+16 (high); src/quantize.rs:238-250.
inline void fs_pack_block(const uint64_t* const* codes, size_t ncodes, size_t nw, uint8_t* out) {
    size_t npos = nw * 16;
    for (size_t p = 0; p < npos / 2; ++p)
        for (size_t half = 0; half < 2; ++half) {
            size_t j = 2 * p + half;
            for (size_t i = 0; i < 16; ++i) {
                uint8_t lo = i < ncodes ? nib(codes[i], j) : 0;
                uint8_t hi = i + 16 < ncodes ? nib(codes[i + 16], j) : 0;
                out[p * 32 + half * 16 + i] = static_cast<uint8_t>(lo | (hi << 4));
            }
        }
}

// Horizontal sum with _mm256 lane order ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)),
// src/index.rs:58-65.
inline float hsum_ps(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 0x55));
    return _mm_cvtss_f32(s);
}

// 8-lane FMA dot + hsum + sequential tail, src/index.rs:136-152.
__attribute__((target("avx2,fma"))) inline float dot_f32(const float* a, const float* b, size_t n) {
    __m256 acc = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 8 <= n; i += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc);
    float s = hsum_ps(acc);
    for (; i < n; ++i) s += a[i] * b[i];
    return s;
}

// f32 x u8 dot, src/index.rs:278-294.
__attribute__((target("avx2,fma"))) inline float dot_f32_u8(const float* qs, const uint8_t* v, size_t n) {
    __m256 acc = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        __m128i b = _mm_loadl_epi64(reinterpret_cast<const __m128i*>(v + i));
        __m256 vf = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(b));
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(qs + i), vf, acc);
    }
    float s = hsum_ps(acc);
    for (; i < n; ++i) s += qs[i] * static_cast<float>(v[i]);
    return s;
}

// f32 x i8 dot, src/index.rs:161-177.
__attribute__((target("avx2,fma"))) inline float dot_f32_i8(const float* q, const int8_t* v, size_t n) {
    __m256 acc = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        __m128i b = _mm_loadl_epi64(reinterpret_cast<const __m128i*>(v + i));
        __m256 vf = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(b));
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(q + i), vf, acc);
    }
    float s = hsum_ps(acc);
    for (; i < n; ++i) s += q[i] * static_cast<float>(v[i]);
    return s;
}

// Rust's f32 `iter().sum()` folds from -0.0 (rustc >= 1.81), so an all-(-0.0) sum stays -0.0.
inline float rust_sum(const float* v, size_t n) {
    float s = -0.0f;
    for (size_t i = 0; i < n; ++i) s += v[i];
    return s;
}

// ---- threading ----

inline unsigned num_threads() {
    for (const char* k : {"MAIVS_NUM_THREADS", "RAYON_NUM_THREADS", "OMP_NUM_THREADS"}) {
        if (const char* e = std::getenv(k)) {
            int v = std::atoi(e);
            if (v > 0) return static_cast<unsigned>(v);
        }
    }
    unsigned h = std::thread::hardware_concurrency();
    return h ? h : 1;
}

// Run f(i) for i in [0, n) on up to num_threads() threads, dynamic chunks of `grain`.
template <class F>
void parallel_for(size_t n, F&& f, size_t grain = 1) {
    if (n == 0) return;
    unsigned nt = std::min<size_t>(num_threads(), (n + grain - 1) / grain);
    if (nt <= 1) {
        for (size_t i = 0; i < n; ++i) f(i);
        return;
    }
    std::atomic<size_t> next{0};
    auto work = [&]() {
        for (;;) {
            size_t s = next.fetch_add(grain);
            if (s >= n) break;
            size_t e = std::min(n, s + grain);
            for (size_t i = s; i < e; ++i) f(i);
        }
    };
    std::vector<std::thread> th;
    th.reserve(nt - 1);
    for (unsigned t = 1; t < nt; ++t) th.emplace_back(work);
    work();
    for (auto& t : th) t.join();
}

}  // namespace maivs
