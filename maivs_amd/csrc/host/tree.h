// Centroid training and the dynamic-depth centroid tree used to place vectors at ingest
// (restated from src/tree.rs). Build-side support only: the batched search routes with the
// flat two-stage router, not the tree (src/index.rs:2105-2107).
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <vector>

namespace maivs {

// Spherical Lloyd k-means over unit vectors, src/tree.rs:179-248. Returns (assign, centroids).
void kmeans_spherical(const float* x, size_t n, size_t dim, size_t k, size_t iters, uint64_t seed,
                      std::vector<uint32_t>& assign, std::vector<float>& cents, bool parallel);

// A batch of independent spherical k-means problems over rows of one matrix x (n_rows x dim).
// Job j clusters the points rows[first .. first + n) (row ids into x; no row list = 0, 1, 2, ...)
// into k clusters with `iters` Lloyd iterations and reseeding state seed | 1. The jobs tile the
// row list in order. A runner fills assign (sum n, cluster within the job) and cents (sum k x dim,
// the jobs' centroids back to back). The default runs kmeans_spherical per job on the host; the
// index's GPU build passes one that calls maivs_gpu_kmeans, which gives bit-identical results.
struct KMeansJob {
    size_t first, n, k, iters;
    uint64_t seed;
};
using KMeansRunner = std::function<void(const float* x, size_t n_rows, size_t dim, const uint32_t* rows,
                                        const std::vector<KMeansJob>& jobs, std::vector<uint32_t>& assign,
                                        std::vector<float>& cents)>;
void run_kmeans_cpu(const float* x, size_t n_rows, size_t dim, const uint32_t* rows, const std::vector<KMeansJob>& jobs,
                    std::vector<uint32_t>& assign, std::vector<float>& cents);

// Two-level balanced k-means, src/tree.rs:257-348. Returns k x dim centroids.
std::vector<float> hierarchical_kmeans(const float* x, size_t n, size_t dim, size_t k, uint64_t seed,
                                       const KMeansRunner* runner = nullptr);

struct TreeLevel {
    size_t n = 0;
    std::vector<float> cents;
    std::vector<uint64_t> codes;
    std::vector<uint32_t> child_start, child_len, child_idx;
};

// The tree in its compacted layout as flat arrays (the GPU placement's input).
struct TreeFlat {
    std::vector<uint32_t> level_n, beams, child_start, child_len, leaf_cells;
    std::vector<uint64_t> level_codes, leaf_codes;
    float beam_frac = 0.5f;
    uint32_t min_beam = 32;
};

struct TreeScratch {
    std::vector<uint32_t> frontier, expand, hist;
    std::vector<std::pair<uint32_t, uint32_t>> scored;  // (hamming, node)
};

class CentroidTree {
public:
    static constexpr size_t kDefaultFanout = 64;   // src/tree.rs:37
    static constexpr size_t kTopMax = 256;         // src/tree.rs:41
    static constexpr size_t kMinBeam = 32;         // src/tree.rs:45
    static constexpr float kDefaultBeamFrac = 0.5f;  // src/tree.rs:66
    static constexpr size_t kMinCellsForTree = 2048;  // src/tree.rs:70

    // Build over live cells (cell_cents row i belongs to cell_ids[i]); false if degenerate.
    bool build(const float* cell_cents, const std::vector<uint32_t>& cell_ids, size_t dim,
               const float* rot_signs, size_t dim_pad, size_t n_words, size_t fanout, float beam_frac,
               const KMeansRunner* runner = nullptr);
    // Up to `want` leaf cell ids, best first by Hamming (ties in encounter order).
    void search(const uint64_t* q_bits, size_t want, TreeScratch& s, std::vector<uint32_t>& out) const;
    size_t depth() const { return levels_.size(); }
    size_t n_leaf() const { return n_leaf_; }
    size_t top_width() const { return levels_.empty() ? 0 : levels_.front().n; }
    size_t bytes() const;
    // Flat arrays of every level (coarsest first) and the leaves, with the beams of search(want).
    void export_flat(size_t want, TreeFlat& f) const;

private:
    std::vector<size_t> beams(size_t want) const;
    void compact_layout();

    size_t dim_ = 0, n_words_ = 0, fanout_ = 0;
    float beam_frac_ = kDefaultBeamFrac;
    std::vector<TreeLevel> levels_;  // coarsest first
    std::vector<uint64_t> leaf_codes_;
    std::vector<uint32_t> leaf_ids_;
    size_t n_leaf_ = 0;
};

}  // namespace maivs
