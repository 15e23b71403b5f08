// FlatCellIndex: the host side of the drop-in. Builds the partitioned index exactly as the
// reference's CPU build does (train_centroids -> add_batch -> compact), and runs
// search_batch through libmaivs_gpu.so's C ABI on the MI355X.
//
// Reference: the pyo3 class FlatCellIndex, src/index.rs:431-566 (state) and :2670-3603
// (methods). Only the state the batched cell-major search, its build and persistence need is
// kept; HNSW routing and split/merge are not implemented by this library.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <optional>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../../include/maivs_gpu.h"
#include "tree.h"

namespace maivs {

struct ValueError : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct Unsupported : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct IoError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

enum class ScanMode { F32, I8, Binary };

// Allocator whose value-initialisation leaves elements default-initialised (for these row arrays:
// unset), so a row array can grow by millions of rows and then be filled by several threads,
// instead of first being zeroed by one. resize(n, value) and assign still write their value.
template <class T>
struct NoInitAlloc : std::allocator<T> {
    template <class U>
    struct rebind {
        using other = NoInitAlloc<U>;
    };
    NoInitAlloc() = default;
    template <class U>
    NoInitAlloc(const NoInitAlloc<U>&) noexcept {}
    template <class U>
    void construct(U* p) noexcept {
        ::new (static_cast<void*>(p)) U;
    }
    template <class U, class... Args>
    void construct(U* p, Args&&... args) {
        ::new (static_cast<void*>(p)) U(std::forward<Args>(args)...);
    }
};
template <class T>
using RowVec = std::vector<T, NoInitAlloc<T>>;

// External id -> slot, the reference's id_to_slot HashMap (src/index.rs:431-566): open addressing
// with linear probing over a power-of-two table kept at most half full, erased entries marked so
// probes pass over them. One flat allocation instead of a node per id, so rebuilding it for
// millions of ids (add_batch, compact) costs a fraction of a node-based map.
class IdMap {
public:
    size_t size() const { return n_; }
    void clear() {
        keys_.clear();
        vals_.clear();
        state_.clear();
        n_ = used_ = 0;
    }
    void reserve(size_t n) {
        if (2 * n >= state_.size()) rehash(n);
    }
    // the slot of id k, or nullptr
    const uint32_t* find(uint64_t k) const {
        if (state_.empty()) return nullptr;
        for (size_t i = hash(k) & mask(), step = 0; step <= mask(); i = (i + 1) & mask(), ++step) {
            if (state_[i] == kEmpty) return nullptr;
            if (state_[i] == kFull && keys_[i] == k) return &vals_[i];
        }
        return nullptr;
    }
    // inserts k or overwrites its slot
    void set(uint64_t k, uint32_t v) {
        if (2 * (used_ + 1) > state_.size()) rehash(n_ + 1);
        size_t tomb = SIZE_MAX;
        for (size_t i = hash(k) & mask();; i = (i + 1) & mask()) {
            if (state_[i] == kFull && keys_[i] == k) {
                vals_[i] = v;
                return;
            }
            if (state_[i] == kTomb && tomb == SIZE_MAX) tomb = i;
            if (state_[i] == kEmpty) {
                if (tomb != SIZE_MAX) {
                    i = tomb;
                } else {
                    ++used_;
                }
                keys_[i] = k;
                vals_[i] = v;
                state_[i] = kFull;
                ++n_;
                return;
            }
        }
    }
    bool erase(uint64_t k) {
        const uint32_t* v = find(k);
        if (!v) return false;
        const size_t i = static_cast<size_t>(v - vals_.data());
        state_[i] = kTomb;
        --n_;
        return true;
    }
    template <class F>
    void for_each(F f) const {
        for (size_t i = 0; i < state_.size(); ++i)
            if (state_[i] == kFull) f(keys_[i], vals_[i]);
    }

private:
    static constexpr uint8_t kEmpty = 0, kFull = 1, kTomb = 2;
    static size_t hash(uint64_t k) {  // splitmix64's finaliser
        k ^= k >> 30;
        k *= 0xBF58476D1CE4E5B9ull;
        k ^= k >> 27;
        k *= 0x94D049BB133111EBull;
        k ^= k >> 31;
        return static_cast<size_t>(k);
    }
    size_t mask() const { return state_.size() - 1; }
    void rehash(size_t n) {
        size_t cap = 16;
        while (cap < 2 * n + 2) cap <<= 1;
        std::vector<uint64_t> keys(cap);
        std::vector<uint32_t> vals(cap);
        std::vector<uint8_t> state(cap, kEmpty);
        const size_t m = cap - 1;
        for (size_t j = 0; j < state_.size(); ++j) {
            if (state_[j] != kFull) continue;
            size_t i = hash(keys_[j]) & m;
            while (state[i] == kFull) i = (i + 1) & m;
            keys[i] = keys_[j];
            vals[i] = vals_[j];
            state[i] = kFull;
        }
        keys_.swap(keys);
        vals_.swap(vals);
        state_.swap(state);
        used_ = n_;
    }
    std::vector<uint64_t> keys_;
    std::vector<uint32_t> vals_;
    std::vector<uint8_t> state_;
    size_t n_ = 0, used_ = 0;  // live entries; live + erased (slots no longer empty)
};

struct Cell {
    std::vector<uint32_t> members;
    std::vector<float> sum, centroid;
    float r_bound = 0.0f, r_max = 0.0f;
};

class GpuSession;  // owns a maivs_gpu_ctx (index.cpp)

void fill_tree_desc(const TreeFlat& tf, maivs_tree_desc& td);

class FlatCellIndex {
public:
    FlatCellIndex(size_t dim, const std::string& scan_mode, size_t rerank_factor, uint64_t seed,
                  size_t code_bits);
    ~FlatCellIndex();

    // ---- configuration (src/index.rs:2806-2984, 3520-3558) ----
    void train_centroids(const float* data, size_t n_all, size_t n_cells, size_t sample, uint64_t seed);
    void set_centroids(const float* cents, size_t n);
    void set_i8_rerank(bool on);
    void set_tree_route(bool on, size_t min_cells, size_t fanout, float beam_frac);
    void set_graph_route(bool on, size_t min_cells);
    void set_centroid_sq8(bool on);
    void set_two_stage(bool on, size_t mult);
    void set_adaptive(bool on, float margin);
    void set_per_dim_sq(bool on);
    void set_f16_rerank(bool on);
    void set_quant_scale(float s) { quant_scale_ = s; }
    void set_rerank_factor(size_t rf) { rerank_factor_ = std::max<size_t>(rf, 1); }
    void set_asym_cascade(size_t f) { asym_cascade_ = f; }
    void set_fastscan(bool on);
    void set_replication(size_t max_assign, float spill_margin);
    void set_orthogonal_polysemy(size_t homes, float lam);
    void set_parallel_scan(bool on) { par_scan_ = on; }
    void set_tags(const std::vector<uint64_t>& ids, const std::vector<uint32_t>& tags);
    void set_filter(std::optional<uint32_t> lo, std::optional<uint32_t> hi);
    void rebuild_tree() { rebuild_centroid_tree(); }
    // Not in the reference: run the index build's heavy steps on the GPU (bit-identical results).
    void set_gpu_build(bool on) { gpu_build_ = on; }
    bool store_mirrors() const { return store_ok_; }
    bool gpu_build() const { return gpu_build_; }
    // One batch of k-means jobs through the CPU or the GPU runner (test hook).
    void run_kmeans(const float* x, size_t n_rows, size_t dim, const uint32_t* rows, const std::vector<KMeansJob>& jobs,
                    bool gpu, std::vector<uint32_t>& assign, std::vector<float>& cents) {
        if (gpu)
            gpu_kmeans_runner()(x, n_rows, dim, rows, jobs, assign, cents);
        else
            run_kmeans_cpu(x, n_rows, dim, rows, jobs, assign, cents);
    }

    // ---- mutation ----
    void add_batch(const std::vector<uint64_t>& ids, const float* data, size_t n);
    bool remove(uint64_t id);
    void compact();

    // ---- search ----
    // Batched cell-major search on the GPU. Fills ids/scores (nq*k), padded u64::MAX / -inf.
    void search_batch(const float* q, size_t nq, size_t k, size_t nprobe, float tc, float beta,
                      bool cell_major, std::vector<uint64_t>& ids, std::vector<float>& scores,
                      maivs_gpu_stats* stats = nullptr);
    // One query through the per-query path (src/index.rs:3283-3305): up to k results, best first.
    void search(const float* q, size_t k, size_t nprobe, float tc, float beta, std::vector<uint64_t>& ids,
                std::vector<float>& scores);
    // Why the batched cell-major path cannot run right now (empty string when it can).
    std::string cellmajor_blocker(bool cell_major) const;
    // Why the per-query path cannot run right now (empty string when it can).
    std::string perquery_blocker() const;
    // Whether search_batch takes the batched cell-major path for nq queries (the reference's cm_ok).
    bool takes_cellmajor(size_t nq, bool cell_major) const;
    // Not in the reference: filtered searches take the batched path too (the filter is applied in
    // its scans); by default they take the per-query path, as the reference's do.
    void set_batched_filter(bool on) { batched_filter_ = on; }

    // ---- persistence (src/persist.rs, format "MAIVS2\0\1" + an extension trailer) ----
    void save(const std::string& path) const;
    // Replaces this index's whole state with the file's.
    void load_file(const std::string& path);

    // ---- introspection ----
    std::map<std::string, double> stats() const;
    size_t len() const { return n_live_; }
    size_t dim() const { return dim_; }
    std::pair<size_t, bool> recommend() const;
    // The compacted arena as a C descriptor (valid until the next mutation).
    const maivs_arena_desc* arena_desc();
    maivs_search_params search_params(size_t k, size_t nprobe, float tc, float beta) const;
    const std::vector<uint64_t>& ext_ids() const { return ext_ids_; }
    const RowVec<uint64_t>& bits() const { return bits_; }
    const std::vector<float>& rot_signs() const { return rot_signs_; }
    uint64_t generation() const { return generation_; }
    // The centroid tree's flat arrays (false when there is no tree).
    bool tree_flat(TreeFlat& f) const {
        if (!tree_) return false;
        tree_->export_flat(64, f);
        return true;
    }

private:
    void refresh_derived();
    void recompute_radii();
    void rebuild_centroid_codes();
    void rebuild_centroid_sq8();
    void maybe_rebuild_centroid_tree();
    void rebuild_centroid_tree();
    size_t live_cell_count() const;
    std::vector<uint32_t> assign_cells(const float* v) const;
    std::vector<uint32_t> assign_cells_routed(const float* v, std::vector<float>& rot, std::vector<uint64_t>& bits,
                                              TreeScratch& ts, std::vector<uint32_t>& out) const;
    std::vector<uint32_t> pick_orthogonal(std::vector<std::pair<uint32_t, float>>& scored) const;
    void encode_slot(const float* v, uint64_t* bits_out, int8_t* i8_out) const;
    void compact_arena();
    void recompute_centroid(Cell& c);
    void touch() { ++generation_; compacted_ = false; }
    KMeansRunner gpu_kmeans_runner();
    void ensure_uploaded();
    void place_on_gpu(const float* data, size_t n, bool store_i8, std::vector<std::vector<uint32_t>>& asg,
                      std::vector<uint64_t>& bits, std::vector<int8_t>& i8, const uint32_t* slots, float* sums);
    bool gpu_radii();
    void refresh_store_token();

    size_t dim_, rerank_factor_, dim_pad_, n_words_;
    ScanMode scan_mode_;
    uint64_t seed_;
    std::vector<float> rot_signs_;

    RowVec<uint64_t> bits_;
    RowVec<int8_t> scan_i8_;
    RowVec<float> vecs_f32_;
    std::vector<uint64_t> ext_ids_;
    std::vector<uint32_t> slot_cell_;
    std::vector<uint32_t> free_slots_;
    IdMap id_to_slot_;

    std::vector<Cell> cells_;
    std::vector<uint64_t> cent_bits_;
    std::vector<uint8_t> cent_sq8_;
    std::vector<float> csq_min_, csq_step_;
    bool centroid_sq8_ = true;
    std::unique_ptr<CentroidTree> tree_;
    bool tree_route_ = true;
    size_t tree_min_cells_ = CentroidTree::kMinCellsForTree;
    size_t tree_fanout_ = CentroidTree::kDefaultFanout;
    float tree_beam_frac_ = CentroidTree::kDefaultBeamFrac;
    size_t tree_cells_ = 0;
    bool par_scan_ = false;
    bool graph_route_ = true;
    size_t graph_min_cells_ = 65536;
    // the reference's cent_graph is Some: rebuilt by refresh_derived and set_graph_route when graph
    // routing is on and enough cells are live, never by a load (src/index.rs:625-636)
    bool graph_built_ = false;
    bool two_stage_ = false;
    size_t shortlist_mult_ = 4;
    float quant_scale_ = 0.0f;
    size_t n_live_ = 0;

    size_t max_assign_ = 1;
    float spill_margin_ = 0.0f, spill_lambda_ = 0.0f;
    bool compacted_ = false;
    size_t asym_cascade_ = 0;
    bool fastscan_ = false;
    std::vector<uint8_t> fs_codes_;
    std::vector<uint32_t> fs_off_;
    std::vector<uint32_t> prim_len_, rep_off_;
    std::vector<uint32_t> slot_cells_;
    std::vector<uint32_t> tags_;
    std::optional<std::pair<uint32_t, uint32_t>> tag_filter_;
    bool i8_rerank_ = false, per_dim_sq_ = false, f16_rerank_ = false, keep_f32_ = true;
    std::vector<float> sq_min_, sq_step_;
    bool adaptive_ = false;
    float at_margin_ = 0.02f;

    // flattened member CSR of the compacted arena (built by compact_arena)
    std::vector<uint32_t> mem_off_, members_flat_;
    std::vector<float> cents_flat_, r_bound_flat_;
    maivs_arena_desc desc_{};
    TreeFlat tree_flat_;
    maivs_tree_desc tree_desc_{};
    uint64_t generation_ = 0;
    bool gpu_build_ = false;
    // The GPU session's row store mirrors bits_, scan_i8_ and vecs_f32_ slot for slot: set by a GPU
    // build's first add_batch, kept by later GPU add_batch / remove / compact, cleared by anything
    // that writes those arrays otherwise (a CPU add_batch, a load, a change of their layout).
    bool store_ok_ = false;
    uint64_t store_token_ = 0;
    bool batched_filter_ = false;
    std::unique_ptr<GpuSession> gpu_;
    std::mutex session_mu_;  // guards the creation of gpu_ (searches share the index)
    GpuSession* session();
};

}  // namespace maivs
