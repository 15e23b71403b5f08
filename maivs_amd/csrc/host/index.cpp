// FlatCellIndex host implementation (see index.h). Each method cites the reference method it
// restates; the arithmetic keeps the reference's operation order (compiled -ffp-contract=off).
#include "index.h"

#include <dlfcn.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <numeric>

#include "cpu_kernels.h"

namespace maivs {

// ---------------------------------------------------------------- GPU session (C ABI client)

namespace {

struct GpuApi {
    int (*create)(int, maivs_gpu_ctx**) = nullptr;
    void (*destroy)(maivs_gpu_ctx*) = nullptr;
    const char* (*last_error)(const maivs_gpu_ctx*) = nullptr;
    int (*upload)(maivs_gpu_ctx*, const maivs_arena_desc*) = nullptr;
    int (*search)(maivs_gpu_ctx*, const float*, uint32_t, const maivs_search_params*, uint32_t*, float*,
                  maivs_gpu_stats*) = nullptr;
    int (*search_pq)(maivs_gpu_ctx*, const float*, uint32_t, const maivs_search_params*, uint32_t*, float*,
                     maivs_gpu_stats*) = nullptr;
    int (*kmeans)(maivs_gpu_ctx*, const float*, uint64_t, uint32_t, const uint32_t*, const maivs_kmeans_job*,
                  uint32_t, uint32_t*, float*) = nullptr;
    int (*place)(maivs_gpu_ctx*, const maivs_place_desc*, const float*, uint32_t, uint32_t*, uint64_t*,
                 int8_t*) = nullptr;
    int (*store_reset)(maivs_gpu_ctx*, uint32_t, uint32_t, uint32_t) = nullptr;
    int (*store_info)(maivs_gpu_ctx*, uint64_t*, uint32_t*) = nullptr;
    int (*store_radii)(maivs_gpu_ctx*, const maivs_radii_desc*, float*, float*) = nullptr;
    int (*store_compact)(maivs_gpu_ctx*, const uint32_t*, uint32_t, uint32_t, const uint32_t*, const uint32_t*,
                         const uint32_t*, uint8_t*, float*, int8_t*, uint64_t*) = nullptr;
    std::string error;
};

std::string module_dir() {
    Dl_info info{};
    if (dladdr(reinterpret_cast<void*>(&module_dir), &info) && info.dli_fname) {
        std::string p = info.dli_fname;
        size_t s = p.rfind('/');
        if (s != std::string::npos) return p.substr(0, s);
    }
    return ".";
}

// libmaivs_gpu.so sits next to this module; it is loaded on the first search, so building and
// inspecting an index needs no GPU runtime. A missing or broken library is an error, never a
// silent CPU path.
const GpuApi& gpu_api() {
    static GpuApi api;
    static std::once_flag once;
    std::call_once(once, [] {
        const char* env = std::getenv("MAIVS_GPU_LIB");
        std::string path = env ? std::string(env) : module_dir() + "/libmaivs_gpu.so";
        void* h = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
        if (!h) {
            api.error = std::string("cannot load ") + path + ": " + dlerror();
            return;
        }
        auto sym = [&](const char* name) {
            void* p = dlsym(h, name);
            if (!p) api.error = std::string("missing symbol ") + name + " in " + path;
            return p;
        };
        api.create = reinterpret_cast<decltype(api.create)>(sym("maivs_gpu_create"));
        api.destroy = reinterpret_cast<decltype(api.destroy)>(sym("maivs_gpu_destroy"));
        api.last_error = reinterpret_cast<decltype(api.last_error)>(sym("maivs_gpu_last_error"));
        api.upload = reinterpret_cast<decltype(api.upload)>(sym("maivs_gpu_upload_arena"));
        api.search = reinterpret_cast<decltype(api.search)>(sym("maivs_gpu_search_batch"));
        api.search_pq = reinterpret_cast<decltype(api.search_pq)>(sym("maivs_gpu_search_queries"));
        api.kmeans = reinterpret_cast<decltype(api.kmeans)>(sym("maivs_gpu_kmeans"));
        api.place = reinterpret_cast<decltype(api.place)>(sym("maivs_gpu_place"));
        api.store_reset = reinterpret_cast<decltype(api.store_reset)>(sym("maivs_gpu_store_reset"));
        api.store_info = reinterpret_cast<decltype(api.store_info)>(sym("maivs_gpu_store_info"));
        api.store_radii = reinterpret_cast<decltype(api.store_radii)>(sym("maivs_gpu_store_radii"));
        api.store_compact = reinterpret_cast<decltype(api.store_compact)>(sym("maivs_gpu_store_compact"));
    });
    return api;
}

}  // namespace

class GpuSession {
public:
    GpuSession() {
        const GpuApi& a = gpu_api();
        if (!a.error.empty()) throw std::runtime_error("MI355X search library unavailable: " + a.error);
        int dev = 0;
        if (const char* e = std::getenv("MAIVS_DEVICE")) dev = std::atoi(e);
        int rc = a.create(dev, &ctx_);
        if (rc != 0 || !ctx_) throw std::runtime_error("maivs_gpu_create failed (status " + std::to_string(rc) + ")");
    }
    ~GpuSession() {
        if (ctx_) gpu_api().destroy(ctx_);
    }
    void check(int rc, const char* what) {
        if (rc == 0) return;
        std::string msg = std::string(what) + ": " + gpu_api().last_error(ctx_);
        if (rc == MAIVS_ERR_UNSUPPORTED) throw Unsupported(msg);
        if (rc == MAIVS_ERR_ARG) throw ValueError(msg);
        throw std::runtime_error(msg);
    }
    maivs_gpu_ctx* ctx_ = nullptr;
    uint64_t uploaded_gen = ~0ull;
    std::mutex mu;
};

// The GPU session, created once: concurrent searches (shared borrows) may both get here first.
GpuSession* FlatCellIndex::session() {
    std::lock_guard<std::mutex> lk(session_mu_);
    if (!gpu_) gpu_ = std::make_unique<GpuSession>();
    return gpu_.get();
}

// The k-means runner of the GPU build: every batch of jobs goes to maivs_gpu_kmeans, whose
// results are bit-identical to run_kmeans_cpu's.
KMeansRunner FlatCellIndex::gpu_kmeans_runner() {
    GpuSession* g = session();
    return [g](const float* x, size_t n_rows, size_t dim, const uint32_t* rows, const std::vector<KMeansJob>& jobs,
               std::vector<uint32_t>& assign, std::vector<float>& cents) {
        std::vector<maivs_kmeans_job> js;
        size_t np = 0, sk = 0;
        for (const auto& J : jobs) {
            size_t k = std::min(std::max<size_t>(J.k, 1), J.n);
            js.push_back(maivs_kmeans_job{static_cast<uint32_t>(J.first), static_cast<uint32_t>(J.n),
                                          static_cast<uint32_t>(k), static_cast<uint32_t>(J.iters), J.seed});
            np += J.n;
            sk += k;
        }
        assign.assign(np, 0);
        cents.assign(sk * dim, 0.0f);
        g->check(gpu_api().kmeans(g->ctx_, x, n_rows, static_cast<uint32_t>(dim), rows, js.data(),
                                  static_cast<uint32_t>(js.size()), assign.data(), cents.data()),
                 "maivs_gpu_kmeans");
    };
}

// ---------------------------------------------------------------- construction, config

FlatCellIndex::FlatCellIndex(size_t dim, const std::string& mode, size_t rerank_factor, uint64_t seed,
                             size_t code_bits)
    : dim_(dim), rerank_factor_(std::max<size_t>(rerank_factor, 1)), seed_(seed) {
    // src/index.rs:2676-2754
    if (mode == "f32")
        scan_mode_ = ScanMode::F32;
    else if (mode == "i8")
        scan_mode_ = ScanMode::I8;
    else if (mode == "binary")
        scan_mode_ = ScanMode::Binary;
    else
        throw ValueError("scan_mode must be 'f32', 'i8' or 'binary', got '" + mode + "'");
    dim_pad_ = pad_dim(dim);
    n_words_ = code_words(code_bits, dim_pad_);
    rot_signs_ = make_signs(dim_pad_, seed);
}

FlatCellIndex::~FlatCellIndex() = default;

void FlatCellIndex::set_i8_rerank(bool on) {  // src/index.rs:2827-2832
    i8_rerank_ = on;
    keep_f32_ = !on;
    store_ok_ = false;  // the rows' layout changes
}

void FlatCellIndex::set_tree_route(bool on, size_t min_cells, size_t fanout, float beam_frac) {  // :2840-2853
    if (beam_frac > 0.0f) tree_beam_frac_ = beam_frac;
    tree_route_ = on;
    if (min_cells > 0) tree_min_cells_ = min_cells;
    if (fanout > 1) tree_fanout_ = fanout;
    rebuild_centroid_tree();
}

void FlatCellIndex::set_graph_route(bool on, size_t min_cells) {  // :2860-2866
    // The centroid HNSW itself is not implemented by this library; only whether the reference would hold
    // one (rebuild_centroid_graph, :625-636) is tracked, so that searches it would route refuse.
    graph_route_ = on;
    if (min_cells > 0) graph_min_cells_ = min_cells;
    graph_built_ = graph_route_ && live_cell_count() >= graph_min_cells_;
    ++generation_;
}

void FlatCellIndex::set_centroid_sq8(bool on) {  // :2873-2880
    centroid_sq8_ = on;
    if (on)
        rebuild_centroid_sq8();
    else
        cent_sq8_.clear();
    ++generation_;
}

void FlatCellIndex::set_two_stage(bool on, size_t mult) {  // :2882-2888
    two_stage_ = on;
    shortlist_mult_ = std::max<size_t>(mult, 1);
    if (on) rebuild_centroid_codes();
    ++generation_;
}

void FlatCellIndex::set_adaptive(bool on, float margin) {  // :2899-2902
    adaptive_ = on;
    at_margin_ = margin;
}

void FlatCellIndex::set_per_dim_sq(bool on) {  // :2908-2915
    per_dim_sq_ = on;
    store_ok_ = false;  // the rows' layout changes
    if (on) {
        i8_rerank_ = true;
        f16_rerank_ = false;
        keep_f32_ = false;
    }
}

void FlatCellIndex::set_f16_rerank(bool on) {  // :2922-2928
    if (on) throw Unsupported("the f16 rerank store is not implemented by this library (f32 or per-dimension SQ8 only)");
    f16_rerank_ = false;
}

void FlatCellIndex::set_fastscan(bool on) {  // :2962-2968
    fastscan_ = on;
    if (!on) {
        fs_codes_.clear();
        fs_off_.clear();
        ++generation_;
    }
}

void FlatCellIndex::set_replication(size_t max_assign, float spill_margin) {  // :2970-2974
    max_assign_ = std::max<size_t>(max_assign, 1);
    spill_margin_ = std::max(spill_margin, 0.0f);
    spill_lambda_ = 0.0f;
}

void FlatCellIndex::set_orthogonal_polysemy(size_t homes, float lam) {  // :2979-2984
    max_assign_ = std::max<size_t>(homes, 1);
    spill_margin_ = 0.0f;
    spill_lambda_ = std::max(lam, 1e-6f);
}

void FlatCellIndex::set_tags(const std::vector<uint64_t>& ids, const std::vector<uint32_t>& tags) {  // :3535-3548
    if (ids.size() != tags.size()) throw ValueError("ids/tags length mismatch");
    if (tags_.size() < ext_ids_.size()) tags_.resize(ext_ids_.size(), 0);
    for (size_t i = 0; i < ids.size(); ++i) {
        if (const uint32_t* slot = id_to_slot_.find(ids[i])) tags_[*slot] = tags[i];
    }
    ++generation_;  // the uploaded arena carries the tags
}

void FlatCellIndex::set_filter(std::optional<uint32_t> lo, std::optional<uint32_t> hi) {  // :3553-3558
    if (!lo && !hi)
        tag_filter_.reset();
    else
        tag_filter_ = std::make_pair(lo.value_or(0u), hi.value_or(UINT32_MAX));
}

// ---------------------------------------------------------------- centroids and derived state

void FlatCellIndex::train_centroids(const float* data, size_t n_all, size_t n_cells, size_t sample,
                                    uint64_t seed) {  // src/index.rs:2762-2804
    std::vector<float> train;
    size_t n_train;
    if (sample > 0 && n_all > sample) {
        size_t stride = n_all / sample;
        train.resize(sample * dim_);
        for (size_t i = 0; i < sample; ++i) {
            size_t s = std::min(i * stride, n_all - 1);
            std::memcpy(&train[i * dim_], data + s * dim_, dim_ * sizeof(float));
        }
        n_train = sample;
    } else {
        train.assign(data, data + n_all * dim_);
        n_train = n_all;
    }
    if (n_train == 0) throw ValueError("train_centroids needs at least one vector");
    KMeansRunner runner;
    if (gpu_build_) runner = gpu_kmeans_runner();
    std::vector<float> cents = hierarchical_kmeans(train.data(), n_train, dim_, n_cells, seed, gpu_build_ ? &runner : nullptr);
    size_t k = cents.size() / dim_;
    cells_.clear();
    cells_.resize(k);
    for (size_t c = 0; c < k; ++c) {
        float* row = &cents[c * dim_];
        float nrm = -0.0f;
        for (size_t j = 0; j < dim_; ++j) nrm += row[j] * row[j];
        nrm = std::sqrt(nrm);
        if (nrm > 1e-12f)
            for (size_t j = 0; j < dim_; ++j) row[j] /= nrm;
        cells_[c].sum.assign(dim_, 0.0f);
        cells_[c].centroid.assign(row, row + dim_);
    }
    touch();
    refresh_derived();
}

void FlatCellIndex::set_centroids(const float* cents, size_t n) {  // :2806-2821
    cells_.clear();
    cells_.resize(n);
    for (size_t c = 0; c < n; ++c) {
        cells_[c].sum.assign(dim_, 0.0f);
        cells_[c].centroid.assign(cents + c * dim_, cents + (c + 1) * dim_);
    }
    touch();
    refresh_derived();
}

size_t FlatCellIndex::live_cell_count() const {
    size_t n = 0;
    for (const auto& c : cells_) n += !c.members.empty();
    return n;
}

void FlatCellIndex::recompute_centroid(Cell& c) {  // src/index.rs:380-394
    if (c.members.empty()) return;
    float norm = 0.0f;
    for (float v : c.sum) norm += v * v;
    norm = std::sqrt(norm);
    if (norm > 1e-12f)
        for (size_t j = 0; j < dim_; ++j) c.centroid[j] = c.sum[j] / norm;
}

void FlatCellIndex::rebuild_centroid_codes() {  // src/index.rs:711-723
    size_t nw = n_words_;
    std::vector<float> rot(dim_pad_);
    cent_bits_.assign(cells_.size() * nw, 0);
    for (size_t ci = 0; ci < cells_.size(); ++ci) {
        rotate(cells_[ci].centroid.data(), dim_, rot_signs_.data(), dim_pad_, rot.data());
        pack_signs_trunc(rot.data(), dim_pad_, &cent_bits_[ci * nw], nw);
    }
}

void FlatCellIndex::rebuild_centroid_sq8() {  // src/index.rs:730-775
    size_t d = dim_;
    std::vector<float> lo(d, INFINITY), hi(d, -INFINITY);
    bool any = false;
    for (const auto& c : cells_) {
        if (c.members.empty()) continue;
        any = true;
        for (size_t j = 0; j < d; ++j) {
            float v = c.centroid[j];
            if (v < lo[j]) lo[j] = v;
            if (v > hi[j]) hi[j] = v;
        }
    }
    if (!any) {
        cent_sq8_.clear();
        csq_min_.clear();
        csq_step_.clear();
        return;
    }
    csq_step_.resize(d);
    for (size_t j = 0; j < d; ++j) {
        float s = (hi[j] - lo[j]) / 255.0f;
        csq_step_[j] = s > 1e-12f ? s : 1e-12f;
    }
    csq_min_ = lo;
    cent_sq8_.assign(cells_.size() * d, 0);
    for (size_t ci = 0; ci < cells_.size(); ++ci)
        for (size_t j = 0; j < d; ++j) {
            float q = std::round((cells_[ci].centroid[j] - csq_min_[j]) / csq_step_[j]);
            q = std::min(std::max(q, 0.0f), 255.0f);
            cent_sq8_[ci * d + j] = static_cast<uint8_t>(q);
        }
}

// The session's row store's current token (the arena description names it, so the upload reads
// the rows where they are).
// A store whose slot count differs from the index's no longer mirrors it: the mirror ends and the
// host steps (exact restatements too) take over, so the index stays usable.
void FlatCellIndex::refresh_store_token() {
    uint32_t n = 0;
    gpu_->check(gpu_api().store_info(gpu_->ctx_, &store_token_, &n), "maivs_gpu_store_info");
    if (n != ext_ids_.size()) store_ok_ = false;
}

// recompute_radii on the GPU, from the row store: the device returns each cell's (p99 + 1)-th
// largest and smallest clamped member dot, and the angles are their acos here. acosf is
// non-increasing on [-1, 1], so these are the reference's p99-th smallest and largest angle.
bool FlatCellIndex::gpu_radii() {
    if (!gpu_build_ || !store_ok_ || !gpu_ || f16_rerank_) return false;
    uint32_t mode;
    if (per_dim_sq_)
        mode = 1;
    else if (keep_f32_)
        mode = 0;
    else
        mode = 2;
    if (mode == 0 ? vecs_f32_.empty() : scan_i8_.empty()) return false;
    const size_t M = cells_.size();
    std::vector<uint32_t> off(M + 1, 0), mem;
    for (size_t c = 0; c < M; ++c) off[c + 1] = off[c] + static_cast<uint32_t>(cells_[c].members.size());
    mem.resize(off[M]);
    std::vector<float> cents(M * dim_);
    for (size_t c = 0; c < M; ++c) {
        std::copy(cells_[c].members.begin(), cells_[c].members.end(), mem.begin() + off[c]);
        std::memcpy(&cents[c * dim_], cells_[c].centroid.data(), dim_ * sizeof(float));
    }
    maivs_radii_desc D{};
    D.n_cells = static_cast<uint32_t>(M);
    D.dim = static_cast<uint32_t>(dim_);
    D.mode = mode;
    D.inv_scale = quant_scale_ > 0.0f ? 1.0f / quant_scale_ : 1.0f;
    D.mem_off = off.data();
    D.members = mem.data();
    D.centroids = cents.data();
    D.sq_min = sq_min_.empty() ? nullptr : sq_min_.data();
    D.sq_step = sq_step_.empty() ? nullptr : sq_step_.data();
    std::vector<float> p99(M), mn(M);
    gpu_->check(gpu_api().store_radii(gpu_->ctx_, &D, p99.data(), mn.data()), "maivs_gpu_store_radii");
    for (size_t c = 0; c < M; ++c) {
        Cell& cell = cells_[c];
        if (cell.members.empty()) {
            cell.r_bound = 0.0f;
            cell.r_max = 0.0f;
        } else {
            cell.r_bound = std::acos(p99[c]);
            cell.r_max = std::acos(mn[c]);
        }
    }
    return true;
}

void FlatCellIndex::recompute_radii() {  // src/index.rs:817-861
    if (gpu_radii()) return;
    float inv = quant_scale_ > 0.0f ? 1.0f / quant_scale_ : 1.0f;
    size_t d = dim_;
    parallel_for(cells_.size(), [&](size_t ci) {
        Cell& cell = cells_[ci];
        if (cell.members.empty()) {
            cell.r_bound = 0.0f;
            cell.r_max = 0.0f;
            return;
        }
        const float* mu = cell.centroid.data();
        std::vector<float> w;
        float base = 0.0f;
        if (per_dim_sq_) {
            w.resize(d);
            for (size_t j = 0; j < d; ++j) w[j] = sq_step_[j] * mu[j];
            base = -0.0f;
            for (size_t j = 0; j < d; ++j) base += sq_min_[j] * mu[j];
        }
        std::vector<float> angs;
        angs.reserve(cell.members.size());
        for (uint32_t slot : cell.members) {
            size_t off = static_cast<size_t>(slot) * d;
            float dot;
            if (per_dim_sq_)
                dot = dot_f32_u8(w.data(), reinterpret_cast<const uint8_t*>(&scan_i8_[off]), d) + base;
            else if (keep_f32_)
                dot = dot_f32(mu, &vecs_f32_[off], d);
            else
                dot = dot_f32_i8(mu, &scan_i8_[off], d) * inv;
            angs.push_back(std::acos(std::min(std::max(dot, -1.0f), 1.0f)));
        }
        size_t len = angs.size();
        size_t p99 = static_cast<size_t>(std::ceil(static_cast<float>(len) * 0.99f));
        p99 = p99 > 0 ? p99 - 1 : 0;
        p99 = std::min(p99, len - 1);
        float r_max = -INFINITY;
        for (float a : angs) r_max = std::max(r_max, a);
        std::nth_element(angs.begin(), angs.begin() + p99, angs.end());
        cell.r_bound = angs[p99];
        cell.r_max = r_max;
    }, 16);
}

void FlatCellIndex::refresh_derived() {  // src/index.rs:864-878
    recompute_radii();
    if (two_stage_) rebuild_centroid_codes();
    if (centroid_sq8_) rebuild_centroid_sq8();
    graph_built_ = graph_route_ && live_cell_count() >= graph_min_cells_;  // rebuild_centroid_graph
    maybe_rebuild_centroid_tree();
    ++generation_;
}

void FlatCellIndex::maybe_rebuild_centroid_tree() {  // src/index.rs:667-677
    size_t live = live_cell_count();
    if (tree_ && tree_cells_ == live) return;
    rebuild_centroid_tree();
}

void FlatCellIndex::rebuild_centroid_tree() {  // src/index.rs:684-708
    ++generation_;  // the uploaded arena carries the tree
    tree_cells_ = live_cell_count();
    std::vector<uint32_t> live;
    for (size_t i = 0; i < cells_.size(); ++i)
        if (!cells_[i].members.empty()) live.push_back(static_cast<uint32_t>(i));
    if (live.empty() && !cells_.empty())
        for (size_t i = 0; i < cells_.size(); ++i) live.push_back(static_cast<uint32_t>(i));
    if (!tree_route_ || live.size() < tree_min_cells_) {
        tree_.reset();
        return;
    }
    std::vector<float> flat(live.size() * dim_);
    for (size_t i = 0; i < live.size(); ++i)
        std::memcpy(&flat[i * dim_], cells_[live[i]].centroid.data(), dim_ * sizeof(float));
    auto t = std::make_unique<CentroidTree>();
    KMeansRunner runner;
    if (gpu_build_) runner = gpu_kmeans_runner();
    if (t->build(flat.data(), live, dim_, rot_signs_.data(), dim_pad_, n_words_, tree_fanout_, tree_beam_frac_,
                 gpu_build_ ? &runner : nullptr))
        tree_ = std::move(t);
    else
        tree_.reset();
}

// ---------------------------------------------------------------- placement

namespace {
// Order used wherever the reference selects/sorts by score with an unstable sort: score
// descending, then cell id ascending (the reference leaves exact-tie order unspecified).
inline bool by_score_desc(const std::pair<uint32_t, float>& a, const std::pair<uint32_t, float>& b) {
    if (a.second != b.second) return a.second > b.second;
    return a.first < b.first;
}
}  // namespace

std::vector<uint32_t> FlatCellIndex::pick_orthogonal(std::vector<std::pair<uint32_t, float>>& scored) const {
    // src/index.rs:2523-2560
    const size_t kPool = 16;
    size_t pool = std::min(kPool, scored.size());
    if (pool < scored.size()) {
        std::nth_element(scored.begin(), scored.begin() + (pool - 1), scored.end(), by_score_desc);
        scored.resize(pool);
    }
    std::sort(scored.begin(), scored.end(), by_score_desc);
    size_t r = std::min(max_assign_, scored.size());
    std::vector<std::pair<uint32_t, float>> homes{scored[0]};
    std::vector<bool> taken(scored.size(), false);
    taken[0] = true;
    while (homes.size() < r) {
        size_t best_j = SIZE_MAX;
        float best_l = INFINITY;
        for (size_t j = 0; j < scored.size(); ++j) {
            if (taken[j]) continue;
            uint32_t cj = scored[j].first;
            float sj = scored[j].second;
            float loss = 2.0f - 2.0f * sj;
            for (const auto& h : homes) {
                float sh = h.second;
                float rn = std::sqrt(std::max(2.0f - 2.0f * sh, 1e-12f));
                float g = dot_f32(cells_[h.first].centroid.data(), cells_[cj].centroid.data(), dim_);
                float p = (1.0f - sh - sj + g) / rn;
                loss += spill_lambda_ * p * p;
            }
            if (loss < best_l) {
                best_j = j;
                best_l = loss;
            }
        }
        if (best_j == SIZE_MAX) break;
        taken[best_j] = true;
        homes.push_back(scored[best_j]);
    }
    std::vector<uint32_t> out;
    for (auto& h : homes) out.push_back(h.first);
    return out;
}

std::vector<uint32_t> FlatCellIndex::assign_cells(const float* v) const {  // src/index.rs:2480-2509
    std::vector<std::pair<uint32_t, float>> scored(cells_.size());
    for (size_t i = 0; i < cells_.size(); ++i)
        scored[i] = {static_cast<uint32_t>(i), dot_f32(v, cells_[i].centroid.data(), dim_)};
    if (max_assign_ <= 1) {
        std::pair<uint32_t, float> best{0, -INFINITY};
        for (auto& s : scored)
            if (s.second > best.second) best = s;
        return {best.first};
    }
    if (spill_lambda_ > 0.0f) return pick_orthogonal(scored);
    size_t r = std::min(max_assign_, scored.size());
    std::nth_element(scored.begin(), scored.begin() + (r - 1), scored.end(), by_score_desc);
    scored.resize(r);
    std::sort(scored.begin(), scored.end(), by_score_desc);
    float cutoff = scored[0].second - spill_margin_;
    std::vector<uint32_t> out;
    for (auto& s : scored)
        if (s.second >= cutoff) out.push_back(s.first);
    return out;
}

std::vector<uint32_t> FlatCellIndex::assign_cells_routed(const float* v, std::vector<float>& rot,
                                                         std::vector<uint64_t>& qb, TreeScratch& ts,
                                                         std::vector<uint32_t>& out) const {
    // src/index.rs:2442-2478
    if (!tree_) return assign_cells(v);
    rotate(v, dim_, rot_signs_.data(), dim_pad_, rot.data());
    pack_signs_trunc(rot.data(), dim_pad_, qb.data(), n_words_);
    size_t want = std::max<size_t>(64, max_assign_ * 8);
    tree_->search(qb.data(), want, ts, out);
    if (out.empty()) return assign_cells(v);
    std::vector<std::pair<uint32_t, float>> scored;
    scored.reserve(out.size());
    for (uint32_t ci : out) scored.emplace_back(ci, dot_f32(v, cells_[ci].centroid.data(), dim_));
    if (max_assign_ <= 1) {
        auto best = scored[0];
        for (auto& s : scored)
            if (s.second > best.second) best = s;
        return {best.first};
    }
    if (spill_lambda_ > 0.0f) return pick_orthogonal(scored);
    size_t r = std::min(max_assign_, scored.size());
    std::nth_element(scored.begin(), scored.begin() + (r - 1), scored.end(), by_score_desc);
    scored.resize(r);
    std::sort(scored.begin(), scored.end(), by_score_desc);
    float cutoff = scored[0].second - spill_margin_;
    std::vector<uint32_t> res;
    for (auto& s : scored)
        if (s.second >= cutoff) res.push_back(s.first);
    return res;
}

// Per-slot codes: sign bits (binary mode) and the i8/SQ8 copy, src/index.rs:2582-2610, 3083-3123.
void FlatCellIndex::encode_slot(const float* v, uint64_t* bits_out, int8_t* i8_out) const {
    if (bits_out) {
        std::vector<float> rot(dim_pad_);
        rotate(v, dim_, rot_signs_.data(), dim_pad_, rot.data());
        pack_signs_trunc(rot.data(), dim_pad_, bits_out, n_words_);
    }
    if (i8_out) {
        if (per_dim_sq_) {
            for (size_t j = 0; j < dim_; ++j) {
                float c = std::round((v[j] - sq_min_[j]) / sq_step_[j]);
                c = std::min(std::max(c, 0.0f), 255.0f);
                i8_out[j] = static_cast<int8_t>(static_cast<uint8_t>(c));
            }
        } else {
            for (size_t j = 0; j < dim_; ++j) {
                float c = std::round(v[j] * quant_scale_);
                c = std::min(std::max(c, -127.0f), 127.0f);
                i8_out[j] = static_cast<int8_t>(c);
            }
        }
    }
}

// A C view of a flattened tree (valid while tf lives).
void fill_tree_desc(const TreeFlat& tf, maivs_tree_desc& td) {
    td = maivs_tree_desc{};
    td.n_levels = static_cast<uint32_t>(tf.level_n.size());
    td.n_leaf = static_cast<uint32_t>(tf.leaf_cells.size());
    td.beam_frac = tf.beam_frac;
    td.min_beam = tf.min_beam;
    td.level_n = tf.level_n.data();
    td.level_codes = tf.level_codes.data();
    td.child_start = tf.child_start.data();
    td.child_len = tf.child_len.data();
    td.leaf_codes = tf.leaf_codes.data();
    td.leaf_cells = tf.leaf_cells.data();
}

// add_batch's per-vector work on the GPU (maivs_gpu_place): the homes of every input vector
// (assign_cells_routed), its 1-bit code and, when kept, its i8 / SQ8 copy.
void FlatCellIndex::place_on_gpu(const float* data, size_t n, bool store_i8, std::vector<std::vector<uint32_t>>& asg,
                                 std::vector<uint64_t>& bits, std::vector<int8_t>& i8, const uint32_t* slots,
                                 float* sums) {
    session();
    const size_t M = cells_.size(), ma = max_assign_;
    std::vector<float> cents(M * dim_);
    for (size_t c = 0; c < M; ++c) std::memcpy(&cents[c * dim_], cells_[c].centroid.data(), dim_ * sizeof(float));
    maivs_place_desc D{};
    D.dim = static_cast<uint32_t>(dim_);
    D.dim_pad = static_cast<uint32_t>(dim_pad_);
    D.n_words = static_cast<uint32_t>(n_words_);
    D.n_cells = static_cast<uint32_t>(M);
    D.max_assign = static_cast<uint32_t>(ma);
    D.spill_lambda = spill_lambda_;
    D.spill_margin = spill_margin_;
    D.code_mode = store_i8 ? (per_dim_sq_ ? 1u : 2u) : 0u;
    D.quant_scale = quant_scale_;
    D.rot_signs = rot_signs_.data();
    D.centroids = cents.data();
    D.sq_min = sq_min_.empty() ? nullptr : sq_min_.data();
    D.sq_step = sq_step_.empty() ? nullptr : sq_step_.data();
    TreeFlat tf;
    maivs_tree_desc td{};
    if (tree_) {
        tree_->export_flat(std::max<size_t>(64, ma * 8), tf);
        fill_tree_desc(tf, td);
        D.tree = td;
        D.tree_want = static_cast<uint32_t>(std::max<size_t>(64, ma * 8));  // the want of src/index.rs:2452
    }
    std::vector<uint32_t> homes(n * ma);
    bits.assign(n * n_words_, 0);
    if (store_i8) i8.assign(n * dim_, 0);
    // batches of at most 2^20 vectors keep the device copy of the inputs bounded
    const size_t step = size_t{1} << 20;
    D.sums = sums;  // in and out: the chunks add in input order
    for (size_t b = 0; b < n; b += step) {
        const size_t m = std::min(step, n - b);
        D.store_slots = slots ? slots + b : nullptr;
        gpu_->check(gpu_api().place(gpu_->ctx_, &D, data + b * dim_, static_cast<uint32_t>(m), &homes[b * ma],
                                    &bits[b * n_words_], store_i8 ? &i8[b * dim_] : nullptr),
                    "maivs_gpu_place");
    }
    for (size_t i = 0; i < n; ++i) {
        asg[i].clear();
        for (size_t j = 0; j < ma; ++j)
            if (homes[i * ma + j] != UINT32_MAX) asg[i].push_back(homes[i * ma + j]);
    }
}

void FlatCellIndex::add_batch(const std::vector<uint64_t>& ids, const float* data, size_t n) {
    // src/index.rs:2987-3212
    if (cells_.empty()) throw ValueError("call set_centroids() before add_batch()");
    if (ids.size() != n) throw ValueError("shape mismatch");
    touch();
    // max |x| and the per-dimension ranges are order-free, so they are taken over chunks of rows
    // on several threads and then combined
    const size_t rows_per = 4096, nch = (n + rows_per - 1) / rows_per;
    if (quant_scale_ == 0.0f) {
        std::vector<float> part(nch, 0.0f);
        parallel_for(nch, [&](size_t ch) {
            float m = 0.0f;
            for (size_t i = ch * rows_per * dim_, e = std::min(n, (ch + 1) * rows_per) * dim_; i < e; ++i)
                m = std::max(m, std::fabs(data[i]));
            part[ch] = m;
        });
        float max_abs = 0.0f;
        for (float m : part) max_abs = std::max(max_abs, m);
        quant_scale_ = max_abs > 0.0f ? 127.0f / max_abs : 1.0f;
    }
    if (per_dim_sq_ && sq_min_.empty() && n > 0) {
        std::vector<float> plo(nch * dim_, INFINITY), phi(nch * dim_, -INFINITY);
        parallel_for(nch, [&](size_t ch) {
            float* lo = &plo[ch * dim_];
            float* hi = &phi[ch * dim_];
            for (size_t i = ch * rows_per, e = std::min(n, (ch + 1) * rows_per); i < e; ++i)
                for (size_t j = 0; j < dim_; ++j) {
                    float x = data[i * dim_ + j];
                    if (x < lo[j]) lo[j] = x;
                    if (x > hi[j]) hi[j] = x;
                }
        });
        std::vector<float> lo(dim_, INFINITY), hi(dim_, -INFINITY);
        for (size_t ch = 0; ch < nch; ++ch)
            for (size_t j = 0; j < dim_; ++j) {
                if (plo[ch * dim_ + j] < lo[j]) lo[j] = plo[ch * dim_ + j];
                if (phi[ch * dim_ + j] > hi[j]) hi[j] = phi[ch * dim_ + j];
            }
        sq_step_.resize(dim_);
        for (size_t j = 0; j < dim_; ++j) sq_step_[j] = std::max(hi[j] - lo[j], 1e-9f) / 255.0f;
        sq_min_ = lo;
    }
    const bool store_bits = scan_mode_ == ScanMode::Binary;
    const bool store_i8 = scan_mode_ == ScanMode::I8 || (scan_mode_ == ScanMode::Binary && i8_rerank_);
    const size_t nw = n_words_, ma = max_assign_;
    std::vector<std::vector<uint32_t>> asg(n);
    // GPU placement: homes, 1-bit codes and i8 / SQ8 copies of the whole batch, bit-identical
    std::vector<uint64_t> g_bits;
    std::vector<int8_t> g_i8;
    const bool on_gpu = gpu_build_ && n > 0;
    if (on_gpu) {
        // The session's row store: started by the first GPU add_batch of an empty index and kept
        // up by the following ones. Each input's slot is the one the loops below give it: free
        // slots from the back of the list first, then appended ones.
        session();
        if (ext_ids_.empty()) {
            const uint32_t flags = (keep_f32_ ? MAIVS_STORE_F32 : 0u) | (store_i8 ? MAIVS_STORE_CODES : 0u) |
                                   (store_bits ? MAIVS_STORE_BITS : 0u);
            gpu_->check(gpu_api().store_reset(gpu_->ctx_, static_cast<uint32_t>(dim_), static_cast<uint32_t>(nw), flags),
                        "maivs_gpu_store_reset");
            store_ok_ = true;
        }
        std::vector<uint32_t> slots;
        if (store_ok_) {
            slots.resize(n);
            const size_t nr = std::min(free_slots_.size(), n);
            for (size_t i = 0; i < n; ++i)
                slots[i] = static_cast<uint32_t>(i < nr ? free_slots_[free_slots_.size() - 1 - i] : ext_ids_.size() + (i - nr));
        }
        // the primary sums on the device too (the same adds in the same order)
        const size_t M = cells_.size();
        std::vector<float> sums(M * dim_);
        for (size_t c = 0; c < M; ++c) std::memcpy(&sums[c * dim_], cells_[c].sum.data(), dim_ * sizeof(float));
        place_on_gpu(data, n, store_i8, asg, g_bits, g_i8, store_ok_ ? slots.data() : nullptr, sums.data());
        for (size_t c = 0; c < M; ++c) std::memcpy(cells_[c].sum.data(), &sums[c * dim_], dim_ * sizeof(float));
    } else {
        store_ok_ = false;  // the rows are written by the host alone
        // one scratch per chunk of 256 vectors keeps allocation out of the inner loop
        size_t nchunk = (n + 255) / 256;
        parallel_for(nchunk, [&](size_t ch) {
            std::vector<float> rot(dim_pad_);
            std::vector<uint64_t> qb(n_words_);
            TreeScratch ts;
            std::vector<uint32_t> out;
            size_t b = ch * 256, e = std::min(n, b + 256);
            for (size_t i = b; i < e; ++i) asg[i] = assign_cells_routed(data + i * dim_, rot, qb, ts, out);
        });
    }
    // the codes of input vector i into a slot's rows
    auto encode_input = [&](size_t i, uint64_t* bits_out, int8_t* i8_out) {
        if (!on_gpu) {
            encode_slot(data + i * dim_, bits_out, i8_out);
            return;
        }
        if (bits_out) std::memcpy(bits_out, &g_bits[i * nw], nw * 8);
        if (i8_out) std::memcpy(i8_out, &g_i8[i * dim_], dim_);
    };
    size_t n_reuse = std::min(free_slots_.size(), n);
    for (size_t i = 0; i < n_reuse; ++i) {
        const float* v = data + i * dim_;
        uint32_t s = free_slots_.back();
        free_slots_.pop_back();
        size_t off = static_cast<size_t>(s) * dim_;
        if (keep_f32_) std::memcpy(&vecs_f32_[off], v, dim_ * sizeof(float));
        encode_input(i, store_bits ? &bits_[static_cast<size_t>(s) * nw] : nullptr, store_i8 ? &scan_i8_[off] : nullptr);
        ext_ids_[s] = ids[i];
        slot_cell_[s] = asg[i][0];
        for (size_t j = 0; j < ma; ++j) slot_cells_[s * ma + j] = j < asg[i].size() ? asg[i][j] : UINT32_MAX;
        for (size_t j = 0; j < asg[i].size(); ++j) {
            Cell& c = cells_[asg[i][j]];
            c.members.push_back(s);
            if (j == 0 && !on_gpu)
                for (size_t d = 0; d < dim_; ++d) c.sum[d] += v[d];
        }
        id_to_slot_.set(ids[i], s);
        n_live_ += 1;
    }
    if (n_reuse < n) {
        // append_parallel, src/index.rs:2566-2667
        size_t m = n - n_reuse;
        const float* dat = data + n_reuse * dim_;
        size_t base = ext_ids_.size();
        // the new rows are written by several threads; every one is written in full
        if (keep_f32_) vecs_f32_.resize((base + m) * dim_);
        if (store_bits) bits_.resize((base + m) * nw);
        if (store_i8) scan_i8_.resize((base + m) * dim_);
        parallel_for(m, [&](size_t i) {
            if (keep_f32_) std::memcpy(&vecs_f32_[(base + i) * dim_], dat + i * dim_, dim_ * sizeof(float));
            encode_input(n_reuse + i, store_bits ? &bits_[(base + i) * nw] : nullptr,
                         store_i8 ? &scan_i8_[(base + i) * dim_] : nullptr);
        }, 512);
        for (size_t i = 0; i < m; ++i) {
            const auto& a = asg[n_reuse + i];
            ext_ids_.push_back(ids[n_reuse + i]);
            slot_cell_.push_back(a[0]);
            for (size_t j = 0; j < ma; ++j) slot_cells_.push_back(j < a.size() ? a[j] : UINT32_MAX);
        }
        id_to_slot_.reserve(id_to_slot_.size() + m);
        for (size_t i = 0; i < m; ++i) {
            uint32_t slot = static_cast<uint32_t>(base + i);
            for (uint32_t ci : asg[n_reuse + i]) cells_[ci].members.push_back(slot);
            id_to_slot_.set(ids[n_reuse + i], slot);
        }
        n_live_ += m;
    }
    if (n_reuse < n && !on_gpu) {
        const size_t m = n - n_reuse;
        const float* dat = data + n_reuse * dim_;
        // primary sums, parallel over cells, input order within a cell
        size_t M = cells_.size();
        std::vector<size_t> start(M + 1, 0);
        for (size_t i = 0; i < m; ++i) start[asg[n_reuse + i][0] + 1] += 1;
        for (size_t c = 0; c < M; ++c) start[c + 1] += start[c];
        std::vector<size_t> pos(start.begin(), start.end() - 1);
        std::vector<uint32_t> order(m);
        for (size_t i = 0; i < m; ++i) order[pos[asg[n_reuse + i][0]]++] = static_cast<uint32_t>(i);
        parallel_for(M, [&](size_t c) {
            for (size_t t = start[c]; t < start[c + 1]; ++t) {
                const float* v = dat + static_cast<size_t>(order[t]) * dim_;
                for (size_t d = 0; d < dim_; ++d) cells_[c].sum[d] += v[d];
            }
        }, 16);
    }
    if (on_gpu && store_ok_) refresh_store_token();
    for (auto& c : cells_) recompute_centroid(c);
    refresh_derived();
}

bool FlatCellIndex::remove(uint64_t id) {  // src/index.rs:3223-3276
    const uint32_t* found = id_to_slot_.find(id);
    if (!found) return false;
    const uint32_t slot = *found;
    id_to_slot_.erase(id);
    touch();
    uint32_t primary = slot_cell_[slot];
    size_t v0 = static_cast<size_t>(slot) * dim_;
    Cell& pc = cells_[primary];
    if (keep_f32_) {
        for (size_t j = 0; j < dim_; ++j) pc.sum[j] -= vecs_f32_[v0 + j];
    } else if (per_dim_sq_) {
        for (size_t j = 0; j < dim_; ++j) {
            float c = static_cast<float>(static_cast<uint8_t>(scan_i8_[v0 + j]));
            pc.sum[j] -= c * sq_step_[j] + sq_min_[j];
        }
    } else {
        float inv = 1.0f / quant_scale_;
        for (size_t j = 0; j < dim_; ++j) pc.sum[j] -= static_cast<float>(scan_i8_[v0 + j]) * inv;
    }
    size_t base = static_cast<size_t>(slot) * max_assign_;
    for (size_t j = 0; j < max_assign_; ++j) {
        uint32_t ci = slot_cells_[base + j];
        if (ci == UINT32_MAX) continue;
        auto& mem = cells_[ci].members;
        auto p = std::find(mem.begin(), mem.end(), slot);
        if (p != mem.end()) {
            *p = mem.back();
            mem.pop_back();
        }
        slot_cells_[base + j] = UINT32_MAX;
    }
    recompute_centroid(cells_[primary]);
    free_slots_.push_back(slot);
    n_live_ -= 1;
    return true;
}

// ---------------------------------------------------------------- compaction

void FlatCellIndex::compact() { compact_arena(); }

void FlatCellIndex::compact_arena() {  // src/index.rs:929-1112
    size_t old_n = ext_ids_.size();
    if (old_n == 0) return;
    const size_t d = dim_, nw = n_words_, ma = max_assign_;
    std::vector<uint32_t> new_of_old(old_n, UINT32_MAX), old_of_new;
    old_of_new.reserve(n_live_);
    for (size_t ci = 0; ci < cells_.size(); ++ci)
        for (uint32_t s : cells_[ci].members) {
            if (slot_cell_[s] != ci) continue;
            if (new_of_old[s] != UINT32_MAX) continue;
            new_of_old[s] = static_cast<uint32_t>(old_of_new.size());
            old_of_new.push_back(s);
        }
    // live slots no primary cell lists keep their data (slot order, deterministic)
    std::vector<uint32_t> missed;
    id_to_slot_.for_each([&](uint64_t, uint32_t s) {
        if (new_of_old[s] == UINT32_MAX) missed.push_back(s);
    });
    std::sort(missed.begin(), missed.end());
    for (uint32_t s : missed) {
        new_of_old[s] = static_cast<uint32_t>(old_of_new.size());
        old_of_new.push_back(s);
    }
    size_t n_new = old_of_new.size();
    // with a mirroring row store the rows move on the GPU (below, after the member lists)
    const bool on_gpu = gpu_build_ && store_ok_ && gpu_;
    if (keep_f32_ && !vecs_f32_.empty() && !on_gpu) {
        RowVec<float> v(n_new * d);
        for (size_t ns = 0; ns < n_new; ++ns)
            std::memcpy(&v[ns * d], &vecs_f32_[static_cast<size_t>(old_of_new[ns]) * d], d * sizeof(float));
        vecs_f32_.swap(v);
    }
    if (!scan_i8_.empty() && !on_gpu) {
        RowVec<int8_t> v(n_new * d);
        for (size_t ns = 0; ns < n_new; ++ns)
            std::memcpy(&v[ns * d], &scan_i8_[static_cast<size_t>(old_of_new[ns]) * d], d);
        scan_i8_.swap(v);
    }
    if (!bits_.empty() && nw > 0 && !on_gpu) {
        RowVec<uint64_t> v(n_new * nw);
        for (size_t ns = 0; ns < n_new; ++ns)
            std::memcpy(&v[ns * nw], &bits_[static_cast<size_t>(old_of_new[ns]) * nw], nw * 8);
        bits_.swap(v);
    }
    std::vector<uint64_t> ext(n_new);
    std::vector<uint32_t> scell(n_new), scells(n_new * ma, UINT32_MAX);
    for (size_t ns = 0; ns < n_new; ++ns) {
        size_t os = old_of_new[ns];
        ext[ns] = ext_ids_[os];
        scell[ns] = slot_cell_[os];
        for (size_t j = 0; j < ma; ++j) scells[ns * ma + j] = slot_cells_[os * ma + j];
    }
    if (!tags_.empty()) {
        std::vector<uint32_t> tg(n_new);
        for (size_t ns = 0; ns < n_new; ++ns) tg[ns] = old_of_new[ns] < tags_.size() ? tags_[old_of_new[ns]] : 0;
        tags_.swap(tg);
    }
    ext_ids_.swap(ext);
    slot_cell_.swap(scell);
    slot_cells_.swap(scells);
    for (auto& c : cells_) {
        std::vector<uint32_t> m2;
        m2.reserve(c.members.size());
        for (uint32_t m : c.members)
            if (new_of_old[m] != UINT32_MAX) m2.push_back(new_of_old[m]);
        std::sort(m2.begin(), m2.end());
        c.members.swap(m2);
    }
    id_to_slot_.clear();
    id_to_slot_.reserve(ext_ids_.size());
    for (size_t ns = 0; ns < ext_ids_.size(); ++ns) id_to_slot_.set(ext_ids_[ns], static_cast<uint32_t>(ns));
    free_slots_.clear();

    prim_len_.clear();
    rep_off_.clear();
    if (max_assign_ > 1 && scan_mode_ == ScanMode::Binary && nw > 0) {
        rep_off_.push_back(0);
        for (size_t ci = 0; ci < cells_.size(); ++ci) {
            std::vector<uint32_t> prim, repl;
            for (uint32_t m : cells_[ci].members) (slot_cell_[m] == ci ? prim : repl).push_back(m);
            std::sort(prim.begin(), prim.end());
            std::sort(repl.begin(), repl.end());
            prim_len_.push_back(static_cast<uint32_t>(prim.size()));
            rep_off_.push_back(rep_off_.back() + static_cast<uint32_t>(repl.size()));
            prim.insert(prim.end(), repl.begin(), repl.end());
            cells_[ci].members.swap(prim);
        }
    }
    fs_codes_.clear();
    fs_off_.clear();
    const bool pack = fastscan_ && scan_mode_ == ScanMode::Binary && nw > 0;
    const size_t bb = fs_block_bytes(nw);
    if (pack) {
        fs_off_.assign(cells_.size() + 1, 0);
        for (size_t ci = 0; ci < cells_.size(); ++ci)
            fs_off_[ci + 1] = fs_off_[ci] + static_cast<uint32_t>((cells_[ci].members.size() + kFsBlock - 1) / kFsBlock);
        fs_codes_.assign(static_cast<size_t>(fs_off_.back()) * bb, 0);
    }
    // flattened CSR for the arena descriptor
    mem_off_.assign(cells_.size() + 1, 0);
    for (size_t ci = 0; ci < cells_.size(); ++ci)
        mem_off_[ci + 1] = mem_off_[ci] + static_cast<uint32_t>(cells_[ci].members.size());
    members_flat_.resize(mem_off_.back());
    for (size_t ci = 0; ci < cells_.size(); ++ci)
        std::copy(cells_[ci].members.begin(), cells_[ci].members.end(), members_flat_.begin() + mem_off_[ci]);
    if (on_gpu) {
        // the store's rows move to their new slots, the FastScan blocks are packed from its codes,
        // and the compacted rows come back over the index's own arrays (each holds old_n >= n_new
        // rows, none of which is read again), which then shrink to n_new rows
        const bool f32 = keep_f32_ && !vecs_f32_.empty(), i8 = !scan_i8_.empty(), b = !bits_.empty() && nw > 0;
        if ((f32 && vecs_f32_.size() < n_new * d) || (i8 && scan_i8_.size() < n_new * d) || (b && bits_.size() < n_new * nw))
            throw std::runtime_error("compact: a row array is shorter than the slot count");
        const uint32_t M = static_cast<uint32_t>(cells_.size());
        gpu_->check(gpu_api().store_compact(gpu_->ctx_, old_of_new.data(), static_cast<uint32_t>(n_new), M, mem_off_.data(),
                                            members_flat_.data(), pack ? fs_off_.data() : nullptr,
                                            pack ? fs_codes_.data() : nullptr, f32 ? vecs_f32_.data() : nullptr,
                                            i8 ? scan_i8_.data() : nullptr, b ? bits_.data() : nullptr),
                    "maivs_gpu_store_compact");
        if (f32) vecs_f32_.resize(n_new * d);
        if (i8) scan_i8_.resize(n_new * d);
        if (b) bits_.resize(n_new * nw);
        refresh_store_token();
    } else if (pack) {
        parallel_for(cells_.size(), [&](size_t ci) {
            const auto& mem = cells_[ci].members;
            size_t nb = fs_off_[ci + 1] - fs_off_[ci];
            for (size_t b = 0; b < nb; ++b) {
                const uint64_t* lanes[kFsBlock];
                size_t lo = b * kFsBlock, hi = std::min(lo + kFsBlock, mem.size());
                for (size_t i = lo; i < hi; ++i) lanes[i - lo] = &bits_[static_cast<size_t>(mem[i]) * nw];
                fs_pack_block(lanes, hi - lo, nw, &fs_codes_[(fs_off_[ci] + b) * bb]);
            }
        }, 16);
    }
    ++generation_;
    compacted_ = true;
}

// ---------------------------------------------------------------- search

std::string FlatCellIndex::cellmajor_blocker(bool cell_major) const {
    // the cm_ok gate of src/index.rs:3343-3348, plus what the MI355X path needs
    if (!cell_major) return "cell_major=False selects the per-query path";
    if (scan_mode_ != ScanMode::Binary) return "the batched path needs scan_mode='binary'";
    if (!compacted_) return "the index is not compacted (call compact() after add_batch/remove)";
    if (!(max_assign_ == 1 || !rep_off_.empty())) return "polysemic runs are missing (compact() again)";
    if (!fastscan_ || fs_off_.empty()) return "the MI355X scan needs set_fastscan(True) before compact()";
    if (!(two_stage_ && !cent_bits_.empty()) && !tree_ && graph_built_)
        return "the centroid-graph router is not implemented by this library (set_graph_route(False, ...))";
    if (f16_rerank_) return "the f16 rerank store is not implemented by this library";
    if (!per_dim_sq_ && (!keep_f32_ || vecs_f32_.empty()))
        return "the rerank needs the f32 rows or the per-dimension SQ8 store";
    if (n_words_ * 64 > 65536) return "codes longer than 65536 bits";
    return "";
}

const maivs_arena_desc* FlatCellIndex::arena_desc() {
    if (cells_.empty()) return nullptr;
    size_t M = cells_.size();
    if (!compacted_) {
        // the member lists as they stand, in any order after deletes and inserts: only the per-query
        // path's Hamming branch runs on them, over the per-slot codes
        mem_off_.assign(M + 1, 0);
        for (size_t c = 0; c < M; ++c) mem_off_[c + 1] = mem_off_[c] + static_cast<uint32_t>(cells_[c].members.size());
        members_flat_.resize(mem_off_.back());
        for (size_t c = 0; c < M; ++c)
            std::copy(cells_[c].members.begin(), cells_[c].members.end(), members_flat_.begin() + mem_off_[c]);
    }
    const bool fs = compacted_ && fastscan_ && !fs_off_.empty();
    cents_flat_.resize(M * dim_);
    r_bound_flat_.resize(M);
    for (size_t c = 0; c < M; ++c) {
        std::memcpy(&cents_flat_[c * dim_], cells_[c].centroid.data(), dim_ * sizeof(float));
        r_bound_flat_[c] = cells_[c].r_bound;
    }
    maivs_arena_desc& a = desc_;
    a = maivs_arena_desc{};
    a.dim = static_cast<uint32_t>(dim_);
    a.dim_pad = static_cast<uint32_t>(dim_pad_);
    a.n_words = static_cast<uint32_t>(n_words_);
    a.n_cells = static_cast<uint32_t>(M);
    a.n_slots = static_cast<uint32_t>(ext_ids_.size());
    a.max_assign = static_cast<uint32_t>(max_assign_);
    a.rerank_mode = per_dim_sq_ ? MAIVS_RERANK_SQ8 : MAIVS_RERANK_F32;
    a.fs_codes = fs && !fs_codes_.empty() ? fs_codes_.data() : nullptr;
    a.fs_off = fs ? fs_off_.data() : nullptr;
    a.slot_codes = bits_.size() >= ext_ids_.size() * n_words_ && !bits_.empty() ? bits_.data() : nullptr;
    a.store_token = store_ok_ ? store_token_ : 0;
    a.mem_off = mem_off_.data();
    a.members = members_flat_.data();
    a.slot_cells = slot_cells_.data();
    // centroid codes only while two-stage routing keeps them current (set_two_stage(False) leaves
    // the last ones behind, src/index.rs:2882-2888)
    a.cent_bits = two_stage_ && cent_bits_.size() == M * n_words_ ? cent_bits_.data() : nullptr;
    a.cent_sq8 = (centroid_sq8_ && !cent_sq8_.empty()) ? cent_sq8_.data() : nullptr;
    a.centroids = cents_flat_.data();
    a.csq_min = csq_min_.empty() ? nullptr : csq_min_.data();
    a.csq_step = csq_step_.empty() ? nullptr : csq_step_.data();
    a.r_bound = r_bound_flat_.data();
    a.rot_signs = rot_signs_.data();
    a.vecs_f32 = vecs_f32_.empty() ? nullptr : vecs_f32_.data();
    a.sq8_codes = scan_i8_.empty() ? nullptr : reinterpret_cast<const uint8_t*>(scan_i8_.data());
    a.sq_min = sq_min_.empty() ? nullptr : sq_min_.data();
    a.sq_step = sq_step_.empty() ? nullptr : sq_step_.data();
    if (!tags_.empty()) {
        // slots added after set_tags carry tag 0 (the reference indexes past its tag array there)
        if (tags_.size() < ext_ids_.size()) tags_.resize(ext_ids_.size(), 0);
        a.tags = tags_.data();
    }
    // the centroid tree, for the per-query path's routing (route_query, src/index.rs:1185-1206)
    if (tree_) {
        tree_->export_flat(64, tree_flat_);
        fill_tree_desc(tree_flat_, tree_desc_);
        a.tree = &tree_desc_;
    }
    return &desc_;
}

maivs_search_params FlatCellIndex::search_params(size_t k, size_t nprobe, float tc, float beta) const {
    maivs_search_params p{};
    p.k = static_cast<uint32_t>(k);
    p.nprobe = static_cast<uint32_t>(nprobe);
    p.target_confidence = tc;
    p.beta = beta;
    p.rerank_factor = static_cast<uint32_t>(rerank_factor_);
    p.shortlist_mult = static_cast<uint32_t>(shortlist_mult_);
    p.adaptive = adaptive_ ? 1u : 0u;
    p.at_margin = at_margin_;
    // route_batch only with two-stage routing and centroid codes, else route_query's routing
    // (src/index.rs:1241, 1875)
    p.route_mode = (two_stage_ && !cent_bits_.empty()) ? 0u : 1u;
    // filtering = tag_filter.is_some() && !tags.is_empty() (src/index.rs:1430-1431)
    if (tag_filter_ && !tags_.empty()) {
        p.filter = 1;
        p.tag_lo = tag_filter_->first;
        p.tag_hi = tag_filter_->second;
    }
    return p;
}

std::string FlatCellIndex::perquery_blocker() const {
    // what the GPU per-query path runs: search_one's FastScan branch (src/index.rs:1689-1757) with
    // route_query's tree or two-stage router (:1185-1257)
    if (scan_mode_ != ScanMode::Binary) return "the per-query path needs scan_mode='binary'";
    if (!(fastscan_ && compacted_ && !fs_off_.empty())) {
        // the Hamming branch (src/index.rs:1694-1760)
        if (asym_cascade_ > 0) return "the asymmetric cascade (set_asym_cascade) is not implemented by this library";
        if (bits_.size() < ext_ids_.size() * n_words_ || bits_.empty())
            return "the Hamming scan needs the per-slot sign codes";
    }
    if (!tree_ && graph_built_)
        return "the centroid-graph router is not implemented by this library (set_graph_route(False, ...))";
    if (par_scan_ && !adaptive_ && max_assign_ <= 1)
        return "set_parallel_scan's within-query parallel scan is not implemented by this library";
    if (f16_rerank_) return "the f16 rerank store is not implemented by this library";
    if (!per_dim_sq_ && (!keep_f32_ || vecs_f32_.empty()))
        return "the rerank needs the f32 rows or the per-dimension SQ8 store";
    if (n_words_ * 64 > 65536) return "codes longer than 65536 bits";
    return "";
}

void FlatCellIndex::ensure_uploaded() {
    // called with the session's mutex held (searches serialise on it)
    if (gpu_->uploaded_gen != generation_) {
        const maivs_arena_desc* desc = arena_desc();
        if (!desc) throw std::runtime_error("the index has no cells");
        maivs_arena_desc a = *desc;
        if (store_ok_) {
            // the rows are in the session's row store: the upload reads them there, and fails
            // rather than falling back to a host copy if the store and the index ever disagree
            a.vecs_f32 = nullptr;
            a.sq8_codes = nullptr;
            a.fs_codes = nullptr;
            a.slot_codes = nullptr;
        }
        gpu_->check(gpu_api().upload(gpu_->ctx_, &a), "maivs_gpu_upload_arena");
        gpu_->uploaded_gen = generation_;
    }
}

bool FlatCellIndex::takes_cellmajor(size_t nq, bool cell_major) const {
    // cm_ok, src/index.rs:3343-3348
    return cell_major && scan_mode_ == ScanMode::Binary && compacted_ && (max_assign_ == 1 || !rep_off_.empty()) &&
           (!tag_filter_ || batched_filter_) && nq >= 2 * static_cast<size_t>(std::max(num_threads(), 1u));
}

void FlatCellIndex::search_batch(const float* q, size_t nq, size_t k, size_t nprobe, float tc, float beta,
                                 bool cell_major, std::vector<uint64_t>& ids, std::vector<float>& scores,
                                 maivs_gpu_stats* stats) {
    // src/index.rs:3317-3392
    ids.assign(nq * k, UINT64_MAX);
    scores.assign(nq * k, -INFINITY);
    if (cells_.empty() || n_live_ == 0 || nq == 0 || k == 0) return;
    const bool cm = takes_cellmajor(nq, cell_major);
    std::string why = cm ? cellmajor_blocker(true) : perquery_blocker();
    if (!why.empty()) throw Unsupported(why);
    GpuSession* g = session();
    std::lock_guard<std::mutex> lk(g->mu);
    ensure_uploaded();
    maivs_search_params p = search_params(k, nprobe, tc, beta);
    std::vector<uint32_t> slots(nq * k);
    std::vector<float> sc(nq * k);
    if (cm)
        gpu_->check(gpu_api().search(gpu_->ctx_, q, static_cast<uint32_t>(nq), &p, slots.data(), sc.data(), stats),
                    "maivs_gpu_search_batch");
    else
        gpu_->check(gpu_api().search_pq(gpu_->ctx_, q, static_cast<uint32_t>(nq), &p, slots.data(), sc.data(), stats),
                    "maivs_gpu_search_queries");
    for (size_t i = 0; i < nq * k; ++i) {
        if (slots[i] == UINT32_MAX) continue;
        ids[i] = ext_ids_[slots[i]];
        scores[i] = sc[i];
    }
}

void FlatCellIndex::search(const float* q, size_t k, size_t nprobe, float tc, float beta, std::vector<uint64_t>& ids,
                           std::vector<float>& scores) {
    // src/index.rs:3283-3305: one query through search_one; only the results found, best first
    ids.clear();
    scores.clear();
    if (cells_.empty() || n_live_ == 0 || k == 0) return;
    std::vector<uint64_t> i2;
    std::vector<float> s2;
    search_batch(q, 1, k, nprobe, tc, beta, false, i2, s2);
    for (size_t i = 0; i < k; ++i) {
        if (i2[i] == UINT64_MAX) break;
        ids.push_back(i2[i]);
        scores.push_back(s2[i]);
    }
}

std::pair<size_t, bool> FlatCellIndex::recommend() const {  // src/index.rs:3485-3497
    size_t n = std::max<size_t>(n_live_, 1);
    size_t target = std::max<size_t>(n / 128, 1);
    return {target, target >= 65536};
}

std::map<std::string, double> FlatCellIndex::stats() const {  // src/index.rs:3393-3472
    std::map<std::string, double> m;
    std::vector<size_t> sizes;
    for (const auto& c : cells_) sizes.push_back(c.members.size());
    double n = static_cast<double>(std::max<size_t>(n_live_, 1));
    size_t entries = std::accumulate(sizes.begin(), sizes.end(), size_t{0});
    m["n_live"] = static_cast<double>(n_live_);
    m["n_cells"] = static_cast<double>(cells_.size());
    m["free_slots"] = static_cast<double>(free_slots_.size());
    m["quant_scale"] = quant_scale_;
    m["scan_bytes_per_vec"] = scan_mode_ == ScanMode::F32 ? dim_ * 4.0
                              : scan_mode_ == ScanMode::I8 ? static_cast<double>(dim_)
                                                           : n_words_ * 8.0;
    m["cell_size_mean"] = static_cast<double>(entries) / static_cast<double>(std::max<size_t>(cells_.size(), 1));
    m["cell_size_max"] = sizes.empty() ? 0.0 : static_cast<double>(*std::max_element(sizes.begin(), sizes.end()));
    m["cell_size_min"] = sizes.empty() ? 0.0 : static_cast<double>(*std::min_element(sizes.begin(), sizes.end()));
    m["max_assign"] = static_cast<double>(max_assign_);
    m["centroid_graph_nodes"] = 0.0;
    m["centroid_graph_bytes"] = 0.0;
    m["tree_depth"] = tree_ ? static_cast<double>(tree_->depth()) : 0.0;
    m["tree_top_width"] = tree_ ? static_cast<double>(tree_->top_width()) : 0.0;
    m["tree_bytes"] = tree_ ? static_cast<double>(tree_->bytes()) : 0.0;
    m["tree_fanout"] = static_cast<double>(tree_fanout_);
    m["tree_beam_frac"] = tree_beam_frac_;
    m["replication_factor"] = static_cast<double>(entries) / n;
    double bytes = vecs_f32_.size() * 4.0 + scan_i8_.size() + bits_.size() * 8.0 + ext_ids_.size() * 12.0 +
                   slot_cells_.size() * 4.0;
    m["arena_bytes_per_vec"] = bytes / n;
    double arena_cap = vecs_f32_.capacity() * 4.0 + scan_i8_.capacity() + bits_.capacity() * 8.0 +
                       ext_ids_.capacity() * 8.0 + slot_cell_.capacity() * 4.0 + slot_cells_.capacity() * 4.0 +
                       tags_.capacity() * 4.0 + free_slots_.capacity() * 4.0;
    double cells_b = 0.0;
    for (const auto& c : cells_)
        cells_b += c.members.capacity() * 4.0 + c.sum.capacity() * 4.0 + c.centroid.capacity() * 4.0 + sizeof(Cell);
    double side = cent_bits_.capacity() * 8.0 + cent_sq8_.capacity() + (csq_min_.capacity() + csq_step_.capacity()) * 4.0 +
                  (tree_ ? tree_->bytes() : 0.0) + (prim_len_.capacity() + rep_off_.capacity()) * 4.0 +
                  fs_codes_.capacity() + fs_off_.capacity() * 4.0;
    double idmap = id_to_slot_.size() * (sizeof(uint64_t) + sizeof(uint32_t) + 1.0);
    m["member_entries"] = static_cast<double>(entries);
    m["rep_bytes"] = 0.0;
    m["total_bytes"] = arena_cap + cells_b + idmap + side;
    return m;
}

}  // namespace maivs
