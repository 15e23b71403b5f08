// FlatCellIndex::save / load: the reference's on-disk format "MAIVS2\0\1" (src/persist.rs:28-281),
// byte for byte, so a file written by either side loads on the other.
//
// Layout (little-endian; a "pod" block is a u64 element count followed by the raw elements):
//   magic[8]
//   u64 hdr[16]: dim, scan_mode (0 f32, 1 i8, 2 binary), rerank_factor, dim_pad, n_words, seed,
//                n_live, max_assign, shortlist_mult, i8_rerank, keep_f32, adaptive, two_stage,
//                tree_route, tree_min_cells, tree_fanout                      (src/persist.rs:86-109)
//   f32 quant_scale, spill_margin, at_margin, tree_beam_frac                  (:113-116)
//   pod bits u64, scan_i8 i8, rr_f16 u16, sq_min f32, sq_step f32, vecs_f32 f32, ext_ids u64,
//       slot_cell u32, free_slots u32, slot_cells u32, tags u32               (:118-131)
//   u64 n_cells, then per cell: pod members u32, pod sum f32, pod centroid f32, f32 r_bound, f32 r_max
//                                                                             (:133-140)
// Derived state is rebuilt on load, as src/persist.rs:153-281 and finish_load (src/index.rs:1116-1124)
// do: the rotation signs from the seed, id -> slot from ext_ids minus free slots, the centroid
// codes (two-stage), the SQ8 centroids and the centroid tree.
//
// Extension trailer, after the last cell. The reference's reader stops at the last cell and never
// looks further, so it loads these files unchanged; its own files have no trailer and load here
// with its defaults. The trailer keeps the settings the reference drops on load (FastScan, the
// orthogonal-polysemy strength, the compacted state, ...), so a loaded index is ready for the
// batched search without a rebuild: with fastscan and compacted set, load re-runs the compaction,
// which on an already compacted member order only repacks the FastScan blocks.
//   magic "MAIVSX\0\1", u64 n_fields, u64 field[n_fields]:
//   fastscan, compacted, centroid_sq8, graph_route, graph_min_cells, asym_cascade, par_scan,
//   spill_lambda (f32 bits in the low 32), f16_rerank (always 0 here). Unknown extra fields are
//   skipped, so later fields can be appended.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <unordered_set>

#include "cpu_kernels.h"
#include "index.h"

namespace maivs {

namespace {

constexpr char kMagic[8] = {'M', 'A', 'I', 'V', 'S', '2', '\0', '\x01'};
constexpr char kTrailerMagic[8] = {'M', 'A', 'I', 'V', 'S', 'X', '\0', '\x01'};
constexpr uint64_t kTrailerFields = 9;

class Writer {
public:
    explicit Writer(const std::string& path) : f_(std::fopen(path.c_str(), "wb")), path_(path) {
        if (!f_) throw IoError("cannot create " + path + ": " + std::strerror(errno));
    }
    ~Writer() {
        if (f_) std::fclose(f_);
    }
    void bytes(const void* p, size_t n) {
        if (n && std::fwrite(p, 1, n, f_) != n) throw IoError("write failed on " + path_);
    }
    void u64(uint64_t v) { bytes(&v, 8); }
    void f32(float v) { bytes(&v, 4); }
    template <class T, class A>
    void pod(const std::vector<T, A>& v) {
        u64(v.size());
        bytes(v.data(), v.size() * sizeof(T));
    }
    void close() {
        int rc = std::fclose(f_);
        f_ = nullptr;
        if (rc != 0) throw IoError("close failed on " + path_);
    }

private:
    std::FILE* f_;
    std::string path_;
};

class Reader {
public:
    explicit Reader(const std::string& path) : f_(std::fopen(path.c_str(), "rb")), path_(path) {
        if (!f_) throw IoError("cannot open " + path + ": " + std::strerror(errno));
        std::fseek(f_, 0, SEEK_END);
        size_ = static_cast<uint64_t>(std::ftell(f_));
        std::fseek(f_, 0, SEEK_SET);
    }
    ~Reader() {
        if (f_) std::fclose(f_);
    }
    uint64_t left() const { return size_ - pos_; }
    void bytes(void* p, size_t n) {
        if (n > left() || (n && std::fread(p, 1, n, f_) != n)) throw IoError("failed to fill whole buffer");
        pos_ += n;
    }
    uint64_t u64() {
        uint64_t v;
        bytes(&v, 8);
        return v;
    }
    float f32() {
        float v;
        bytes(&v, 4);
        return v;
    }
    template <class T, class V = std::vector<T>>
    V pod() {
        uint64_t n = u64();
        // a length the rest of the file cannot hold is a truncated or corrupt file
        if (n > left() / sizeof(T)) throw IoError("failed to fill whole buffer");
        V v(n);
        bytes(v.data(), n * sizeof(T));
        return v;
    }

private:
    std::FILE* f_;
    std::string path_;
    uint64_t size_ = 0, pos_ = 0;
};

uint64_t scan_mode_code(ScanMode m) { return m == ScanMode::F32 ? 0 : m == ScanMode::I8 ? 1 : 2; }

}  // namespace

void FlatCellIndex::save(const std::string& path) const {  // src/persist.rs:80-142
    Writer w(path);
    w.bytes(kMagic, 8);
    const uint64_t hdr[16] = {
        dim_, scan_mode_code(scan_mode_), rerank_factor_, dim_pad_, n_words_, seed_, n_live_, max_assign_,
        shortlist_mult_, i8_rerank_, keep_f32_, adaptive_, two_stage_, tree_route_, tree_min_cells_, tree_fanout_,
    };
    for (uint64_t v : hdr) w.u64(v);
    w.f32(quant_scale_);
    w.f32(spill_margin_);
    w.f32(at_margin_);
    w.f32(tree_beam_frac_);
    w.pod(bits_);
    w.pod(scan_i8_);
    w.pod(std::vector<uint16_t>{});  // rr_f16: this library keeps no f16 rerank store
    w.pod(sq_min_);
    w.pod(sq_step_);
    w.pod(vecs_f32_);
    w.pod(ext_ids_);
    w.pod(slot_cell_);
    w.pod(free_slots_);
    w.pod(slot_cells_);
    w.pod(tags_);
    w.u64(cells_.size());
    for (const Cell& c : cells_) {
        w.pod(c.members);
        w.pod(c.sum);
        w.pod(c.centroid);
        w.f32(c.r_bound);
        w.f32(c.r_max);
    }
    w.bytes(kTrailerMagic, 8);
    w.u64(kTrailerFields);
    uint32_t lam_bits;
    std::memcpy(&lam_bits, &spill_lambda_, 4);
    const uint64_t ext[kTrailerFields] = {fastscan_, compacted_, centroid_sq8_, graph_route_, graph_min_cells_,
                                          asym_cascade_, par_scan_, lam_bits, 0};
    for (uint64_t v : ext) w.u64(v);
    w.close();
}

void FlatCellIndex::load_file(const std::string& path) {  // src/persist.rs:145-281
    Reader r(path);
    char magic[8];
    if (r.left() < 8) throw IoError("failed to fill whole buffer");
    r.bytes(magic, 8);
    if (std::memcmp(magic, kMagic, 8) != 0)
        throw ValueError("not a MAIVS v2 index file (bad magic or format version)");
    uint64_t h[16];
    for (uint64_t& v : h) v = r.u64();
    const float quant_scale = r.f32(), spill_margin = r.f32(), at_margin = r.f32(), tree_beam_frac = r.f32();
    auto bits = r.pod<uint64_t, RowVec<uint64_t>>();
    auto scan_i8 = r.pod<int8_t, RowVec<int8_t>>();
    auto rr_f16 = r.pod<uint16_t>();
    auto sq_min = r.pod<float>();
    auto sq_step = r.pod<float>();
    auto vecs_f32 = r.pod<float, RowVec<float>>();
    auto ext_ids = r.pod<uint64_t>();
    auto slot_cell = r.pod<uint32_t>();
    auto free_slots = r.pod<uint32_t>();
    auto slot_cells = r.pod<uint32_t>();
    auto tags = r.pod<uint32_t>();
    const uint64_t ncell = r.u64();
    if (ncell > r.left() / 32) throw IoError("failed to fill whole buffer");
    std::vector<Cell> cells(ncell);
    for (Cell& c : cells) {
        c.members = r.pod<uint32_t>();
        c.sum = r.pod<float>();
        c.centroid = r.pod<float>();
        c.r_bound = r.f32();
        c.r_max = r.f32();
    }
    // optional extension trailer (absent in files the reference wrote)
    std::vector<uint64_t> ext;
    if (r.left() >= 16) {
        char tm[8];
        r.bytes(tm, 8);
        if (std::memcmp(tm, kTrailerMagic, 8) == 0) {
            uint64_t nf = r.u64();
            if (nf > r.left() / 8) throw IoError("failed to fill whole buffer");
            ext.resize(nf);
            for (uint64_t& v : ext) v = r.u64();
        }
    }
    if (!rr_f16.empty()) throw Unsupported("the index file holds an f16 rerank store, which this library does not keep");

    // The reference trusts the file; the arena is uploaded to the GPU, so the sizes are checked.
    const uint64_t dim = h[0], dim_pad = h[3], nw = h[4], ma = h[7];
    const size_t n = ext_ids.size();
    auto corrupt = [](const char* what) { throw ValueError(std::string("corrupt index file: ") + what); };
    if (dim == 0 || dim_pad < dim || dim_pad > (1u << 20) || (dim_pad & (dim_pad - 1)) != 0) corrupt("dimensions");
    if (ma == 0 || ma > 64) corrupt("max_assign");
    if (nw * 64 > dim_pad) corrupt("code words");
    if (!bits.empty() && bits.size() != n * nw) corrupt("code array size");
    if (slot_cell.size() != n || slot_cells.size() != n * ma) corrupt("slot arrays");
    if (!vecs_f32.empty() && vecs_f32.size() != n * dim) corrupt("f32 rows");
    if (!scan_i8.empty() && scan_i8.size() != n * dim) corrupt("int8 rows");
    if (!sq_min.empty() && (sq_min.size() != dim || sq_step.size() != dim)) corrupt("SQ8 ranges");
    if (!tags.empty() && tags.size() > n) corrupt("tags");
    for (uint32_t s : free_slots)
        if (s >= n) corrupt("free slot");
    for (size_t s = 0; s < n; ++s) {
        if (slot_cell[s] >= ncell) corrupt("slot cell");
        for (size_t j = 0; j < ma; ++j)
            if (slot_cells[s * ma + j] != UINT32_MAX && slot_cells[s * ma + j] >= ncell) corrupt("slot homes");
    }
    for (const Cell& c : cells) {
        if (c.centroid.size() != dim || (!c.sum.empty() && c.sum.size() != dim)) corrupt("cell vectors");
        for (uint32_t m : c.members)
            if (m >= n) corrupt("cell member");
    }

    // the new state, as src/persist.rs:201-279 sets it
    dim_ = dim;
    scan_mode_ = h[1] == 0 ? ScanMode::F32 : h[1] == 1 ? ScanMode::I8 : ScanMode::Binary;
    rerank_factor_ = h[2];
    dim_pad_ = dim_pad;
    n_words_ = nw;
    seed_ = h[5];
    rot_signs_ = make_signs(dim_pad_, seed_);
    bits_.swap(bits);
    scan_i8_.swap(scan_i8);
    vecs_f32_.swap(vecs_f32);
    ext_ids_.swap(ext_ids);
    slot_cell_.swap(slot_cell);
    free_slots_.swap(free_slots);
    slot_cells_.swap(slot_cells);
    tags_.swap(tags);
    cells_.swap(cells);
    std::unordered_set<uint32_t> free(free_slots_.begin(), free_slots_.end());
    id_to_slot_.clear();
    id_to_slot_.reserve(ext_ids_.size());
    for (size_t s = 0; s < ext_ids_.size(); ++s)
        if (!free.count(static_cast<uint32_t>(s))) id_to_slot_.set(ext_ids_[s], static_cast<uint32_t>(s));
    cent_bits_.clear();
    cent_sq8_.clear();
    csq_min_.clear();
    csq_step_.clear();
    graph_route_ = true;
    graph_min_cells_ = 65536;
    graph_built_ = false;  // a load builds no centroid graph (src/persist.rs:228)
    store_ok_ = false;     // the loaded rows are not in the GPU session's row store
    tag_filter_.reset();
    tree_.reset();
    tree_route_ = h[13] != 0;
    tree_min_cells_ = h[14];
    tree_fanout_ = h[15];
    tree_beam_frac_ = tree_beam_frac;
    tree_cells_ = 0;
    par_scan_ = false;
    two_stage_ = h[12] != 0;
    centroid_sq8_ = true;
    shortlist_mult_ = h[8];
    quant_scale_ = quant_scale;
    n_live_ = h[6];
    max_assign_ = ma;
    spill_margin_ = spill_margin;
    spill_lambda_ = 0.0f;
    compacted_ = false;
    asym_cascade_ = 0;
    fastscan_ = false;
    fs_codes_.clear();
    fs_off_.clear();
    prim_len_.clear();
    rep_off_.clear();
    i8_rerank_ = h[9] != 0;
    f16_rerank_ = false;
    per_dim_sq_ = !sq_min.empty();
    sq_min_.swap(sq_min);
    sq_step_.swap(sq_step);
    keep_f32_ = h[10] != 0;
    adaptive_ = h[11] != 0;
    at_margin_ = at_margin;
    mem_off_.clear();
    members_flat_.clear();
    // an attached GPU session re-uploads: the generation below changes

    bool compacted = false;
    if (ext.size() >= 8) {
        fastscan_ = ext[0] != 0;
        compacted = ext[1] != 0;
        centroid_sq8_ = ext[2] != 0;
        graph_route_ = ext[3] != 0;
        graph_min_cells_ = ext[4];
        asym_cascade_ = ext[5];
        par_scan_ = ext[6] != 0;
        const uint32_t lam_bits = static_cast<uint32_t>(ext[7]);
        std::memcpy(&spill_lambda_, &lam_bits, 4);
        if (!std::isfinite(spill_lambda_) || spill_lambda_ < 0.0f) corrupt("spill_lambda");
    }
    // finish_load (src/index.rs:1116-1124)
    if (two_stage_) rebuild_centroid_codes();
    if (centroid_sq8_) rebuild_centroid_sq8();
    rebuild_centroid_tree();
    ++generation_;
    if (compacted) compact_arena();
}

}  // namespace maivs
