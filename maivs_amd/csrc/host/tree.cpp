// Centroid k-means and tree, restated from src/tree.rs (see tree.h).
#include "tree.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>

#include "cpu_kernels.h"

namespace maivs {

namespace {

// normalise() of src/tree.rs:166-173: divide by the f32 norm when it exceeds 1e-12.
void normalize(float* v, size_t dim) {
    float n = -0.0f;
    for (size_t i = 0; i < dim; ++i) n += v[i] * v[i];
    n = std::sqrt(n);
    if (n > 1e-12f)
        for (size_t i = 0; i < dim; ++i) v[i] /= n;
}

// keep_smallest of src/tree.rs:120-159: keep the `keep` smallest Hamming distances in O(n),
// ties at the cut-off kept in encounter order.
void keep_smallest(std::vector<std::pair<uint32_t, uint32_t>>& v, size_t keep, std::vector<uint32_t>& hist,
                   size_t bits) {
    if (keep >= v.size()) return;
    if (hist.size() < bits + 1) hist.assign(bits + 1, 0);
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
        size_t h = e.first;
        if (h < t || (h == t && need_eq > 0)) {
            if (h == t) --need_eq;
            v[w++] = e;
        }
    }
    v.resize(w);
    std::fill(hist.begin(), hist.begin() + bits + 1, 0u);
}

}  // namespace

void kmeans_spherical(const float* x, size_t n, size_t dim, size_t k, size_t iters, uint64_t seed,
                      std::vector<uint32_t>& assign, std::vector<float>& cents, bool parallel) {
    k = std::min(std::max<size_t>(k, 1), n);
    cents.assign(k * dim, 0.0f);
    size_t stride = std::max<size_t>(n / k, 1);
    for (size_t j = 0; j < k; ++j) {
        size_t src = std::min(j * stride, n - 1);
        std::memcpy(&cents[j * dim], x + src * dim, dim * sizeof(float));
    }
    assign.assign(n, 0);
    uint64_t state = seed | 1;
    auto next_u = [&]() {
        state ^= state << 13;
        state ^= state >> 7;
        state ^= state << 17;
        return state;
    };
    std::vector<float> sums;
    std::vector<uint32_t> counts;
    for (size_t it = 0; it < iters; ++it) {
        auto assign_one = [&](size_t i) {
            const float* v = x + i * dim;
            uint32_t best = 0;
            float best_s = -INFINITY;
            for (size_t j = 0; j < k; ++j) {
                float s = dot_f32(v, &cents[j * dim], dim);
                if (s > best_s) {
                    best_s = s;
                    best = static_cast<uint32_t>(j);
                }
            }
            assign[i] = best;
        };
        if (parallel)
            parallel_for(n, assign_one, 256);
        else
            for (size_t i = 0; i < n; ++i) assign_one(i);
        sums.assign(k * dim, 0.0f);
        counts.assign(k, 0);
        for (size_t i = 0; i < n; ++i) {
            size_t j = assign[i];
            counts[j] += 1;
            const float* v = x + i * dim;
            float* s = &sums[j * dim];
            for (size_t d = 0; d < dim; ++d) s[d] += v[d];
        }
        for (size_t j = 0; j < k; ++j) {
            if (counts[j] == 0) {
                size_t src = static_cast<size_t>(next_u() % n);
                std::memcpy(&cents[j * dim], x + src * dim, dim * sizeof(float));
                continue;
            }
            std::memcpy(&cents[j * dim], &sums[j * dim], dim * sizeof(float));
            normalize(&cents[j * dim], dim);
        }
    }
}

void run_kmeans_cpu(const float* x, size_t n_rows, size_t dim, const uint32_t* rows, const std::vector<KMeansJob>& jobs,
                    std::vector<uint32_t>& assign, std::vector<float>& cents) {
    (void)n_rows;
    size_t np = 0, sk = 0;
    std::vector<size_t> coff(jobs.size());
    for (size_t j = 0; j < jobs.size(); ++j) {
        coff[j] = sk;
        np += jobs[j].n;
        sk += jobs[j].k;
    }
    assign.assign(np, 0);
    cents.assign(sk * dim, 0.0f);
    // one job: parallel inside it; several (the second level): parallel over jobs
    const bool single = jobs.size() == 1;
    auto one = [&](size_t j) {
        const KMeansJob& J = jobs[j];
        std::vector<float> buf;
        const float* xs = x + J.first * dim;
        if (rows) {
            buf.resize(J.n * dim);
            for (size_t r = 0; r < J.n; ++r)
                std::memcpy(&buf[r * dim], x + static_cast<size_t>(rows[J.first + r]) * dim, dim * sizeof(float));
            xs = buf.data();
        }
        std::vector<uint32_t> a;
        std::vector<float> cs;
        kmeans_spherical(xs, J.n, dim, J.k, J.iters, J.seed, a, cs, single);
        std::copy(a.begin(), a.end(), assign.begin() + J.first);
        std::copy(cs.begin(), cs.end(), cents.begin() + coff[j] * dim);
    };
    if (single)
        one(0);
    else
        parallel_for(jobs.size(), one);
}

std::vector<float> hierarchical_kmeans(const float* x, size_t n, size_t dim, size_t k, uint64_t seed,
                                       const KMeansRunner* runner) {
    k = std::min(std::max<size_t>(k, 1), n);
    std::vector<uint32_t> assign;
    std::vector<float> cents;
    auto run = [&](const uint32_t* rows, const std::vector<KMeansJob>& jobs) {
        if (runner)
            (*runner)(x, n, dim, rows, jobs, assign, cents);
        else
            run_kmeans_cpu(x, n, dim, rows, jobs, assign, cents);
    };
    if (k <= 64 || n <= k * 4) {
        run(nullptr, {KMeansJob{0, n, k, 12, seed}});
        return cents;
    }
    size_t k1 = static_cast<size_t>(std::ceil(std::sqrt(static_cast<double>(k))));
    run(nullptr, {KMeansJob{0, n, k1, 8, seed}});
    std::vector<std::vector<uint32_t>> groups(k1);
    for (size_t i = 0; i < n; ++i) groups[assign[i]].push_back(static_cast<uint32_t>(i));

    std::vector<size_t> subs(groups.size(), 0), offs(groups.size(), 0);
    size_t written = 0, before = 0;
    for (size_t g = 0; g < groups.size(); ++g) {
        const auto& idx = groups[g];
        size_t prev = before;
        before += idx.size();
        if (idx.empty() || written >= k) continue;
        size_t remaining_groups = k1 - g;
        double denom = static_cast<double>(std::max<size_t>(n - prev, 1));
        size_t want = static_cast<size_t>(
            std::round(static_cast<double>(k - written) * static_cast<double>(idx.size()) / denom));
        size_t sub = std::min(std::min(std::max<size_t>(want, 1), k - written), idx.size());
        if (remaining_groups == 1) sub = std::max<size_t>(std::min(k - written, idx.size()), 1);
        if (sub == 0) continue;
        subs[g] = std::min(sub, k - written);
        offs[g] = written;
        written += subs[g];
    }
    std::vector<float> out(k * dim, 0.0f);
    // the second level: one job per group with clusters, each over the group's points in order
    std::vector<uint32_t> rows;
    std::vector<KMeansJob> jobs;
    std::vector<size_t> job_group;
    for (size_t g = 0; g < groups.size(); ++g) {
        if (subs[g] == 0) continue;
        jobs.push_back(KMeansJob{rows.size(), groups[g].size(), subs[g], 12,
                                 seed ^ ((static_cast<uint64_t>(g) + 1) * 0x9E3779B9ull)});
        job_group.push_back(g);
        rows.insert(rows.end(), groups[g].begin(), groups[g].end());
    }
    if (!jobs.empty()) {
        run(rows.data(), jobs);
        size_t coff = 0;
        for (size_t j = 0; j < jobs.size(); ++j) {
            size_t g = job_group[j];
            std::memcpy(&out[offs[g] * dim], &cents[coff * dim], subs[g] * dim * sizeof(float));
            coff += jobs[j].k;
        }
    }
    size_t fill = 0;
    while (written < k) {
        size_t src = (fill * 7919) % n;
        std::memcpy(&out[written * dim], x + src * dim, dim * sizeof(float));
        ++written;
        ++fill;
    }
    return out;
}

bool CentroidTree::build(const float* cell_cents, const std::vector<uint32_t>& cell_ids, size_t dim,
                         const float* rot_signs, size_t dim_pad, size_t n_words, size_t fanout,
                         float beam_frac, const KMeansRunner* runner) {
    size_t m = cell_ids.size();
    if (m < 2 || n_words == 0) return false;
    fanout = std::max<size_t>(fanout, 2);
    std::vector<float> rot(dim_pad);
    std::vector<uint64_t> tmp(n_words);
    auto code = [&](const float* v) {
        rotate(v, dim, rot_signs, dim_pad, rot.data());
        pack_signs_trunc(rot.data(), dim_pad, tmp.data(), n_words);
    };
    leaf_codes_.clear();
    leaf_codes_.reserve(m * n_words);
    for (size_t i = 0; i < m; ++i) {
        code(cell_cents + i * dim);
        leaf_codes_.insert(leaf_codes_.end(), tmp.begin(), tmp.end());
    }
    std::vector<TreeLevel> rev;
    std::vector<float> cur(cell_cents, cell_cents + m * dim);
    size_t cur_n = m;
    while (cur_n > kTopMax) {
        size_t k = std::max<size_t>((cur_n + fanout - 1) / fanout, 1);
        if (k >= cur_n) break;
        std::vector<uint32_t> assign;
        std::vector<float> parents;
        const std::vector<KMeansJob> job{KMeansJob{0, cur_n, k, 10, 0x9E3779B97F4A7C15ull}};
        if (runner)
            (*runner)(cur.data(), cur_n, dim, nullptr, job, assign, parents);
        else
            run_kmeans_cpu(cur.data(), cur_n, dim, nullptr, job, assign, parents);
        TreeLevel lv;
        lv.n = k;
        lv.child_len.assign(k, 0);
        for (uint32_t a : assign) lv.child_len[a] += 1;
        lv.child_start.assign(k, 0);
        uint32_t acc = 0;
        for (size_t j = 0; j < k; ++j) {
            lv.child_start[j] = acc;
            acc += lv.child_len[j];
        }
        std::vector<uint32_t> fill = lv.child_start;
        lv.child_idx.assign(cur_n, 0);
        for (size_t i = 0; i < cur_n; ++i) lv.child_idx[fill[assign[i]]++] = static_cast<uint32_t>(i);
        lv.codes.reserve(k * n_words);
        for (size_t j = 0; j < k; ++j) {
            code(&parents[j * dim]);
            lv.codes.insert(lv.codes.end(), tmp.begin(), tmp.end());
        }
        lv.cents = parents;
        rev.push_back(std::move(lv));
        cur = std::move(parents);
        cur_n = k;
    }
    if (rev.empty()) {
        levels_.clear();
        return false;
    }
    std::reverse(rev.begin(), rev.end());
    dim_ = dim;
    n_words_ = n_words;
    fanout_ = fanout;
    beam_frac_ = beam_frac > 0.0f ? beam_frac : kDefaultBeamFrac;
    levels_ = std::move(rev);
    leaf_ids_ = cell_ids;
    n_leaf_ = m;
    compact_layout();
    return true;
}

// Renumber every level so a node's children are contiguous, src/tree.rs:462-527.
void CentroidTree::compact_layout() {
    size_t d = levels_.size();
    for (size_t i = 0; i < d; ++i) {
        std::vector<uint32_t> order = levels_[i].child_idx;
        if (i + 1 < d) {
            TreeLevel& l = levels_[i + 1];
            if (order.size() == l.n) {
                std::vector<float> cents(l.n * dim_);
                std::vector<uint64_t> codes(l.n * n_words_);
                std::vector<uint32_t> ns(l.n), nl(l.n), nidx;
                nidx.reserve(l.child_idx.size());
                uint32_t acc = 0;
                for (size_t np = 0; np < order.size(); ++np) {
                    size_t o = order[np];
                    std::memcpy(&cents[np * dim_], &l.cents[o * dim_], dim_ * sizeof(float));
                    std::memcpy(&codes[np * n_words_], &l.codes[o * n_words_], n_words_ * 8);
                    ns[np] = acc;
                    nl[np] = l.child_len[o];
                    acc += l.child_len[o];
                    nidx.insert(nidx.end(), l.child_idx.begin() + l.child_start[o],
                                l.child_idx.begin() + l.child_start[o] + l.child_len[o]);
                }
                l.cents = std::move(cents);
                l.codes = std::move(codes);
                l.child_start = std::move(ns);
                l.child_len = std::move(nl);
                l.child_idx = std::move(nidx);
            }
        } else {
            std::vector<uint64_t> codes(order.size() * n_words_);
            std::vector<uint32_t> ids(order.size());
            for (size_t np = 0; np < order.size(); ++np) {
                size_t o = order[np];
                std::memcpy(&codes[np * n_words_], &leaf_codes_[o * n_words_], n_words_ * 8);
                ids[np] = leaf_ids_[o];
            }
            leaf_codes_ = std::move(codes);
            leaf_ids_ = std::move(ids);
            n_leaf_ = order.size();
        }
        for (size_t j = 0; j < levels_[i].child_idx.size(); ++j) levels_[i].child_idx[j] = static_cast<uint32_t>(j);
    }
}

size_t CentroidTree::bytes() const {
    size_t b = leaf_codes_.size() * 8 + leaf_ids_.size() * 4;
    for (const auto& l : levels_)
        b += l.cents.size() * 4 + l.codes.size() * 8 +
             (l.child_start.size() + l.child_len.size() + l.child_idx.size()) * 4;
    return b;
}

void CentroidTree::export_flat(size_t want, TreeFlat& f) const {
    f = TreeFlat{};
    for (const auto& l : levels_) {
        f.level_n.push_back(static_cast<uint32_t>(l.n));
        f.level_codes.insert(f.level_codes.end(), l.codes.begin(), l.codes.end());
        f.child_start.insert(f.child_start.end(), l.child_start.begin(), l.child_start.end());
        f.child_len.insert(f.child_len.end(), l.child_len.begin(), l.child_len.end());
        // compact_layout made every child list contiguous: child_idx is the identity
        for (size_t j = 0; j < l.child_idx.size(); ++j)
            if (l.child_idx[j] != j) throw std::logic_error("centroid tree is not in its compacted layout");
    }
    for (size_t b : beams(want)) f.beams.push_back(static_cast<uint32_t>(b));
    f.beam_frac = beam_frac_;
    f.min_beam = static_cast<uint32_t>(kMinBeam);
    f.leaf_codes = leaf_codes_;
    f.leaf_cells = leaf_ids_;
}

// Beam per level, top-down from the leaves, src/tree.rs:559-570.
std::vector<size_t> CentroidTree::beams(size_t want) const {
    size_t d = levels_.size();
    std::vector<size_t> b(d, 0);
    size_t need = std::max<size_t>(want, 1);
    for (size_t ii = d; ii-- > 0;) {
        size_t raw = static_cast<size_t>(std::ceil(static_cast<float>(need) * beam_frac_));
        size_t bb = std::min(std::max(raw, kMinBeam), levels_[ii].n);
        b[ii] = bb;
        need = bb;
    }
    return b;
}

// Beam descent, src/tree.rs:574-628.
void CentroidTree::search(const uint64_t* q_bits, size_t want, TreeScratch& s, std::vector<uint32_t>& out) const {
    out.clear();
    if (levels_.empty()) return;
    size_t nw = n_words_, bits = nw * 64;
    std::vector<size_t> bm = beams(want);
    s.frontier.clear();
    for (uint32_t i = 0; i < levels_[0].n; ++i) s.frontier.push_back(i);
    for (size_t li = 0; li < levels_.size(); ++li) {
        const TreeLevel& lv = levels_[li];
        s.scored.clear();
        for (uint32_t node : s.frontier)
            s.scored.emplace_back(hamming(q_bits, &lv.codes[static_cast<size_t>(node) * nw], nw), node);
        size_t keep = std::min(bm[li], s.scored.size());
        if (keep == 0) return;
        keep_smallest(s.scored, keep, s.hist, bits);
        s.expand.clear();
        for (auto& e : s.scored) {
            uint32_t st = lv.child_start[e.second], ln = lv.child_len[e.second];
            s.expand.insert(s.expand.end(), lv.child_idx.begin() + st, lv.child_idx.begin() + st + ln);
        }
        std::swap(s.frontier, s.expand);
        if (li + 1 == levels_.size()) break;
    }
    s.scored.clear();
    for (uint32_t leaf : s.frontier)
        s.scored.emplace_back(hamming(q_bits, &leaf_codes_[static_cast<size_t>(leaf) * nw], nw), leaf);
    size_t keep = std::min(want, s.scored.size());
    if (keep == 0) return;
    keep_smallest(s.scored, keep, s.hist, bits);
    for (auto& e : s.scored) out.push_back(leaf_ids_[e.second]);
}

}  // namespace maivs
