// Python module maivs_amd._maivs: the FlatCellIndex class with the reference's Python
// signatures (src/index.rs:2670-3603, pyo3) so callers of `maivs.FlatCellIndex` switch by import.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <atomic>
#include <cstring>
#include <type_traits>

#include "index.h"

namespace py = pybind11;
using maivs::FlatCellIndex;

namespace {

struct BorrowError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// A float32 (n, d) C-contiguous view, with the reference's error messages.
struct F32Rows {
    const float* ptr;
    size_t rows, cols;
};

F32Rows as_rows(const py::array& a, const char* what, const char* contig_msg) {
    if (!py::dtype::of<float>().is(a.dtype()))
        throw py::type_error(std::string(what) + " must be a float32 array, got dtype " +
                             py::str(a.dtype()).cast<std::string>());
    if (a.ndim() != 2) throw py::value_error(std::string(what) + " must be 2-dimensional");
    if (!(a.flags() & py::array::c_style)) throw py::value_error(contig_msg);
    return {static_cast<const float*>(a.data()), static_cast<size_t>(a.shape(0)), static_cast<size_t>(a.shape(1))};
}

// Flat Python lists of the results, as the reference returns them: one allocation for the list and
// one object per entry (the C API directly, without the generic caster's per-element checks).
py::list ids_list(const std::vector<uint64_t>& v) {
    PyObject* l = PyList_New(static_cast<Py_ssize_t>(v.size()));
    if (!l) throw py::error_already_set();
    for (size_t i = 0; i < v.size(); ++i) {
        PyObject* o = PyLong_FromUnsignedLongLong(v[i]);
        if (!o) {
            Py_DECREF(l);
            throw py::error_already_set();
        }
        PyList_SET_ITEM(l, static_cast<Py_ssize_t>(i), o);
    }
    return py::reinterpret_steal<py::list>(l);
}
py::list scores_list(const std::vector<float>& v) {
    PyObject* l = PyList_New(static_cast<Py_ssize_t>(v.size()));
    if (!l) throw py::error_already_set();
    for (size_t i = 0; i < v.size(); ++i) {
        PyObject* o = PyFloat_FromDouble(static_cast<double>(v[i]));
        if (!o) {
            Py_DECREF(l);
            throw py::error_already_set();
        }
        PyList_SET_ITEM(l, static_cast<Py_ssize_t>(i), o);
    }
    return py::reinterpret_steal<py::list>(l);
}

// Index errors cross into Python through a registered translator (it runs with the GIL held,
// so C++ code may throw them from regions that released the GIL).
template <class F>
auto translate(F&& f) -> decltype(f()) {
    return f();
}

py::dict stats_dict(const maivs_gpu_stats& s) {
    py::dict d;
    d["ms_total"] = s.ms_total;
    d["ms_prep"] = s.ms_prep;
    d["ms_route"] = s.ms_route;
    d["ms_seed"] = s.ms_seed;
    d["ms_invert"] = s.ms_invert;
    d["ms_scan"] = s.ms_scan;
    d["ms_select"] = s.ms_select;
    d["ms_rerank"] = s.ms_rerank;
    d["scan_pairs"] = s.scan_pairs;
    d["scan_blocks"] = s.scan_blocks;
    d["seed_blocks"] = s.seed_blocks;
    d["survivors"] = s.survivors;
    d["rerank_rows"] = s.rerank_rows;
    d["host_checks"] = s.host_checks;
    d["host_fixes"] = s.host_fixes;
    d["reruns"] = s.reruns;
    return d;
}

struct PyIndex {
    FlatCellIndex ix;
    maivs_gpu_stats last{};
    // pyo3's borrow flag (src/concurrent.rs:3-5): > 0 shared borrows (searches), -1 one exclusive
    // borrow (a mutation). Methods release the GIL, so two calls can overlap; a conflicting one
    // raises as the reference's does instead of racing.
    std::atomic<int> borrow{0};
    PyIndex(size_t dim, const std::string& mode, size_t rf, uint64_t seed, size_t code_bits)
        : ix(dim, mode, rf, seed, code_bits) {}
};

// A shared borrow (&self): fails while a mutation runs, with pyo3's PyBorrowError message.
struct Ref {
    std::atomic<int>& f;
    explicit Ref(PyIndex& s) : f(s.borrow) {
        int v = f.load();
        do {
            if (v < 0) throw BorrowError("Already mutably borrowed");
        } while (!f.compare_exchange_weak(v, v + 1));
    }
    ~Ref() { f.fetch_sub(1); }
};

// An exclusive borrow (&mut self): fails while any other call holds the index, with pyo3's
// PyBorrowMutError message.
struct Mut {
    std::atomic<int>& f;
    explicit Mut(PyIndex& s) : f(s.borrow) {
        int v = 0;
        if (!f.compare_exchange_strong(v, -1)) throw BorrowError("Already borrowed");
    }
    ~Mut() { f.store(0); }
};

}  // namespace

PYBIND11_MODULE(_maivs, m) {
    m.doc() = "MI355X-native batched cell-major search behind the MAIVS FlatCellIndex API";
    py::register_exception_translator([](std::exception_ptr p) {
        try {
            if (p) std::rethrow_exception(p);
        } catch (const maivs::ValueError& e) {
            PyErr_SetString(PyExc_ValueError, e.what());
        } catch (const maivs::Unsupported& e) {
            PyErr_SetString(PyExc_NotImplementedError, e.what());
        } catch (const maivs::IoError& e) {
            PyErr_SetString(PyExc_OSError, e.what());
        } catch (const BorrowError& e) {
            PyErr_SetString(PyExc_RuntimeError, e.what());
        }
    });

    py::class_<PyIndex>(m, "FlatCellIndex")
        .def(py::init([](size_t dim, const std::string& scan_mode, size_t rerank_factor, uint64_t seed,
                         size_t code_bits) {
                 return translate([&] { return new PyIndex(dim, scan_mode, rerank_factor, seed, code_bits); });
             }),
             py::arg("dim"), py::arg("scan_mode") = "f32", py::arg("rerank_factor") = 4,
             py::arg("seed") = 0x5EEDull, py::arg("code_bits") = 0)
        .def(
            "train_centroids",
            [](PyIndex& s, const py::array& vectors, size_t n_cells, size_t sample, uint64_t seed) { Mut _b(s); 
                F32Rows r = as_rows(vectors, "vectors", "vectors must be C-contiguous");
                if (r.cols != s.ix.dim()) throw py::value_error("dim mismatch");
                py::gil_scoped_release nogil;
                translate([&] { s.ix.train_centroids(r.ptr, r.rows, n_cells, sample, seed); });
            },
            py::arg("vectors"), py::arg("n_cells"), py::arg("sample") = 262144, py::arg("seed") = 0x5EEDull)
        .def("set_centroids",
             [](PyIndex& s, const py::array& c) { Mut _b(s); 
                 F32Rows r = as_rows(c, "centroids", "centroids must be C-contiguous");
                 if (r.cols != s.ix.dim()) throw py::value_error("centroid dim mismatch");
                 translate([&] { s.ix.set_centroids(r.ptr, r.rows); });
             })
        .def("set_i8_rerank", [](PyIndex& s, bool on) { Mut _b(s);  s.ix.set_i8_rerank(on); })
        .def(
            "set_tree_route",
            [](PyIndex& s, bool on, size_t min_cells, size_t fanout, float beam_frac) { Mut _b(s); 
                py::gil_scoped_release nogil;
                s.ix.set_tree_route(on, min_cells, fanout, beam_frac);
            },
            py::arg("on"), py::arg("min_cells") = 0, py::arg("fanout") = 0, py::arg("beam_frac") = 0.0f)
        .def(
            "set_graph_route", [](PyIndex& s, bool on, size_t min_cells) { Mut _b(s);  s.ix.set_graph_route(on, min_cells); },
            py::arg("on"), py::arg("min_cells") = 0)
        .def("set_centroid_sq8", [](PyIndex& s, bool on) { Mut _b(s);  s.ix.set_centroid_sq8(on); })
        .def("set_two_stage", [](PyIndex& s, bool on, size_t mult) { Mut _b(s);  s.ix.set_two_stage(on, mult); })
        .def("set_adaptive", [](PyIndex& s, bool on, float margin) { Mut _b(s);  s.ix.set_adaptive(on, margin); })
        .def("set_per_dim_sq", [](PyIndex& s, bool on) { Mut _b(s);  s.ix.set_per_dim_sq(on); })
        .def("set_f16_rerank", [](PyIndex& s, bool on) { Mut _b(s);  translate([&] { s.ix.set_f16_rerank(on); }); })
        .def("set_quant_scale", [](PyIndex& s, float v) { Mut _b(s);  s.ix.set_quant_scale(v); })
        .def("set_rerank_factor", [](PyIndex& s, size_t rf) { Mut _b(s);  s.ix.set_rerank_factor(rf); })
        .def("set_asym_cascade", [](PyIndex& s, size_t f) { Mut _b(s);  s.ix.set_asym_cascade(f); })
        .def("set_fastscan", [](PyIndex& s, bool on) { Mut _b(s);  s.ix.set_fastscan(on); })
        .def("set_replication", [](PyIndex& s, size_t ma, float margin) { Mut _b(s);  s.ix.set_replication(ma, margin); })
        .def(
            "set_orthogonal_polysemy", [](PyIndex& s, size_t homes, float lam) { Mut _b(s);  s.ix.set_orthogonal_polysemy(homes, lam); },
            py::arg("homes") = 2, py::arg("lam") = 1.0f)
        .def("set_parallel_scan", [](PyIndex& s, bool on) { Mut _b(s);  s.ix.set_parallel_scan(on); })
        .def("set_tags",
             [](PyIndex& s, std::vector<uint64_t> ids, std::vector<uint32_t> tags) { Mut _b(s); 
                 translate([&] { s.ix.set_tags(ids, tags); });
             })
        .def(
            "set_filter",
            [](PyIndex& s, std::optional<uint32_t> lo, std::optional<uint32_t> hi) { Mut _b(s);  s.ix.set_filter(lo, hi); },
            py::arg("lo") = py::none(), py::arg("hi") = py::none())
        .def("rebuild_tree",
             [](PyIndex& s) { Mut _b(s); 
                 py::gil_scoped_release nogil;
                 s.ix.rebuild_tree();
             })
        .def("add_batch",
             [](PyIndex& s, std::vector<uint64_t> ids, const py::array& vectors) { Mut _b(s); 
                 F32Rows r = as_rows(vectors, "vectors", "vectors must be C-contiguous (use np.ascontiguousarray)");
                 if (r.rows != ids.size() || r.cols != s.ix.dim()) throw py::value_error("shape mismatch");
                 py::gil_scoped_release nogil;
                 translate([&] { s.ix.add_batch(ids, r.ptr, r.rows); });
             })
        .def("remove", [](PyIndex& s, uint64_t id) { Mut _b(s);  return s.ix.remove(id); })
        .def("compact",
             [](PyIndex& s) { Mut _b(s); 
                 py::gil_scoped_release nogil;
                 s.ix.compact();
             })
        .def(
            "search",
            [](PyIndex& s, const py::array& query, size_t k, size_t nprobe, float tc, float beta) -> py::tuple { Ref _b(s); 
                if (!py::dtype::of<float>().is(query.dtype())) throw py::type_error("query must be a float32 array");
                if (query.ndim() != 1) throw py::value_error("query must be 1-dimensional");
                if (static_cast<size_t>(query.shape(0)) != s.ix.dim()) throw py::value_error("query dim mismatch");
                // the reference copies the query element by element, so any stride is accepted
                py::array_t<float, py::array::c_style | py::array::forcecast> qc(query);
                std::vector<uint64_t> ids;
                std::vector<float> scores;
                {
                    py::gil_scoped_release nogil;
                    translate([&] { s.ix.search(qc.data(), k, nprobe, tc, beta, ids, scores); });
                }
                return py::make_tuple(ids_list(ids), scores_list(scores));
            },
            py::arg("query"), py::arg("k"), py::arg("nprobe") = 16, py::arg("target_confidence") = 0.95f,
            py::arg("beta") = 8.0f)
        .def(
            "search_batch",
            [](PyIndex& s, const py::array& queries, size_t k, size_t nprobe, float tc, float beta,
               bool cell_major) { Ref _b(s); 
                if (!py::dtype::of<float>().is(queries.dtype()))
                    throw py::type_error("queries must be a float32 array");
                if (queries.ndim() != 2) throw py::value_error("queries must be 2-dimensional");
                if (static_cast<size_t>(queries.shape(1)) != s.ix.dim()) throw py::value_error("query dim mismatch");
                if (!(queries.flags() & py::array::c_style))
                    throw py::value_error("queries must be C-contiguous (use np.ascontiguousarray)");
                size_t nq = static_cast<size_t>(queries.shape(0));
                const float* q = static_cast<const float*>(queries.data());
                std::vector<uint64_t> ids;
                std::vector<float> scores;
                {
                    py::gil_scoped_release nogil;
                    translate([&] { s.ix.search_batch(q, nq, k, nprobe, tc, beta, cell_major, ids, scores, &s.last); });
                }
                return py::make_tuple(ids_list(ids), scores_list(scores));
            },
            py::arg("queries"), py::arg("k"), py::arg("nprobe") = 16, py::arg("target_confidence") = 0.95f,
            py::arg("beta") = 8.0f, py::arg("cell_major") = true)
        .def(
            "save",
            [](PyIndex& s, const std::string& path) { Ref _b(s); 
                py::gil_scoped_release nogil;
                translate([&] { s.ix.save(path); });
            },
            py::arg("path"))
        .def_static(
            "load",
            [](const std::string& path) {
                auto p = std::make_unique<PyIndex>(1, "binary", 1, 0, 0);
                {
                    py::gil_scoped_release nogil;
                    translate([&] { p->ix.load_file(path); });
                }
                return p;
            },
            py::arg("path"))
        .def("stats", [](PyIndex& s) { Ref _b(s);  return s.ix.stats(); })
        .def("__len__", [](PyIndex& s) { Ref _b(s);  return s.ix.len(); })
        .def("recommend", [](PyIndex& s) { Ref _b(s);  return s.ix.recommend(); })
        // ---- not in the reference: hooks for the C-ABI tests and the benchmark ----
        .def("set_gpu_build", [](PyIndex& s, bool on) { Mut _b(s);  s.ix.set_gpu_build(on); },
             "Run the index build's k-means (train_centroids, the centroid tree) on the GPU; the "
             "result is bit-identical to the CPU build.")
        .def("_kmeans",
             [](PyIndex& s, const py::array& x, std::vector<uint32_t> rows, std::vector<std::vector<uint64_t>> jobs,
                bool gpu) { Ref _b(s); 
                 F32Rows r = as_rows(x, "x", "x must be C-contiguous");
                 std::vector<maivs::KMeansJob> js;
                 size_t total = 0;
                 for (auto& j : jobs) {
                     if (j.size() != 5) throw py::value_error("a job is (first, n, k, iters, seed)");
                     if (j[0] != total || j[1] == 0) throw py::value_error("jobs must tile the row list in order");
                     js.push_back(maivs::KMeansJob{j[0], j[1], j[2], j[3], j[4]});
                     total += j[1];
                 }
                 if (rows.empty() ? total > r.rows : rows.size() != total)
                     throw py::value_error("the row list must hold one row id per point of the jobs");
                 for (uint32_t v : rows)
                     if (v >= r.rows) throw py::value_error("row id past the end of x");
                 std::vector<uint32_t> assign;
                 std::vector<float> cents;
                 {
                     py::gil_scoped_release nogil;
                     translate([&] { s.ix.run_kmeans(r.ptr, r.rows, r.cols, rows.empty() ? nullptr : rows.data(), js, gpu, assign, cents); });
                 }
                 return py::make_tuple(py::cast(assign), py::array_t<float>(static_cast<py::ssize_t>(cents.size()), cents.data()));
             },
             py::arg("x"), py::arg("rows"), py::arg("jobs"), py::arg("gpu"),
             "One batch of k-means jobs (first, n, k, iters, seed) on the CPU or the GPU (test hook).")
        .def("last_search_stats", [](PyIndex& s) { Ref _b(s);  return stats_dict(s.last); },
             "Device timings and work counters of the last search_batch call.")
        .def("cellmajor_blocker", [](PyIndex& s, bool cell_major) { Ref _b(s);  return s.ix.cellmajor_blocker(cell_major); },
             py::arg("cell_major") = true)
        .def("perquery_blocker", [](PyIndex& s) { Ref _b(s);  return s.ix.perquery_blocker(); })
        .def("takes_cellmajor", [](PyIndex& s, size_t nq, bool cell_major) { Ref _b(s);  return s.ix.takes_cellmajor(nq, cell_major); },
             py::arg("nq"), py::arg("cell_major") = true,
             "Whether search_batch(nq queries) takes the batched cell-major path (the reference's cm_ok).")
        .def("set_batched_filter", [](PyIndex& s, bool on) { Mut _b(s);  s.ix.set_batched_filter(on); },
             "Filtered searches take the batched path too (not in the reference; off by default).")
        .def("_arena_desc",
             [](PyIndex& s) -> uintptr_t { Mut _b(s); 
                 const maivs_arena_desc* d = s.ix.arena_desc();
                 if (!d) throw py::value_error("index has no cells");
                 return reinterpret_cast<uintptr_t>(d);
             },
             "Address of the maivs_arena_desc of the arena (valid until the next mutation).")
        .def("_store_mirrors", [](PyIndex& s) { Ref _b(s); return s.ix.store_mirrors(); },
             "Whether the GPU session's row store holds this index's rows (a GPU build keeps it).")
        .def("_search_params",
             [](PyIndex& s, size_t k, size_t nprobe, float tc, float beta) { Ref _b(s); 
                 maivs_search_params p = s.ix.search_params(k, nprobe, tc, beta);
                 return py::bytes(reinterpret_cast<const char*>(&p), sizeof(p));
             },
             py::arg("k"), py::arg("nprobe"), py::arg("target_confidence") = 1.0f, py::arg("beta") = 8.0f,
             "The maivs_search_params struct search_batch would pass, as raw bytes.")
        .def("_ext_ids",
             [](PyIndex& s) { Ref _b(s); 
                 const auto& e = s.ix.ext_ids();
                 py::array_t<uint64_t> a(static_cast<py::ssize_t>(e.size()));
                 std::memcpy(a.mutable_data(), e.data(), e.size() * sizeof(uint64_t));
                 return a;
             })
        .def("_codes",
             [](PyIndex& s) { Ref _b(s); 
                 const auto& b = s.ix.bits();
                 py::array_t<uint64_t> a(static_cast<py::ssize_t>(b.size()));
                 std::memcpy(a.mutable_data(), b.data(), b.size() * sizeof(uint64_t));
                 return a;
             })
        .def("_arena_arrays",
             [](PyIndex& s) { Mut _b(s); 
                 const maivs_arena_desc* a = s.ix.arena_desc();
                 if (!a) throw py::value_error("index has no cells");
                 auto copy = [](const auto* p, size_t n) {
                     using T = std::remove_cv_t<std::remove_pointer_t<decltype(p)>>;
                     py::array_t<T> out(static_cast<py::ssize_t>(p ? n : 0));
                     if (p && n) std::memcpy(out.mutable_data(), p, n * sizeof(T));
                     return out;
                 };
                 const size_t M = a->n_cells, N = a->n_slots, d = a->dim, W = a->n_words;
                 const size_t E = a->mem_off[M], B = a->fs_off ? a->fs_off[M] : 0;
                 py::dict r;
                 r["dim"] = a->dim;
                 r["dim_pad"] = a->dim_pad;
                 r["n_words"] = a->n_words;
                 r["n_cells"] = a->n_cells;
                 r["n_slots"] = a->n_slots;
                 r["max_assign"] = a->max_assign;
                 r["rerank_mode"] = a->rerank_mode;
                 r["fs_codes"] = copy(a->fs_codes, B * W * 256);
                 r["fs_off"] = copy(a->fs_off, a->fs_off ? M + 1 : 0);
                 r["mem_off"] = copy(a->mem_off, M + 1);
                 r["members"] = copy(a->members, E);
                 r["slot_cells"] = copy(a->slot_cells, N * a->max_assign);
                 r["cent_bits"] = copy(a->cent_bits, M * W);
                 r["cent_sq8"] = copy(a->cent_sq8, M * d);
                 r["centroids"] = copy(a->centroids, M * d);
                 r["csq_min"] = copy(a->csq_min, d);
                 r["csq_step"] = copy(a->csq_step, d);
                 r["r_bound"] = copy(a->r_bound, M);
                 r["rot_signs"] = copy(a->rot_signs, 2 * static_cast<size_t>(a->dim_pad));
                 r["vecs_f32"] = copy(a->vecs_f32, N * d);
                 r["sq8_codes"] = copy(a->sq8_codes, N * d);
                 r["sq_min"] = copy(a->sq_min, d);
                 r["sq_step"] = copy(a->sq_step, d);
                 return r;
             },
             "Copies of the compacted arena arrays (for brute-force checks).")
        .def("_tree_arrays",
             [](PyIndex& s) -> py::object { Ref _b(s); 
                 maivs::TreeFlat f;
                 if (!s.ix.tree_flat(f)) return py::none();
                 auto arr = [](const auto& v) {
                     using T = typename std::decay_t<decltype(v)>::value_type;
                     py::array_t<T> a(static_cast<py::ssize_t>(v.size()));
                     if (!v.empty()) std::memcpy(a.mutable_data(), v.data(), v.size() * sizeof(T));
                     return a;
                 };
                 py::dict d;
                 d["level_n"] = arr(f.level_n);
                 d["level_codes"] = arr(f.level_codes);
                 d["child_start"] = arr(f.child_start);
                 d["child_len"] = arr(f.child_len);
                 d["leaf_codes"] = arr(f.leaf_codes);
                 d["leaf_cells"] = arr(f.leaf_cells);
                 d["beam_frac"] = f.beam_frac;
                 d["min_beam"] = f.min_beam;
                 return d;
             },
             "The centroid tree as flat arrays (None without a tree).")
        .def("_rot_signs", [](PyIndex& s) { Ref _b(s); 
            const auto& r = s.ix.rot_signs();
            py::array_t<float> a(static_cast<py::ssize_t>(r.size()));
            std::memcpy(a.mutable_data(), r.data(), r.size() * sizeof(float));
            return a;
        });
}
