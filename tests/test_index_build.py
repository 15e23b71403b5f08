"""The host build path and the drop-in binding: arena invariants after compact()
(src/index.rs:929-1112), polysemy (tests/test_index.py:304-350 style), deletes
(src/index.rs:3223-3276), the Python API surface and its errors (src/index.rs:3316-3391),
and that the C-ABI library exports every entry point include/maivs_gpu.h declares.
"""
import ctypes
import os
import re

import numpy as np
import pytest

import maivs_amd as M
import oracle
from maivs_amd import capi, mixture

from .conftest import ROOT, small_clustered


def _check_arena(ix, expect_homes=2):
    a = ix._arena_arrays()
    mem_off, members, fs_off = a["mem_off"], a["members"], a["fs_off"]
    nw, ma = a["n_words"], a["max_assign"]
    codes = ix._codes().reshape(-1, nw)
    sc = a["slot_cells"].reshape(-1, ma)
    N = a["n_slots"]
    count = np.zeros(N, np.int64)
    for c in range(a["n_cells"]):
        mem = members[mem_off[c]: mem_off[c + 1]]
        count[mem] += 1
        prim = [s for s in mem if sc[s][0] == c]
        rep = [s for s in mem if sc[s][0] != c]
        # polysemic run: primaries ascending, then replicas ascending (src/index.rs:1043-1071)
        assert list(mem) == sorted(prim) + sorted(rep)
        assert len(set(mem.tolist())) == len(mem)
        for s in mem:
            assert c in sc[s]
        # FastScan blocks are the members' codes, 32 lanes per block (src/index.rs:1076-1110)
        assert fs_off[c + 1] - fs_off[c] == (len(mem) + 31) // 32
        for b in range(fs_off[c], fs_off[c + 1]):
            blk = a["fs_codes"][b * nw * 256:(b + 1) * nw * 256]
            lanes = mem[(b - fs_off[c]) * 32:(b - fs_off[c] + 1) * 32]
            assert np.array_equal(blk, oracle.fs_pack_block(codes[lanes], nw))
    homes = (sc != 0xFFFFFFFF).sum(axis=1)
    assert np.array_equal(count, homes)
    assert homes.min() >= 1 and homes.max() <= expect_homes
    # primaries are one contiguous ascending run per cell, cell-major (the compacted layout)
    prim_of = sc[:, 0]
    assert np.all(np.diff(prim_of.astype(np.int64)) >= 0)
    return a


def test_compacted_arena_invariants(quality50k):
    a = _check_arena(quality50k)
    st = quality50k.stats()
    assert st["n_cells"] == 390 and st["n_live"] == 50000
    assert a["rerank_mode"] == capi.RERANK_F32
    assert abs(st["replication_factor"] - 2.0) < 1e-9


def test_codes_are_rotated_signs(quality50k, mix50k):
    base, _, _ = mix50k
    ix = quality50k
    a = ix._arena_arrays()
    codes = ix._codes().reshape(-1, a["n_words"])
    ext = ix._ext_ids()
    for slot in range(0, len(ext), 997):
        v = base[ext[slot]]
        want = oracle.pack_signs(oracle.rotate(v, a["rot_signs"], a["dim_pad"]), a["n_words"])
        assert np.array_equal(codes[slot], want)
        assert np.array_equal(a["vecs_f32"].reshape(-1, a["dim"])[slot], v)


def test_memory_preset_sq8_rows(memory50k, mix50k):
    base, _, _ = mix50k
    a = memory50k._arena_arrays()
    assert a["rerank_mode"] == capi.RERANK_SQ8
    assert a["vecs_f32"].size == 0  # set_per_dim_sq drops the f32 arena (src/index.rs:2908-2915)
    ext = memory50k._ext_ids()
    codes = a["sq8_codes"].reshape(-1, a["dim"]).astype(np.float64)
    rec = codes * a["sq_step"] + a["sq_min"]
    v = base[ext]
    assert np.max(np.abs(rec - v)) <= float(a["sq_step"].max()) * 0.5 + 1e-6
    assert np.allclose(a["sq_min"], base.min(axis=0))


def test_centroid_routing_state(quality50k):
    a = quality50k._arena_arrays()
    M_, d = a["n_cells"], a["dim"]
    cent = a["centroids"].reshape(M_, d)
    live = np.diff(a["mem_off"]) > 0
    assert np.allclose(np.linalg.norm(cent[live], axis=1), 1.0, atol=1e-4)
    for c in range(0, M_, 37):
        want = oracle.pack_signs(oracle.rotate(cent[c], a["rot_signs"], a["dim_pad"]), a["n_words"])
        assert np.array_equal(a["cent_bits"].reshape(M_, -1)[c], want)
    sq = a["cent_sq8"].reshape(M_, d).astype(np.float64) * a["csq_step"] + a["csq_min"]
    assert np.max(np.abs(sq[live] - cent[live])) <= float(a["csq_step"].max()) * 0.5 + 1e-6
    assert np.all(a["r_bound"][live] >= 0) and np.all(a["r_bound"][live] <= np.pi)


def test_delete_and_recompact():
    x = small_clustered(3000, 64, 30, seed=1)
    ix = M.preset(64, len(x))
    ix.train_centroids(x, max(16, len(x) // 128))
    ix.add_batch(list(range(len(x))), x)
    ix.compact()
    assert ix.cellmajor_blocker(True) == ""
    gone = list(range(0, 3000, 7))
    for i in gone:
        assert ix.remove(i)
    assert not ix.remove(0)  # unknown id (src/index.rs:3224-3227)
    assert len(ix) == 3000 - len(gone)
    assert "not compacted" in ix.cellmajor_blocker(True)
    # re-inserting reuses freed slots first (src/index.rs:3077-3199)
    ix.add_batch([100000 + i for i in range(50)], x[:50].copy())
    ix.compact()
    a = _check_arena(ix)
    ext = ix._ext_ids()
    assert len(ext) == len(ix) == a["n_slots"]
    live = set(ext.tolist())
    assert not (live & set(gone))
    assert all(100000 + i in live for i in range(50))


def test_binding_errors_and_padding():
    ix = M.FlatCellIndex(64, "binary", 8)
    with pytest.raises(ValueError):
        M.FlatCellIndex(64, "bogus")
    q = np.zeros((4, 64), np.float32)
    # empty index: padded results, no device needed (src/index.rs:3337-3339)
    ids, scores = ix.search_batch(q, 5)
    assert ids == [2 ** 64 - 1] * 20 and all(s == -np.inf for s in scores)
    with pytest.raises(ValueError):
        ix.add_batch([1], np.zeros((1, 64), np.float32))  # no centroids yet
    x = small_clustered(600, 64, 10, seed=2)
    ix.train_centroids(x, 16)
    ix.add_batch(list(range(600)), x)
    with pytest.raises(ValueError):
        ix.search_batch(np.zeros((4, 32), np.float32), 5)  # dim mismatch
    with pytest.raises(ValueError):
        ix.search_batch(np.zeros((64, 4), np.float32).T, 5)  # not C-contiguous
    with pytest.raises(TypeError):
        ix.search_batch(np.zeros((4, 64), np.float64), 5)
    # not compacted, no FastScan: the per-query path's Hamming branch runs (src/index.rs:1694-1760),
    # routed over every live cell without two-stage routing (:1260-1269)
    assert ix.perquery_blocker() == ""
    p = np.frombuffer(ix._search_params(5, 8, 1.0, 1.0), np.uint32)
    assert p[-1] == 1  # route_mode 1: route_query's routing
    # a centroid graph exists once graph routing is on past min_cells live cells (src/index.rs:625-636);
    # the graph router is not implemented by this library, so a search it would route refuses
    ix.set_graph_route(True, 8)
    assert "graph" in ix.perquery_blocker()
    ix.set_graph_route(False, 0)
    assert ix.perquery_blocker() == ""
    ix.set_two_stage(True, 2)
    assert ix.perquery_blocker() == ""
    p = np.frombuffer(ix._search_params(5, 8, 1.0, 1.0), np.uint32)
    assert p[-1] == 0  # two-stage routing with centroid codes
    assert not ix.takes_cellmajor(64, True)
    ix.set_asym_cascade(4)
    assert "cascade" in ix.perquery_blocker()
    with pytest.raises(NotImplementedError):
        ix.search_batch(q, 5)
    ix.set_asym_cascade(0)
    with pytest.raises(NotImplementedError):
        ix.set_f16_rerank(True)
    with pytest.raises(ValueError):
        ix.set_tags([1, 2], [3])


def test_blockers_name_the_missing_piece(quality50k):
    ix = quality50k
    assert ix.cellmajor_blocker(True) == ""
    assert "per-query" in ix.cellmajor_blocker(False)
    # a tag filter no longer blocks the batched path: the predicate runs inside the scans
    ix.set_filter(0, 10)
    try:
        assert ix.cellmajor_blocker(True) == ""
    finally:
        ix.set_filter()
    assert ix.cellmajor_blocker(True) == ""


def test_filter_params_need_tags():
    """filtering = a filter is set and tags exist (src/index.rs:1430-1431); the range is inclusive,
    an omitted bound is open (src/index.rs:3553-3558)."""
    x = small_clustered(3000, 64)
    ix = M.build_preset(x, "quality")
    sp = lambda: capi.params_from_bytes(ix._search_params(10, 8, 1.0, 8.0))
    ix.set_filter(3, 7)
    assert sp().filter == 0  # no tags yet: inert
    ix.set_tags(list(range(3000)), [i % 10 for i in range(3000)])
    p = sp()
    assert (p.filter, p.tag_lo, p.tag_hi) == (1, 3, 7)
    ix.set_filter(None, 4)
    p = sp()
    assert (p.filter, p.tag_lo, p.tag_hi) == (1, 0, 4)
    ix.set_filter(5)
    p = sp()
    assert (p.filter, p.tag_lo, p.tag_hi) == (1, 5, 2 ** 32 - 1)
    ix.set_filter()
    assert sp().filter == 0


def test_recall_of_the_restated_path(quality50k, mix50k):
    """Cell-major results are exact-reranked neighbours: high recall, no duplicate ids,
    best first (tests/test_index.py:352-418 thresholds)."""
    _, queries, gt = mix50k
    ix = quality50k
    p = capi.params_from_bytes(ix._search_params(10, 16, 1.0, 8.0))
    slots, scores = oracle.search_batch(ix._arena_desc(), queries, p, nthreads=8)
    ext = ix._ext_ids()
    ids = ext[slots].astype(np.int64)
    assert mixture.recall_at(ids, gt) > 0.99
    for row, sc in zip(ids, scores):
        assert len(set(row.tolist())) == len(row)
        assert np.all(np.diff(sc) <= 0)


def test_header_entry_points_exported():
    """libmaivs_gpu.so exports every maivs_gpu_* function include/maivs_gpu.h declares (loads
    without a GPU; nothing is called)."""
    hdr = open(os.path.join(ROOT, "include", "maivs_gpu.h")).read()
    declared = set(re.findall(r"\b(maivs_gpu_\w+)\s*\(", hdr))
    assert declared == set(capi.SIGNATURES), declared ^ set(capi.SIGNATURES)
    lib = ctypes.CDLL(capi.LIB_PATH)
    for name in declared:
        assert hasattr(lib, name), name


def test_mixture_generator_is_deterministic():
    a1, q1 = mixture.workload("mix50k", n=2000, nq=50)
    a2, q2 = mixture.workload("mix50k", n=2000, nq=50)
    assert np.array_equal(a1, a2) and np.array_equal(q1, q2)
    assert np.allclose(np.linalg.norm(a1, axis=1), 1.0, atol=1e-5)
    b, s = mixture.workload("mix500k-shift", n=1000, nq=20)
    assert b.shape == (1000, 384) and s.shape == (20, 384)


def test_overlapping_calls_follow_the_borrow_rules():
    """A mutation that released the GIL holds the index exclusively: a search, a read or another
    mutation that overlaps it raises RuntimeError with pyo3's messages (src/concurrent.rs:3-5),
    and the index works again once the mutation ends. Runs on the CPU: add_batch of 200k vectors
    keeps the exclusive borrow for long enough to be seen from the main thread."""
    import threading

    x = small_clustered(200_000, 64, 50, seed=7)
    ix = M.FlatCellIndex(64, "binary", 8)
    ix.train_centroids(x[:20_000], 64)
    errs, done = [], threading.Event()

    def mutate():
        try:
            ix.add_batch(list(range(len(x))), x)
        except Exception as e:  # pragma: no cover - reported below
            errs.append(e)
        finally:
            done.set()

    t = threading.Thread(target=mutate)
    t.start()
    seen_read = seen_mut = None
    while not done.is_set() and (seen_read is None or seen_mut is None):
        try:
            len(ix)
        except RuntimeError as e:
            seen_read = str(e)
        try:
            ix.set_adaptive(True, 0.02)
        except RuntimeError as e:
            seen_mut = str(e)
    t.join()
    assert not errs, errs
    assert seen_read == "Already mutably borrowed"
    assert seen_mut == "Already borrowed"
    assert len(ix) == len(x)
    ix.set_adaptive(True, 0.02)  # free again


def test_id_map_through_churn():
    """The id -> slot map under repeated deletes and re-inserts of the same ids (erased entries
    reused, the table rebuilt by compact): every present id removes once, absent ids never, and
    the slots' ids stay a permutation of the live ids."""
    rs = np.random.RandomState(5)
    x = small_clustered(2000, 64, 10, seed=9)
    ix = M.FlatCellIndex(64, "binary", 8)
    ix.train_centroids(x, 16)
    ids = list(range(10**12, 10**12 + 2000))
    ix.add_batch(ids, x)
    live = set(ids)
    for rnd in range(6):
        gone = rs.choice(sorted(live), 400, replace=False).tolist()
        for i in gone:
            assert ix.remove(i)
            assert not ix.remove(i)
            live.discard(i)
        back = gone[: 200 + 20 * rnd]
        ix.add_batch(back, np.ascontiguousarray(x[: len(back)]))
        live.update(back)
        assert len(ix) == len(live)
        if rnd % 2:
            ix.compact()
            ext = ix._ext_ids()
            assert sorted(ext.tolist()) == sorted(live)
    assert not ix.remove(7)
    for i in sorted(live):
        assert ix.remove(i)
    assert len(ix) == 0
