"""The index build's k-means on the GPU (maivs_gpu_kmeans) against the CPU restatement of
kmeans_spherical (src/tree.rs:179-248): bit-identical assignments and centroids, and a whole
index built with set_gpu_build(True) identical, array for array, to the CPU build.

The CPU k-means itself is pinned by what k-means fixes (CPU tests below): every point sits in a
cluster whose centroid scores within rounding of its best; every non-empty centroid is the
normalised sum of its points; an empty cluster's centroid is one of the data points (the
reseeding pick); the first iteration starts from the strided points.
"""
import numpy as np
import pytest

import maivs_amd as M

from .conftest import small_clustered


def _jobs(sizes, ks, iters, seed=0x5EED):
    out, first = [], 0
    for j, (n, k) in enumerate(zip(sizes, ks)):
        it = iters[j] if isinstance(iters, (list, tuple)) else iters
        out.append((first, n, k, it, seed + 97 * j))
        first += n
    return out


def _kmeans(x, rows, jobs, gpu):
    ix = M.FlatCellIndex(x.shape[1], "binary", 4, 1, 0)
    a, c = ix._kmeans(np.ascontiguousarray(x, np.float32), list(rows), [list(map(int, j)) for j in jobs], gpu)
    return np.asarray(a, np.uint32), c.reshape(-1, x.shape[1])


def _degenerate(n=240, d=37, distinct=5, seed=4):
    """Few distinct points: most clusters empty after the first iteration (reseeding runs)."""
    rs = np.random.RandomState(seed)
    base = rs.standard_normal((distinct, d)).astype(np.float32)
    base /= np.linalg.norm(base, axis=1, keepdims=True)
    return base[rs.randint(0, distinct, n)]


# ---------------------------------------------------------------- CPU: what k-means fixes


@pytest.mark.parametrize("d", [64, 37])
def test_cpu_kmeans_invariants(d):
    x = small_clustered(3000, d, 30, seed=11)
    jobs = _jobs([3000], [24], 12)
    assign, cents = _kmeans(x, [], jobs, gpu=False)
    assert assign.shape == (3000,) and cents.shape == (24, d)
    # assignment: the chosen centroid scores within rounding of the best one (computed in f64)
    # against the centroids the last assignment used; rebuild those from the final centroids'
    # definition: each non-empty final centroid is the normalised sum of its points
    x64 = x.astype(np.float64)
    for j in range(24):
        mem = assign == j
        if mem.any():
            s = x[mem].sum(axis=0, dtype=np.float64)
            ref = s / np.linalg.norm(s)
            assert np.allclose(cents[j], ref, atol=2e-6), j
        else:  # reseeded: a data point
            assert (np.abs(x - cents[j]).max(axis=1) == 0).any(), j
    # every centroid is unit length (or a unit data point)
    assert np.allclose(np.linalg.norm(cents.astype(np.float64), axis=1), 1.0, atol=1e-5)
    # a second run from the same inputs is identical (no run-to-run order dependence)
    a2, c2 = _kmeans(x, [], jobs, gpu=False)
    assert np.array_equal(assign, a2) and np.array_equal(cents, c2)
    del x64


def test_cpu_kmeans_zero_iterations_is_the_strided_start():
    x = small_clustered(1000, 16, 8, seed=2)
    a, c = _kmeans(x, [], _jobs([1000], [7], 0), gpu=False)
    stride = 1000 // 7
    assert np.array_equal(c, x[[min(j * stride, 999) for j in range(7)]])
    assert not a.any()


def test_cpu_kmeans_assignment_is_the_argmax():
    x = small_clustered(2000, 48, 20, seed=5)
    # one iteration: the assignment is against the strided initial centroids
    a, _ = _kmeans(x, [], _jobs([2000], [16], 1), gpu=False)
    init = x[[min(j * (2000 // 16), 1999) for j in range(16)]].astype(np.float64)
    s = x.astype(np.float64) @ init.T
    best = s.max(axis=1)
    assert (s[np.arange(2000), a] >= best - 1e-6).all()
    clear = np.sort(s, axis=1)[:, -1] - np.sort(s, axis=1)[:, -2] > 1e-5
    assert np.array_equal(a[clear], s.argmax(axis=1)[clear])


def test_cpu_kmeans_reseeds_empty_clusters():
    x = _degenerate()
    a, c = _kmeans(x, [], _jobs([240], [20], 6), gpu=False)
    used = set(np.unique(a).tolist())
    assert len(used) <= 5
    for j in range(20):
        if j in used:  # the normalised sum of identical unit points: the point, within rounding
            assert np.abs(x[a == j][0] - c[j]).max() < 1e-6, j
        else:  # empty at the last assignment: reseeded with a data point, exactly
            assert (np.abs(x - c[j]).max(axis=1) == 0).any(), j


def test_kmeans_hook_checks_the_row_list():
    x = small_clustered(100, 8, 4, seed=1)
    with pytest.raises(ValueError, match="row list"):
        _kmeans(x, np.arange(50, dtype=np.uint32), _jobs([60], [4], 2), gpu=False)
    with pytest.raises(ValueError, match="row id"):
        _kmeans(x, np.full(60, 100, np.uint32), _jobs([60], [4], 2), gpu=False)


def test_gpu_build_flag_is_inert_on_cpu_state():
    ix = M.preset(32, 100)
    ix.set_gpu_build(False)
    x = small_clustered(500, 32, 4, seed=1)
    ix.train_centroids(x, 8)
    assert ix.stats()["n_cells"] == 8


# ---------------------------------------------------------------- GPU: bit-identical to the CPU

@pytest.mark.gpu
@pytest.mark.parametrize("d", [384, 37])
def test_gpu_kmeans_single_job_matches_cpu(d):
    x = small_clustered(5000, d, 40, seed=21)
    jobs = _jobs([5000], [63], 8)
    ac, cc = _kmeans(x, [], jobs, gpu=False)
    ag, cg = _kmeans(x, [], jobs, gpu=True)
    assert np.array_equal(ac, ag)
    assert cc.tobytes() == cg.tobytes()


@pytest.mark.gpu
def test_gpu_kmeans_batched_jobs_match_cpu():
    """The second k-means level: many jobs over row lists, different sizes, k and iterations."""
    x = small_clustered(6000, 64, 50, seed=8)
    rs = np.random.RandomState(3)
    sizes = [1000, 700, 1, 1300, 1500]
    rows = rs.permutation(6000)[:sum(sizes)].astype(np.uint32)
    ks = [12, 30, 1, 5, 64]
    jobs = _jobs(sizes, ks, [12, 3, 12, 0, 7])
    ac, cc = _kmeans(x, rows, jobs, gpu=False)
    ag, cg = _kmeans(x, rows, jobs, gpu=True)
    assert np.array_equal(ac, ag)
    assert cc.tobytes() == cg.tobytes()


@pytest.mark.gpu
def test_gpu_kmeans_reseeding_matches_cpu():
    x = _degenerate()
    jobs = _jobs([240], [20], 6)
    ac, cc = _kmeans(x, [], jobs, gpu=False)
    ag, cg = _kmeans(x, [], jobs, gpu=True)
    assert np.array_equal(ac, ag)
    assert cc.tobytes() == cg.tobytes()


@pytest.mark.gpu
def test_gpu_build_matches_cpu_build(mix50k):
    """train_centroids (two-level k-means) and a one-level centroid tree on the GPU, then
    add_batch + compact: the arena is identical to the CPU build's, array for array."""
    base, queries, _ = mix50k
    built = []
    for gpu in (False, True):
        ix = M.preset(384, len(base))
        ix.set_gpu_build(gpu)
        ix.set_tree_route(True, 256, 16)  # 390 cells -> a 25-node tree level, trained by k-means
        ix.train_centroids(base, len(base) // 128)
        ix.add_batch(list(range(len(base))), base)
        ix.compact()
        built.append(ix)
    assert built[1]._store_mirrors() and not built[0]._store_mirrors()
    _same_arena(*built)
    assert built[0].stats()["tree_depth"] == built[1].stats()["tree_depth"] >= 1
    q = np.ascontiguousarray(queries[:200])
    assert built[0].search_batch(q, 10, 16, 1.0, 8.0, True) == built[1].search_batch(q, 10, 16, 1.0, 8.0, True)


# ---------------------------------------------------------------- GPU placement (add_batch)


def _configure(ix, case):
    if case == "memory":
        ix.set_per_dim_sq(True)
    elif case == "replicate3":
        ix.set_replication(3, 0.02)
    elif case == "single":
        ix.set_replication(1, 0.0)
    elif case == "i8":
        ix.set_i8_rerank(True)


def _same_arena(a, b):
    """Two indexes' arena arrays (every array the upload reads, radii and FastScan blocks included)
    byte for byte."""
    x, y = a._arena_arrays(), b._arena_arrays()
    assert x.keys() == y.keys()
    for key in x:
        if isinstance(x[key], np.ndarray):
            assert x[key].tobytes() == y[key].tobytes(), key
        else:
            assert x[key] == y[key], key


def _pair(x, n_cells, case, tree_min=2048, churn=False):
    """Two identical indexes (CPU-trained centroids); one builds with the GPU (placement, sums,
    radii and compaction through its row store). Checks their arenas byte for byte and returns
    the saved files' bytes of both after add_batch (+ churn) + compact."""
    import os
    import tempfile
    out, built = [], []
    for gpu in (False, True):
        ix = M.preset(x.shape[1], len(x))
        _configure(ix, case)
        ix.set_tree_route(True, tree_min, 16)
        ix.train_centroids(x, n_cells)
        ix.set_gpu_build(gpu)
        n0 = len(x) if not churn else len(x) * 3 // 4
        ix.add_batch(list(range(n0)), np.ascontiguousarray(x[:n0]))
        if churn:
            for v in range(0, n0, 7):
                assert ix.remove(v)
            ix.add_batch(list(range(n0, len(x))), np.ascontiguousarray(x[n0:]))  # reuses free slots
        ix.compact()
        assert ix._store_mirrors() == gpu
        built.append(ix)
        with tempfile.TemporaryDirectory() as td:
            p = os.path.join(td, "ix.maivs")
            ix.save(p)
            out.append(open(p, "rb").read())
    _same_arena(*built)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["quality", "memory", "replicate3", "single", "i8"])
def test_gpu_placement_matches_cpu_without_tree(mix50k, case):
    base, _, _ = mix50k
    x = np.ascontiguousarray(base[:20000])
    a, b = _pair(x, 156, case)
    assert a == b


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["quality", "replicate3"])
def test_gpu_placement_matches_cpu_with_tree(mix50k, case):
    """312 cells with the tree threshold lowered: one 20-node level, beams of 32, 64 leaves."""
    base, _, _ = mix50k
    x = np.ascontiguousarray(base[:40000])
    a, b = _pair(x, 312, case, tree_min=256)
    assert a == b


@pytest.mark.gpu
def test_gpu_placement_odd_dim_and_churn():
    x = small_clustered(6000, 37, 40, seed=13)
    a, b = _pair(x, 46, "quality", churn=True)
    assert a == b


# ---------------------------------------------------------------- the row store (sums, radii, compaction)


@pytest.mark.gpu
@pytest.mark.parametrize("profile", ["quality", "memory"])
def test_gpu_build_500k_matches_cpu_build(profile):
    """The 500k mixture, both presets: the GPU build (k-means, placement, primary sums, radii, row
    moves and FastScan packing on the device) gives the CPU build's arena byte for byte, and its
    searches (uploaded from the row store) return the same ids and score bits."""
    from maivs_amd import mixture
    base, queries = mixture.workload("mix500k")
    built = [M.build_preset(base, profile, gpu_build=g) for g in (False, True)]
    assert built[1]._store_mirrors() and not built[0]._store_mirrors()
    _same_arena(*built)
    q = np.ascontiguousarray(queries[:300])
    assert built[0].search_batch(q, 10, 24, 1.0, 8.0, True) == built[1].search_batch(q, 10, 24, 1.0, 8.0, True)


@pytest.mark.gpu
def test_store_follows_removes_and_reuse_then_stops_at_a_cpu_write(mix50k):
    """The row store mirrors the index through GPU add_batch, remove (slots freed) and a second
    GPU add_batch reusing them; a CPU add_batch ends the mirror (the host steps run again), and
    every stage stays identical to an all-CPU build."""
    base, queries, _ = mix50k
    x = np.ascontiguousarray(base[:30000])
    built = []
    for gpu in (False, True):
        ix = M.preset(384, len(x))
        ix.set_tree_route(True, 256, 16)
        ix.train_centroids(x[:20000], 156)
        ix.set_gpu_build(gpu)
        ix.add_batch(list(range(20000)), np.ascontiguousarray(x[:20000]))
        for v in range(0, 20000, 5):
            assert ix.remove(v)
        ix.add_batch(list(range(20000, 25000)), np.ascontiguousarray(x[20000:25000]))
        assert ix._store_mirrors() == gpu
        ix.compact()
        assert ix._store_mirrors() == gpu
        built.append(ix)
    _same_arena(*built)
    q = np.ascontiguousarray(queries[:200])
    assert built[0].search_batch(q, 10, 16, 1.0, 8.0, True) == built[1].search_batch(q, 10, 16, 1.0, 8.0, True)
    for ix in built:
        ix.set_gpu_build(False)
        ix.add_batch(list(range(25000, 30000)), np.ascontiguousarray(x[25000:]))
        assert not ix._store_mirrors()
        ix.compact()
    _same_arena(*built)
    assert built[0].search_batch(q, 10, 16, 1.0, 8.0, True) == built[1].search_batch(q, 10, 16, 1.0, 8.0, True)
