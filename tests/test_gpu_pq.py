"""The per-query path on the GPU (maivs_gpu_search_queries, through the C ABI) against the
oracle's restatement of route_query + search_one + rerank_exact (src/index.rs:1168-1305,
1381-1864, 1309-1378): slots and score bits identical, query by query.
"""
import numpy as np
import pytest

import maivs_amd as M
import oracle
from maivs_amd import capi

from .test_oracle_pq import tree40k  # noqa: F401  (fixture)

pytestmark = pytest.mark.gpu


def _params(ix, k, nprobe, tc=1.0, beta=8.0):
    return capi.params_from_bytes(ix._search_params(k, nprobe, tc, beta))


@pytest.fixture(scope="module")
def ctx():
    c = capi.Context(0)
    yield c
    c.close()


def _compare(ctx, ix, queries, p, stats=None):
    ctx.upload(ix._arena_desc())
    slots, scores = ctx.search_queries(queries, p, stats)
    oslots, oscores = oracle.search_one(ix._arena_desc(), queries, p, nthreads=8)
    bad = [i for i in range(len(queries)) if not (np.array_equal(slots[i], oslots[i])
                                                   and scores[i].tobytes() == oscores[i].tobytes())]
    assert not bad, f"{len(bad)} queries differ, first {bad[:5]}"
    return slots, scores


@pytest.mark.parametrize("nprobe,rf", [(1, 8), (8, 8), (16, 32), (64, 16), (390, 4)])
def test_pq_quality_two_stage_matches_oracle(ctx, quality50k, mix50k, nprobe, rf):
    _, queries, _ = mix50k
    quality50k.set_rerank_factor(rf)
    try:
        _compare(ctx, quality50k, queries[:300], _params(quality50k, 10, nprobe))
    finally:
        quality50k.set_rerank_factor(32)


@pytest.mark.parametrize("nprobe", [8, 64])
def test_pq_pair_tables_match_oracle(ctx, quality50k, memory50k, tree40k, mix50k, nprobe):
    """Batches of at most 256 queries look up position pairs in the per-query scan (one 256-entry
    table per pair of positions, built from the query's FastScan table): bit-exact with the oracle
    for both presets and the tree route, for 200 queries and for one."""
    _, queries, _ = mix50k
    for ix in (quality50k, memory50k, tree40k):
        _compare(ctx, ix, queries[:200], _params(ix, 10, nprobe))
        _compare(ctx, ix, queries[200:201], _params(ix, 10, nprobe))


@pytest.mark.parametrize("nprobe,tc", [(16, 0.95), (64, 0.5)])
def test_pq_nucleus_matches_oracle(ctx, quality50k, mix50k, nprobe, tc):
    _, queries, _ = mix50k
    st = capi.GpuStats()
    _compare(ctx, quality50k, queries[:300], _params(quality50k, 10, nprobe, tc), st)


@pytest.mark.parametrize("nprobe", [8, 32])
def test_pq_memory_matches_oracle(ctx, memory50k, mix50k, nprobe):
    _, queries, _ = mix50k
    _compare(ctx, memory50k, queries[:300], _params(memory50k, 10, nprobe))


@pytest.mark.parametrize("nprobe", [4, 16, 64, 200])
def test_pq_tree_route_matches_oracle(ctx, tree40k, mix50k, nprobe):
    _, queries, _ = mix50k
    _compare(ctx, tree40k, queries[:300], _params(tree40k, 10, nprobe))


@pytest.mark.parametrize("t,nprobe", [(500, 16), (100, 64), (10, 128), (1, 312)])
def test_pq_churned_filtered_matches_oracle(ctx, churn50k, mix50k, t, nprobe):
    _, queries, _ = mix50k
    ix, tags, _ = churn50k
    ix.set_filter(0, t - 1)
    try:
        p = _params(ix, 10, nprobe)
        assert p.filter == 1
        _compare(ctx, ix, queries[:300], p)
        ids, _ = ix.search_batch(queries[:40], 10, nprobe, 1.0, 8.0, True)  # filtered: the per-query path
        got = [i for i in ids if i != 2 ** 64 - 1]
        assert got and all(tags[i] <= t - 1 for i in got)
    finally:
        ix.set_filter()


def test_pq_exhaustive_large_candidate_lists(ctx, quality50k, mix50k):
    """No adaptive stop, every cell, k * rf > N: the candidate lists exceed the on-chip staging."""
    _, queries, _ = mix50k
    ix = quality50k
    ix.set_adaptive(False, 0.02)
    ix.set_rerank_factor(5001)
    try:
        _compare(ctx, ix, queries[:12], _params(ix, 10, 390))
    finally:
        ix.set_adaptive(True, 0.02)
        ix.set_rerank_factor(32)


def test_pq_edge_cases(ctx, quality50k, mix50k):
    _, queries, _ = mix50k
    ix = quality50k
    ctx.upload(ix._arena_desc())
    slots, scores = ctx.search_queries(queries[:5], _params(ix, 10, 0))  # nprobe 0: nothing probed
    assert (slots == 0xFFFFFFFF).all() and np.isneginf(scores).all()
    _compare(ctx, ix, queries[:1], _params(ix, 1, 1))
    _compare(ctx, ix, queries[:7], _params(ix, 100, 3))  # fewer than k survivors: padded


def test_binding_search_and_small_batches(quality50k, tree40k, mix50k):
    """search() and search_batch below cm_ok's batch size take the per-query path."""
    _, queries, _ = mix50k
    for ix in (quality50k, tree40k):
        ext = ix._ext_ids()
        p = _params(ix, 10, 16, 0.95)
        oslots, oscores = oracle.search_one(ix._arena_desc(), queries[:3], p, nthreads=4)
        for i in range(3):
            ids, sc = ix.search(queries[i], 10, 16, 0.95, 8.0)
            want = [int(ext[s]) for s in oslots[i] if s != 0xFFFFFFFF]
            assert ids == want
            assert np.array_equal(np.array(sc, np.float32), oscores[i][: len(want)])
        assert not ix.takes_cellmajor(3, True)
        ids, sc = ix.search_batch(queries[:3], 10, 16, 0.95, 8.0, True)
        assert ids == [int(ext[s]) if s != 0xFFFFFFFF else 2 ** 64 - 1 for s in oslots.reshape(-1)]


@pytest.fixture(scope="module")
def tree2lvl(mix50k):
    """40k vectors, 600 cells and fanout 2: a two-level centroid tree (300 and 150 nodes)."""
    base, _, _ = mix50k
    x = np.ascontiguousarray(base[:40000])
    ix = M.preset(384, len(x))
    ix.set_tree_route(True, 256, 2)
    ix.train_centroids(x, 600)
    ix.add_batch(list(range(len(x))), x)
    ix.compact()
    assert len(ix._tree_arrays()["level_n"]) == 2
    return ix


@pytest.mark.parametrize("block_max_q", ["0", "1000000"])
def test_pq_tree_descent_kernels_match_oracle(monkeypatch, tree40k, tree2lvl, mix50k, block_max_q):
    """The tree descent one wave per query (MAIVS_GPU_PQ_TREE_BLOCK=0) and one workgroup per query:
    the same leaves, so slots and score bits identical to the oracle, for one- and two-level trees,
    300 queries and one."""
    _, queries, _ = mix50k
    monkeypatch.setenv("MAIVS_GPU_PQ_TREE_BLOCK", block_max_q)
    c = capi.Context(0)
    try:
        for ix in (tree40k, tree2lvl):
            for nprobe in (4, 40):
                _compare(c, ix, queries[:300], _params(ix, 10, nprobe))
                _compare(c, ix, queries[300:301], _params(ix, 10, nprobe))
    finally:
        c.close()
