"""Pins for the oracle's routing without two-stage routing (route_mode 1: route_query's tree or
every-live-cell branch, src/index.rs:1185-1206, 1260-1269, which search_batch_cellmajor falls back
to when route_batch returns None, :1873-1877, 2105-2124):

* every-live-cell routing: the probe list is the nprobe best exact centroid scores over all live
  cells (float64 brute force, ties within rounding exempt), and the nucleus count is the float64
  one wherever no cumulative mass sits within 1e-4 of target_confidence;
* when the lists cannot differ (every live cell probed, tc = 1: route_batch's shortlist then holds
  every live cell, and so do the tree's leaves when its beam covers the top level), the batched
  search routed either way is bit-identical;
* with few probes the batched search under route_mode 1 only returns vectors homed in the cells
  route_query chose, while route_batch chooses other cells for some of the same queries.
"""
import numpy as np
import pytest

import oracle
from maivs_amd import capi

from .test_oracle_pq import _cent_scores, tree40k  # noqa: F401  (fixture)


def _params(ix, k, nprobe, tc=1.0, beta=8.0, route_mode=None):
    p = capi.params_from_bytes(ix._search_params(k, nprobe, tc, beta))
    if route_mode is not None:
        p.route_mode = route_mode
    return p


def _live(arr):
    return arr["mem_off"][1:] > arr["mem_off"][:-1]


@pytest.mark.parametrize("nprobe,tc", [(16, 1.0), (1, 1.0), (64, 1.0), (16, 0.9), (40, 0.5)])
def test_route_query_every_live_cell_bruteforce(quality50k, mix50k, nprobe, tc):
    _, queries, _ = mix50k
    ix = quality50k
    assert ix._tree_arrays() is None
    arr = ix._arena_arrays()
    live = np.flatnonzero(_live(arr))
    p = _params(ix, 10, nprobe, tc, route_mode=1)
    qs = queries[:48]
    ch, cs, nch = oracle.route_query(ix._arena_desc(), qs, p, nthreads=4)
    checked = 0
    for i, q in enumerate(qs):
        sc = _cent_scores(arr, q)
        ranked = sorted(live.tolist(), key=lambda c: (-sc[c], c))[:nprobe]
        cap = len(ranked)
        got = [int(c) for c in ch[i, : nch[i]]]
        assert np.allclose(cs[i, : nch[i]], sc[got], atol=1e-5)
        # the ranked prefix, up to scores within rounding of each other
        for j, c in enumerate(got):
            if c != ranked[j]:
                assert abs(sc[c] - sc[ranked[j]]) <= 1e-5, (i, j)
        assert all(ch[i, nch[i]:] == np.uint32(0xFFFFFFFF))
        if tc >= 1.0:
            assert nch[i] == cap
            continue
        s = np.array([sc[c] for c in ranked])
        w = np.exp((s - s[0]) * 8.0)
        cum = np.cumsum(w / w.sum())
        if np.any(np.abs(cum - tc) < 1e-4):
            continue
        assert nch[i] == int(np.argmax(cum >= tc)) + 1, i
        checked += 1
    assert tc >= 1.0 or checked > len(qs) // 2


@pytest.mark.parametrize("use_tree", [False, True])
def test_batched_routing_agrees_when_every_live_cell_is_probed(quality50k, tree40k, mix50k, use_tree):
    _, queries, _ = mix50k
    ix = tree40k if use_tree else quality50k
    arr = ix._arena_arrays()
    n_live = int(_live(arr).sum())
    nprobe = arr["n_cells"]
    if use_tree:
        tree = ix._tree_arrays()
        assert len(tree["level_n"]) == 1 and len(tree["leaf_cells"]) == arr["n_cells"]
        assert np.ceil(nprobe * tree["beam_frac"]) >= tree["level_n"][0]  # the descent reaches every leaf
    qs = queries[:32]
    p0 = _params(ix, 10, nprobe, route_mode=0)
    p1 = _params(ix, 10, nprobe, route_mode=1)
    _, ch0, cs0, n0 = oracle.route_batch(ix._arena_desc(), qs, p0, arr["n_words"], nthreads=4)
    ch1, cs1, n1 = oracle.route_query(ix._arena_desc(), qs, p1, nthreads=4)
    assert np.all(n0 == n_live) and np.array_equal(n0, n1)
    assert np.array_equal(ch0, ch1) and np.array_equal(cs0.view(np.uint32), cs1.view(np.uint32))
    s0, sc0 = oracle.search_batch(ix._arena_desc(), qs, p0, nthreads=4)
    s1, sc1 = oracle.search_batch(ix._arena_desc(), qs, p1, nthreads=4)
    assert np.array_equal(s0, s1)
    assert np.array_equal(sc0.view(np.uint32), sc1.view(np.uint32))


@pytest.mark.parametrize("use_tree,nprobe", [(False, 4), (False, 12), (True, 4), (True, 12)])
def test_batched_route_mode_1_probes_route_query_cells(quality50k, tree40k, mix50k, use_tree, nprobe):
    _, queries, _ = mix50k
    ix = tree40k if use_tree else quality50k
    arr = ix._arena_arrays()
    ma = int(arr["max_assign"])
    homes = arr["slot_cells"].reshape(-1, ma)
    qs = queries[:64]
    p1 = _params(ix, 10, nprobe, route_mode=1)
    p0 = _params(ix, 10, nprobe, route_mode=0)
    ch1, _, n1 = oracle.route_query(ix._arena_desc(), qs, p1, nthreads=4)
    _, ch0, _, n0 = oracle.route_batch(ix._arena_desc(), qs, p0, arr["n_words"], nthreads=4)
    differ = 0
    slots, _ = oracle.search_batch(ix._arena_desc(), qs, p1, nthreads=4)
    for i in range(len(qs)):
        mine = set(ch1[i, : n1[i]].tolist())
        differ += mine != set(ch0[i, : n0[i]].tolist())
        for s in slots[i]:
            if s == np.uint32(0xFFFFFFFF):
                continue
            assert any(int(h) in mine for h in homes[s] if h != np.uint32(0xFFFFFFFF)), (i, int(s))
    assert differ > 0
