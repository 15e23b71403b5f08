"""Routing without two-stage routing on the GPU (route_mode 1: route_query's tree or every-live-cell
branch, src/index.rs:1185-1206, 1260-1269; the batched search's fallback when route_batch returns
None, :1873-1877, 2105-2124), through the C ABI against the oracle: probe lists, slots and score
bits identical, for the batched path, the per-query path, the route entry point and the no-alloc
entry point, and end to end through the index with set_two_stage(False).
"""
import numpy as np
import pytest

import maivs_amd as M
import oracle
from maivs_amd import capi

from .test_oracle_pq import tree40k  # noqa: F401  (fixture)

pytestmark = pytest.mark.gpu


def _params(ix, k, nprobe, tc=1.0, beta=8.0, route_mode=1):
    p = capi.params_from_bytes(ix._search_params(k, nprobe, tc, beta))
    p.route_mode = route_mode
    return p


@pytest.fixture(scope="module")
def ctx():
    c = capi.Context(0)
    yield c
    c.close()


def _same(a_slots, a_scores, b_slots, b_scores):
    bad = [i for i in range(len(a_slots)) if not (np.array_equal(a_slots[i], b_slots[i])
                                                   and a_scores[i].tobytes() == b_scores[i].tobytes())]
    assert not bad, f"{len(bad)} queries differ, first {bad[:5]}"


@pytest.mark.parametrize("use_tree", [False, True])
@pytest.mark.parametrize("nprobe,tc", [(1, 1.0), (8, 1.0), (40, 1.0), (16, 0.9)])
def test_route_entry_matches_route_query(ctx, quality50k, tree40k, mix50k, use_tree, nprobe, tc):
    _, queries, _ = mix50k
    ix = tree40k if use_tree else quality50k
    ctx.upload(ix._arena_desc())
    p = _params(ix, 10, nprobe, tc)
    q = queries[:300]
    ch, cs, nch = ctx.route(q, p)
    och, ocs, onch = oracle.route_query(ix._arena_desc(), q, p, nthreads=8)
    assert np.array_equal(nch, onch)
    for i in range(len(q)):  # the probe list proper (the nucleus prefix)
        n = int(nch[i])
        assert np.array_equal(ch[i, :n], och[i, :n]), i
        assert cs[i, :n].tobytes() == ocs[i, :n].tobytes(), i


@pytest.mark.parametrize("use_tree", [False, True])
@pytest.mark.parametrize("nprobe,rf,tc", [(1, 8, 1.0), (8, 8, 1.0), (16, 32, 1.0), (40, 16, 1.0), (64, 8, 0.9),
                                          (312, 4, 1.0)])
def test_batched_route_mode_1_matches_oracle(ctx, quality50k, tree40k, mix50k, use_tree, nprobe, rf, tc):
    _, queries, _ = mix50k
    ix = tree40k if use_tree else quality50k
    ix.set_rerank_factor(rf)
    try:
        ctx.upload(ix._arena_desc())
        p = _params(ix, 10, nprobe, tc)
        q = queries[:500]
        slots, scores = ctx.search(q, p)
        oslots, oscores = oracle.search_batch(ix._arena_desc(), q, p, nthreads=8)
        _same(slots, scores, oslots, oscores)
    finally:
        ix.set_rerank_factor(32)


@pytest.mark.parametrize("fused", ["0", "1000000"])
@pytest.mark.parametrize("nprobe", [8, 64])
def test_per_query_every_live_cell_matches_oracle(monkeypatch, quality50k, memory50k, mix50k, nprobe, fused):
    """Separate prep / route launches and the fused prep + route (MAIVS_GPU_PQ_FRONT)."""
    _, queries, _ = mix50k
    monkeypatch.setenv("MAIVS_GPU_PQ_FRONT", fused)
    c = capi.Context(0)
    try:
        for ix in (quality50k, memory50k):
            c.upload(ix._arena_desc())
            p = _params(ix, 10, nprobe)
            for q in (queries[:200], queries[200:201]):
                slots, scores = c.search_queries(q, p)
                oslots, oscores = oracle.search_one(ix._arena_desc(), q, p, nthreads=8)
                _same(slots, scores, oslots, oscores)
    finally:
        c.close()


def test_noalloc_tree_route_matches_device_entry(tree40k, mix50k):
    import torch
    _, queries, _ = mix50k
    ix = tree40k
    c = capi.Context(0)
    try:
        c.upload(ix._arena_desc())
        for nq, nprobe in ((600, 24), (200, 8)):
            p = _params(ix, 10, nprobe)
            q = torch.from_numpy(np.ascontiguousarray(queries[:nq])).to("cuda:0")
            out = []
            for fn in (c.search_device, c.search_device_noalloc):
                s = torch.empty((nq, p.k), dtype=torch.int32, device="cuda:0")
                v = torch.empty((nq, p.k), dtype=torch.float32, device="cuda:0")
                torch.cuda.synchronize()
                fn(q.data_ptr(), nq, p, s.data_ptr(), v.data_ptr())
                out.append((s.cpu().numpy().view(np.uint32), v.cpu().numpy()))
            _same(*out[0], *out[1])
            o_s, o_v = oracle.search_batch(ix._arena_desc(), queries[:nq], p, 8)
            _same(*out[1], o_s, o_v)
    finally:
        c.close()


def test_index_without_two_stage_routing_end_to_end(mix50k):
    """The drop-in call: an index built with set_two_stage(False) routes every query over its live
    cells (search_batch_cellmajor -> route_query), on the GPU, identical to the oracle."""
    base, queries, _ = mix50k
    x = np.ascontiguousarray(base[:20000])
    ix = M.preset(384, len(x))
    ix.set_two_stage(False, 2)
    ix.train_centroids(x, 156)
    ix.add_batch(list(range(len(x))), x)
    ix.compact()
    assert ix.cellmajor_blocker(True) == ""
    desc = ix._arena_arrays()
    assert desc["cent_bits"] is None or len(desc["cent_bits"]) == 0
    p = _params(ix, 10, 16, route_mode=1)
    assert np.frombuffer(ix._search_params(10, 16, 1.0, 8.0), np.uint32)[-1] == 1
    ids, scores = ix.search_batch(queries[:256], 10, 16)
    oslots, oscores = oracle.search_batch(ix._arena_desc(), queries[:256], p, nthreads=8)
    ext = ix._ext_ids()
    want = [int(ext[s]) if s != 0xFFFFFFFF else 2 ** 64 - 1 for s in oslots.reshape(-1)]
    assert list(ids) == want
    assert np.asarray(scores, np.float32).tobytes() == oscores.reshape(-1).tobytes()
