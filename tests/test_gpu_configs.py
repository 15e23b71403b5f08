"""GPU parity at the full size of every benchmark workload, against the oracle on the same arena:

* 500k x 384, 4,096-component mixture, `quality` preset (3,906 cells), 1,000 queries;
* the same base with 1,000 shifted queries (20 degree Givens rotation + 0.15 noise), `memory` preset;
* 5.2M x 384, 16,384-component mixture, `quality` preset built on the GPU (40,625 cells: the
  query-tiled Hamming rows and the route from global rows), 1,000 of its 10,000 queries;
* 400k from the 500k mixture under 25% turnover (10 x (10k deletes + 10k inserts), compact()),
  tags in [0, 1000), filter tag < t for t in 500, 100, 10, 1, on the per-query path (what the
  reference runs with a filter) and on the batched path with the filter inside its scans.

Each comparison asserts equal slots, score bits, seed cut-offs tau, adaptive rest_end, the
tie-inclusive cut G, candidate counts and candidate sets (d, slot), work counters, and equal R@10
(src/index.rs:1999-2311; bench/fair/fairbench.py:98-123; bench/fair/churn.py:47-61;
bench/fair/filtered.py:28-33,83-85).
"""
import numpy as np
import pytest

import oracle
from maivs_amd import capi, mixture

from .test_gpu_parity import _compare_search, _params

pytestmark = [pytest.mark.gpu, pytest.mark.slow, pytest.mark.timeout(900)]


def _log(msg):
    print(f"[configs] {msg}", flush=True)


@pytest.fixture(scope="module")
def ctx():
    c = capi.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def mix500k():
    base, queries = mixture.workload("mix500k")
    _log(f"mix500k generated: {base.shape}")
    return base, queries


@pytest.fixture(scope="module")
def quality500k(mix500k):
    import maivs_amd as M
    base, queries = mix500k
    ix = M.build_preset(base, "quality")
    gt = mixture.exact_topk(base, queries, 10, device="cuda:0")
    _log(f"quality500k built: {int(ix.stats()['n_cells'])} cells")
    return ix, gt


@pytest.mark.parametrize("nprobe,rf", [(10, 8), (64, 16), (512, 32)])
def test_mix500k_quality(ctx, quality500k, mix500k, nprobe, rf):
    ix, gt = quality500k
    _, queries = mix500k
    ix.set_rerank_factor(rf)
    try:
        st = _compare_search(ctx, ix, queries, _params(ix, 10, nprobe), gt)
        _log(f"mix500k quality np{nprobe}/rf{rf}: bit-exact, {st.scan_pairs} rest (query, cell) pairs")
    finally:
        ix.set_rerank_factor(32)


def test_mix500k_shifted_memory(ctx, mix500k):
    """The memory preset on shifted queries: the recall plateau is the oracle's too."""
    import maivs_amd as M
    base, _ = mix500k
    _, queries = mixture.workload("mix500k-shift")
    ix = M.build_preset(base, "memory")
    gt = mixture.exact_topk(base, queries, 10, device="cuda:0")
    ext = ix._ext_ids()
    recalls = []
    for nprobe, rf in ((16, 8), (96, 16)):
        ix.set_rerank_factor(rf)
        p = _params(ix, 10, nprobe)
        _compare_search(ctx, ix, queries, p, gt)
        s, _ = oracle.search_batch(ix._arena_desc(), queries, p, 8)
        recalls.append(mixture.recall_at(np.where(s == 0xFFFFFFFF, -1, ext[np.minimum(s, len(ext) - 1)].astype(np.int64)), gt))
    _log(f"mix500k-shift memory: bit-exact; oracle R@10 {recalls}")


def test_mix5m_quality_gpu_build(ctx):
    """5.2M vectors, 40,625 cells; 1,000 of the 10,000 queries at nprobe 512, rerank_factor 32."""
    import maivs_amd as M
    base, queries = mixture.workload("mix5m")
    _log(f"mix5m generated: {base.shape}")
    ix = M.build_preset(base, "quality", gpu_build=True)
    st = ix.stats()
    assert int(st["n_cells"]) == 40_625
    _log(f"mix5m built on the GPU: {int(st['n_cells'])} cells, {int(st['member_entries'])} entries")
    ix.set_rerank_factor(32)
    q = np.ascontiguousarray(queries[:1000])
    s = _compare_search(ctx, ix, q, _params(ix, 10, 512))
    _log(f"mix5m np512/rf32: bit-exact on 1,000 queries, {s.scan_pairs} rest (query, cell) pairs")
    del ix, base


@pytest.fixture(scope="module")
def churn400k(mix500k):
    import maivs_amd as M
    base, _ = mix500k
    n0, nnew, rounds = 400_000, 100_000, 10
    ix = M.build_preset(base[:n0], "quality")
    dele = np.random.RandomState(501).choice(n0, nnew, replace=False)
    per = nnew // rounds
    for r in range(rounds):
        for i in dele[r * per:(r + 1) * per]:
            assert ix.remove(int(i))
        lo = n0 + r * per
        ix.add_batch(list(range(lo, lo + per)), np.ascontiguousarray(base[lo:lo + per]))
    ix.compact()
    gone = np.zeros(n0 + nnew, bool)
    gone[dele] = True
    live = np.nonzero(~gone)[0]
    tags = np.random.RandomState(502).randint(0, 1000, n0 + nnew).astype(np.uint32)
    ix.set_tags([int(i) for i in live], [int(tags[i]) for i in live])
    _log(f"churn400k: {int(ix.stats()['n_live'])} live, {int(ix.stats()['n_cells'])} cells")
    return ix, tags, live


@pytest.mark.parametrize("t,nprobe", [(500, 64), (100, 256), (10, 1024), (1, 1024)])
def test_churn400k_filtered(ctx, churn400k, mix500k, t, nprobe):
    ix, tags, live = churn400k
    base, queries = mix500k
    ix.set_filter(0, t - 1)
    try:
        ix.set_rerank_factor(16)
        p = _params(ix, 10, nprobe)
        assert p.filter == 1
        # the batched path with the filter inside its scans
        _compare_search(ctx, ix, queries, p)
        # the per-query path, which the reference runs whenever a filter is set
        s, v = ctx.search_queries(queries, p)
        os_, ov = oracle.search_one(ix._arena_desc(), queries, p, 8)
        assert np.array_equal(s, os_)
        assert v.tobytes() == ov.tobytes()
        ext = ix._ext_ids()
        got = ext[s[s != 0xFFFFFFFF]]
        assert len(got) and np.all(tags[got] <= t - 1)
        _log(f"churn400k t={t} np{nprobe}: batched and per-query bit-exact")
    finally:
        ix.set_filter()
        ix.set_rerank_factor(32)


def test_churn400k_unfiltered(ctx, churn400k, mix500k):
    ix, _, _ = churn400k
    _, queries = mix500k
    _compare_search(ctx, ix, queries, _params(ix, 10, 128))
