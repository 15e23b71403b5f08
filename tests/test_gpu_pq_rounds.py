"""The per-query scan's three forms on the GPU, each against the oracle's search_one
(src/index.rs:1381-1864): cell by cell (what batches above 64 queries run), in rounds of up to
eight probed cells scanned together by one workgroup, and split (every probed cell scored by its
own workgroup, then the bucket queue replayed from the cells' histograms; the default for batches
of up to 64 queries and 256 probes). Each form is forced for every batch size here. Slots and
score bits identical, query by query, for FastScan and the Hamming branch, adaptive stops inside a
round, multi-home vectors, the tag filter, nucleus probe lists and candidate buffers that overflow
and grow; the finish's two workgroup sizes, the rerank spread over workgroups and the fused or
separate prep, descent and route likewise.
"""
import numpy as np
import pytest

import oracle
from maivs_amd import capi

from .test_oracle_pq import churned_uncompacted, tight_uncompacted, tree40k  # noqa: F401  (fixtures)

pytestmark = pytest.mark.gpu

# (MAIVS_GPU_PQ_ROUNDS, MAIVS_GPU_PQ_SPLIT, MAIVS_GPU_FINISH_WIDE, MAIVS_GPU_PQ_FRONT,
# MAIVS_GPU_PQ_FINISH_SPLIT): the largest batch each form serves; the split form also runs the
# fused prep + descent + route and the rerank over workgroups for every batch size, the rounds form
# the 1024-thread finish, the cell-by-cell form the separate launches and the 256-thread finish
MODES = [("0", "0", "0", "0", "0"), ("1000000", "0", "1000000", "0", "0"),
         ("0", "1000000", "0", "1000000", "1000000")]


def _params(ix, k, nprobe, tc=1.0, beta=8.0):
    return capi.params_from_bytes(ix._search_params(k, nprobe, tc, beta))


@pytest.fixture(params=MODES, ids=["cell_by_cell", "rounds", "split"])
def ctx(request, monkeypatch):
    monkeypatch.setenv("MAIVS_GPU_PQ_ROUNDS", request.param[0])
    monkeypatch.setenv("MAIVS_GPU_PQ_SPLIT", request.param[1])
    monkeypatch.setenv("MAIVS_GPU_FINISH_WIDE", request.param[2])
    monkeypatch.setenv("MAIVS_GPU_PQ_FRONT", request.param[3])
    monkeypatch.setenv("MAIVS_GPU_PQ_FINISH_SPLIT", request.param[4])
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


def test_rounds_fastscan_presets_and_routes(ctx, quality50k, memory50k, tree40k, mix50k):
    _, queries, _ = mix50k
    for ix in (quality50k, memory50k, tree40k):
        for nprobe, rf in ((1, 8), (10, 8), (64, 16), (200, 4)):
            ix.set_rerank_factor(rf)
            try:
                _compare(ctx, ix, queries[:200], _params(ix, 10, nprobe))
                _compare(ctx, ix, queries[200:201], _params(ix, 10, nprobe))
            finally:
                ix.set_rerank_factor(32)


def test_rounds_nucleus_and_adaptive_stops(ctx, quality50k, mix50k):
    """All 390 cells probed with the adaptive stop on: the scan ends inside a round for most
    queries, and the round's entries of the cells after the stop are dropped."""
    _, queries, _ = mix50k
    st = capi.GpuStats()
    _compare(ctx, quality50k, queries[:300], _params(quality50k, 10, 390), st)
    _compare(ctx, quality50k, queries[:300], _params(quality50k, 10, 64, 0.9), st)


def test_rounds_filtered(ctx, churn50k, mix50k):
    _, queries, _ = mix50k
    ix, _, _ = churn50k
    for t, nprobe in ((100, 64), (1, 312)):
        ix.set_filter(0, t - 1)
        try:
            _compare(ctx, ix, queries[:200], _params(ix, 10, nprobe))
        finally:
            ix.set_filter()


def test_rounds_hamming_branch(ctx, churned_uncompacted, tight_uncompacted, mix50k):
    _, queries, _ = mix50k
    ix = churned_uncompacted
    for nprobe, rf, adaptive in ((8, 8, True), (156, 2, True), (40, 16, False)):
        ix.set_rerank_factor(rf)
        ix.set_adaptive(adaptive, 0.02)
        try:
            _compare(ctx, ix, queries[:200], _params(ix, 10, nprobe))
        finally:
            ix.set_rerank_factor(32)
            ix.set_adaptive(True, 0.02)
    # tight clusters: the stop fires after a cluster's cells, ties at tau
    tix, x = tight_uncompacted
    q = np.ascontiguousarray(x[:200] + 0.0)
    for nprobe, rf in ((64, 2), (128, 1)):
        tix.set_rerank_factor(rf)
        try:
            _compare(ctx, tix, q, _params(tix, 10, nprobe))
        finally:
            tix.set_rerank_factor(32)


def test_rounds_candidate_buffer_grows(ctx, quality50k, mix50k):
    """No adaptive stop, (nearly) every cell, k * rf > N: the candidate lists outgrow the scan's
    buffer (the host grows it and runs the scan again) and the on-chip staging."""
    _, queries, _ = mix50k
    ix = quality50k
    ix.set_adaptive(False, 0.02)
    ix.set_rerank_factor(5001)
    try:
        _compare(ctx, ix, queries[:12], _params(ix, 10, 390))
        _compare(ctx, ix, queries[12:20], _params(ix, 10, 256))
    finally:
        ix.set_adaptive(True, 0.02)
        ix.set_rerank_factor(32)
