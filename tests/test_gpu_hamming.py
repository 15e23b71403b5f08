"""The per-query path's Hamming branch on the GPU (search_one over an index that is not compacted,
src/index.rs:1694-1760), bit-exact against the oracle: after deletes and inserts without
compact(), with the tag filter, with the adaptive stop firing, with ties at tau past the candidate
room, through the C ABI and through the drop-in FlatCellIndex.search_batch / search. Includes the
reference's own check that a delete sends search_batch down this path and the deleted id never
comes back (tests/test_index.py:377-382)."""
import numpy as np
import pytest

import maivs_amd as M
import oracle
from maivs_amd import capi

from .test_oracle_pq import churned_uncompacted, tight_uncompacted  # noqa: F401 (fixtures)

pytestmark = pytest.mark.gpu


def _params(ix, k, nprobe, tc=1.0, beta=8.0):
    return capi.params_from_bytes(ix._search_params(k, nprobe, tc, beta))


def _ids(ix, slots):
    ext = ix._ext_ids()
    return np.where(slots == 0xFFFFFFFF, np.iinfo(np.uint64).max, ext[np.minimum(slots, len(ext) - 1)])


@pytest.mark.parametrize("nprobe,rf,adaptive,filt", [(8, 8, True, None), (24, 4, False, None),
                                                     (156, 2, True, None), (16, 8, True, (0, 99)),
                                                     (40, 16, False, (0, 9))])
def test_hamming_branch_matches_oracle(churned_uncompacted, mix50k, nprobe, rf, adaptive, filt):
    _, queries, _ = mix50k
    ix = churned_uncompacted
    ix.set_rerank_factor(rf)
    ix.set_adaptive(adaptive, 0.02)
    ext = ix._ext_ids()
    tags = np.random.RandomState(502).randint(0, 1000, len(ext)).astype(np.uint32)
    if filt is not None:
        ix.set_tags([int(e) for e in ext], [int(t) for t in tags])
        ix.set_filter(*filt)
    c = capi.Context(0)
    try:
        c.upload(ix._arena_desc())
        p = _params(ix, 10, nprobe)
        s, v = c.search_queries(queries, p)
        os_, ov = oracle.search_one(ix._arena_desc(), queries, p, 8)
        assert np.array_equal(s, os_)
        assert v.tobytes() == ov.tobytes()
        # the drop-in: search_batch takes the per-query path (not compacted), ids and scores alike
        ids, sc = ix.search_batch(queries, 10, nprobe, 1.0, 8.0, True)
        assert np.array_equal(np.array(ids, np.uint64).reshape(-1, 10), _ids(ix, os_))
        assert np.array(sc, np.float32).tobytes() == ov.tobytes()
        if filt is not None:
            got = s[s != 0xFFFFFFFF]
            assert len(got) and np.all(tags[got] <= filt[1])
    finally:
        c.close()
        ix.set_filter()
        ix.set_rerank_factor(32)
        ix.set_adaptive(True, 0.02)


def test_hamming_branch_adaptive_stop_and_ties(tight_uncompacted, monkeypatch):
    """64-bit codes in tight clusters: the adaptive stop fires after a cluster's cells, and ties at
    tau leave far more survivors than the target, past a 16-entry candidate room that then grows."""
    ix, x = tight_uncompacted
    q = np.ascontiguousarray(x[:300] + 0.0)
    monkeypatch.setenv("MAIVS_GPU_CAND_CAP", "16")
    c = capi.Context(0)
    reruns = 0
    try:
        c.upload(ix._arena_desc())
        for nprobe, rf in ((64, 2), (128, 1), (16, 4)):
            ix.set_rerank_factor(rf)
            p = _params(ix, 10, nprobe)
            st = capi.GpuStats()
            s, v = c.search_queries(q, p, st)
            os_, ov = oracle.search_one(ix._arena_desc(), q, p, 8)
            assert np.array_equal(s, os_), (nprobe, rf)
            assert v.tobytes() == ov.tobytes(), (nprobe, rf)
            reruns += st.reruns
        assert reruns >= 1  # the candidate room grew at least once
    finally:
        c.close()
        ix.set_rerank_factor(32)


def test_delete_sends_search_batch_to_the_hamming_branch(mix50k):
    """The reference's check (tests/test_index.py:377-382): search, delete one returned id, search
    again: the call falls back to the per-query path, and the id is gone; equal to the oracle."""
    base, queries, _ = mix50k
    x = np.ascontiguousarray(base[:20000])
    ix = M.build_preset(x, "quality")
    qq = np.ascontiguousarray(queries[:200])
    assert ix.takes_cellmajor(len(qq), True)
    a, _ = ix.search_batch(qq, 10, 64, 1.0, 8.0, True)
    victim = int(a[0])
    assert ix.remove(victim)
    assert not ix.takes_cellmajor(len(qq), True)
    b, sb = ix.search_batch(qq, 10, 64, 1.0, 8.0, True)
    assert victim not in b
    p = _params(ix, 10, 64)
    os_, ov = oracle.search_one(ix._arena_desc(), qq, p, 8)
    assert np.array_equal(np.array(b, np.uint64).reshape(-1, 10), _ids(ix, os_))
    assert np.array(sb, np.float32).tobytes() == ov.tobytes()
    # search() (one query) on the same path
    ids1, sc1 = ix.search(qq[5], 10, 64, 1.0, 8.0)
    assert list(ids1) == [int(i) for i in _ids(ix, os_[5]) if i != np.iinfo(np.uint64).max]
    # compact() brings the batched path back, with the id still gone
    ix.compact()
    assert ix.takes_cellmajor(len(qq), True)
    c2, _ = ix.search_batch(qq, 10, 64, 1.0, 8.0, True)
    assert victim not in c2
