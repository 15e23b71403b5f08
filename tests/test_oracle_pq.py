"""Pins for the oracle's per-query path (route_query + search_one + rerank_exact, src/index.rs:
1168-1305, 1381-1864, 1309-1378), against what the algorithm fixes:

* two-stage routing with shortlist_mult 2 is route_batch's rule, already pinned by brute force;
* the centroid-tree route with every top node in the beam reaches every leaf: its shortlist is
  the stable `want` smallest Hamming distances in leaf order (keep_smallest), and the probe list
  the best exact centroid scores among them (float64 within 1e-5);
* an exhaustive search (every cell probed, no adaptive stop, k * rerank_factor >= N) returns the
  exact top-k of all live vectors, each vector once;
* the bucket queue: its incremental threshold equals the closed form tau = min(maxk >> 6,
  max{t : #(h <= t - 1) < target}) over the scanned entries (after the tag filter and the
  first-ranked-home rule), recomputed here in numpy from the FastScan distances.
"""
import numpy as np
import pytest

import maivs_amd as M
import oracle
from maivs_amd import capi

from .conftest import small_clustered
from .test_oracle import _all_nibbles


def _params(ix, k, nprobe, tc=1.0, beta=8.0):
    return capi.params_from_bytes(ix._search_params(k, nprobe, tc, beta))


@pytest.fixture(scope="module")
def tree40k(mix50k):
    """40k vectors, 312 cells, a one-level centroid tree (the threshold lowered to 256 cells)."""
    base, _, _ = mix50k
    x = np.ascontiguousarray(base[:40000])
    ix = M.preset(384, len(x))
    ix.set_tree_route(True, 256, 16)
    ix.train_centroids(x, 312)
    ix.add_batch(list(range(len(x))), x)
    ix.compact()
    assert ix._tree_arrays() is not None
    return ix


def _cent_scores(arr, q):
    """Exact centroid scores of route_query (src/index.rs:777-800), float64: SQ8 copy when present."""
    d = arr["dim"]
    code = arr["cent_sq8"].reshape(-1, d).astype(np.float64)
    return (code * arr["csq_step"].astype(np.float64) + arr["csq_min"].astype(np.float64)) @ q.astype(np.float64)


@pytest.mark.parametrize("nprobe,tc", [(16, 1.0), (5, 1.0), (64, 1.0), (16, 0.9)])
def test_route_query_two_stage_is_route_batch(quality50k, mix50k, nprobe, tc):
    _, queries, _ = mix50k
    ix = quality50k
    assert ix._tree_arrays() is None  # 390 cells: below the tree threshold, two-stage routing
    p = _params(ix, 10, nprobe, tc)
    assert p.shortlist_mult == 2
    qs = queries[:64]
    a = ix._arena_arrays()
    _, ch_b, cs_b, n_b = oracle.route_batch(ix._arena_desc(), qs, p, a["n_words"], nthreads=4)
    ch_q, cs_q, n_q = oracle.route_query(ix._arena_desc(), qs, p, nthreads=4)
    assert np.array_equal(n_b, n_q)
    assert np.array_equal(ch_b, ch_q)
    assert np.array_equal(cs_b.view(np.uint32), cs_q.view(np.uint32))


def _leaf_hamming(tree, arr, q):
    W = arr["n_words"]
    rq = oracle.rotate(q, arr["rot_signs"], arr["dim_pad"])
    qb = oracle.pack_signs(rq, W)
    leaves = tree["leaf_codes"].reshape(-1, W)
    x = np.bitwise_xor(leaves, qb[None, :])
    return np.array([sum(bin(int(w)).count("1") for w in row) for row in x])


@pytest.mark.parametrize("nprobe", [40, 100])
def test_route_query_tree_bruteforce(tree40k, mix50k, nprobe):
    _, queries, _ = mix50k
    ix = tree40k
    arr = ix._arena_arrays()
    tree = ix._tree_arrays()
    n_top = int(tree["level_n"][0])
    assert len(tree["level_n"]) == 1
    p = _params(ix, 10, nprobe)
    want = min(nprobe * max(p.shortlist_mult, 2), len(tree["leaf_cells"]))
    # every top node sits in the beam (ceil(want * frac) >= its size): the descent reaches every leaf
    assert np.ceil(want * tree["beam_frac"]) >= n_top
    qs = queries[:24]
    ch, cs, nch = oracle.route_query(ix._arena_desc(), qs, p, nthreads=4)
    live = arr["mem_off"][1:] > arr["mem_off"][:-1]
    for i, q in enumerate(qs):
        h = _leaf_hamming(tree, arr, q)
        # keep_smallest over the leaves in order: the `want` smallest, ties at the cut by leaf order
        order = np.argsort(h, kind="stable")[:want]
        cells = [int(c) for c in tree["leaf_cells"][np.sort(order)] if live[c]]
        sc = _cent_scores(arr, q)
        ranked = sorted(cells, key=lambda c: (-sc[c], c))[:nprobe]
        got = [int(c) for c in ch[i, : nch[i]]]
        assert len(got) == len(ranked)
        assert np.allclose(cs[i, : nch[i]], sc[got], atol=1e-5)
        assert all(a >= b for a, b in zip(cs[i, : nch[i]], cs[i, 1: nch[i]]))
        # the same set, up to scores within rounding of the cut
        if len(cells) > nprobe:
            cut = sc[ranked[-1]]
            nxt = max(sc[c] for c in cells if c not in ranked)
            if cut - nxt > 1e-5:
                assert set(got) == set(ranked), i
        else:
            assert set(got) == set(cells)


@pytest.mark.parametrize("use_tree", [False, True])
def test_search_one_exhaustive_is_exact_topk(quality50k, tree40k, mix50k, use_tree):
    base, queries, _ = mix50k
    ix = tree40k if use_tree else quality50k
    arr = ix._arena_arrays()
    n = arr["n_slots"]
    ix.set_adaptive(False, 0.02)
    ix.set_rerank_factor((n + 9) // 10 + 1)
    try:
        nprobe = arr["n_cells"]
        p = _params(ix, 10, nprobe)
        qs = queries[:16]
        slots, scores = oracle.search_one(ix._arena_desc(), qs, p, nthreads=8)
        vecs = arr["vecs_f32"].reshape(n, -1).astype(np.float64)
        for i, q in enumerate(qs):
            ex = vecs @ q.astype(np.float64)
            top = np.argsort(-ex, kind="stable")[:11]
            got = [int(s) for s in slots[i]]
            assert len(set(got)) == 10  # each vector once
            assert np.allclose(scores[i], ex[got], rtol=1e-5, atol=1e-6)
            if ex[top[9]] - ex[top[10]] > 1e-5:
                assert set(got) == set(top[:10].tolist()), i
    finally:
        ix.set_adaptive(True, 0.02)
        ix.set_rerank_factor(32)


@pytest.mark.parametrize("nprobe,rf,filt", [(16, 8, None), (4, 32, None), (32, 4, None), (16, 8, (0, 99)),
                                             (48, 8, (0, 9))])
def test_search_one_bucket_queue_closed_form(quality50k, mix50k, nprobe, rf, filt):
    _, queries, _ = mix50k
    ix = quality50k
    ix.set_rerank_factor(rf)
    ix.set_adaptive(False, 0.02)
    ext = ix._ext_ids()
    tags = np.random.RandomState(502).randint(0, 1000, len(ext)).astype(np.uint32)
    if filt is not None:
        ix.set_tags([int(x) for x in ext], [int(t) for t in tags])
        ix.set_filter(*filt)
    try:
        arr = ix._arena_arrays()
        nibs = _all_nibbles(ix._codes().reshape(-1, arr["n_words"]))
        npos = nibs.shape[1]
        maxk = 255 * npos
        target = 10 * rf
        p = _params(ix, 10, nprobe)
        qs = queries[:12]
        slots, scores = oracle.search_one(ix._arena_desc(), qs, p, nthreads=4)
        ch, _, nch = oracle.route_query(ix._arena_desc(), qs, p, nthreads=4)
        sc = arr["slot_cells"].reshape(-1, arr["max_assign"])
        vecs = arr["vecs_f32"].reshape(-1, arr["dim"]).astype(np.float64)
        for i, q in enumerate(qs):
            chosen = [int(c) for c in ch[i, : nch[i]]]
            rank = {c: r for r, c in enumerate(chosen)}
            rq = oracle.rotate(q, arr["rot_signs"], arr["dim_pad"])
            tab = oracle.fs_query(rq, arr["n_words"])[0].reshape(npos, 16).astype(np.int64)
            U = []
            for r, c in enumerate(chosen):
                mem = arr["members"][arr["mem_off"][c]: arr["mem_off"][c + 1]].astype(np.int64)
                dd = maxk - tab[np.arange(npos)[None, :], nibs[mem]].sum(axis=1)
                for slot, d in zip(mem.tolist(), dd.tolist()):
                    if filt is not None and not (filt[0] <= tags[slot] <= filt[1]):
                        continue
                    if any(h != 0xFFFFFFFF and h != c and h in rank and rank[h] < r for h in sc[slot].tolist()):
                        continue  # scored at its first-ranked probed home
                    U.append((d, slot))
            h = np.array([d >> 6 for d, _ in U], np.int64)
            tau = maxk >> 6
            while tau > 0 and (h <= tau - 1).sum() >= target:
                tau -= 1
            kept = sorted(x for x, hh in zip(U, h) if hh <= tau)[:target]
            ex = sorted(((float(vecs[s] @ q.astype(np.float64)), s) for _, s in kept), key=lambda t: (-t[0], t[1]))
            kk = min(10, len(ex))
            got = [int(s) for s in slots[i] if s != 0xFFFFFFFF]
            assert len(got) == kk and len(set(got)) == kk
            assert np.allclose([e for e, _ in ex[:kk]], scores[i][:kk], rtol=1e-5, atol=1e-6)
            if kk == len(ex) or ex[kk - 1][0] - ex[kk][0] > 1e-5:
                assert set(got) == {s for _, s in ex[:kk]}, i
            if filt is not None:
                assert all(filt[0] <= tags[s] <= filt[1] for s in got)
    finally:
        ix.set_rerank_factor(32)
        ix.set_adaptive(True, 0.02)
        ix.set_filter()


def test_gate_mirrors_the_reference(quality50k):
    """cm_ok (src/index.rs:3343-3348): batched only for cell_major, enough queries and no filter."""
    import os
    ix = quality50k
    threads = int(os.environ.get("MAIVS_NUM_THREADS") or os.environ.get("RAYON_NUM_THREADS")
                  or os.environ.get("OMP_NUM_THREADS") or os.cpu_count())
    assert ix.takes_cellmajor(2 * threads, True)
    assert not ix.takes_cellmajor(2 * threads - 1, True)
    assert not ix.takes_cellmajor(10 ** 6, False)
    ix.set_filter(0, 10)
    try:
        assert not ix.takes_cellmajor(10 ** 6, True)
        ix.set_batched_filter(True)
        assert ix.takes_cellmajor(10 ** 6, True)
    finally:
        ix.set_batched_filter(False)
        ix.set_filter()
    assert ix.perquery_blocker() == ""


def test_search_binding_errors():
    x = small_clustered(800, 32, 8, seed=3)
    ix = M.preset(32, len(x))
    assert ix.search(x[0], 5) == ([], [])  # empty index (src/index.rs:3295-3297)
    ix.train_centroids(x, 8)
    ix.add_batch(list(range(len(x))), x)
    # not compacted: search() takes the Hamming branch over the per-slot codes (no blocker)
    assert ix.perquery_blocker() == ""
    with pytest.raises(ValueError):
        ix.search(np.zeros(31, np.float32), 5)
    with pytest.raises(TypeError):
        ix.search(np.zeros(32, np.float64), 5)


@pytest.fixture(scope="module")
def churned_uncompacted(mix50k):
    """20k vectors, 156 cells, then 3 rounds of (delete 1,000 random ids, insert 1,000 new ones) and
    no compact(): member lists in swap_remove order, per-slot codes, no FastScan blocks."""
    base, _, _ = mix50k
    x = np.ascontiguousarray(base[:20000])
    ix = M.preset(384, len(x))
    ix.train_centroids(x, 156)
    ix.add_batch(list(range(len(x))), x)
    ix.compact()
    rs = np.random.RandomState(11)
    dele = rs.choice(20000, 3000, replace=False)
    for r in range(3):
        for i in dele[r * 1000:(r + 1) * 1000]:
            assert ix.remove(int(i))
        lo = 20000 + r * 1000
        ix.add_batch(list(range(lo, lo + 1000)), np.ascontiguousarray(base[lo:lo + 1000]))
    arr = ix._arena_arrays()
    assert len(arr["fs_codes"]) == 0 and len(arr["fs_off"]) == 0  # the Hamming branch's arena
    assert not ix.takes_cellmajor(10 ** 6, True)
    return ix


def _popcounts(x):
    """Per-row popcount of a (n, W) uint64 array."""
    b = np.ascontiguousarray(x).view(np.uint8)
    return np.unpackbits(b, axis=1).sum(axis=1).astype(np.int64)


def _hamming_branch_closed_form(ix, q, p, chosen, tags=None, filt=None, upto=None):
    """search_one's Hamming branch over the first `upto` probed cells (all when None), restated in
    numpy from its definition: the canonical entries (tag filter, first-ranked probed home), their
    Hamming distances h to the query's code, the final bucket-queue threshold
    tau = min{t : #(h <= t) >= target} (W * 64 when fewer than target entries), every entry with
    h <= tau reranked exactly in float64. Returns (tau, kept count, [(score, slot)] sorted)."""
    arr = ix._arena_arrays()
    W = arr["n_words"]
    dp = W * 64
    target = p.k * max(p.rerank_factor, 1)
    codes = ix._codes().reshape(-1, W)
    rq = oracle.rotate(q, arr["rot_signs"], arr["dim_pad"])
    qb = oracle.pack_signs(rq, W)
    sc = arr["slot_cells"].reshape(-1, arr["max_assign"])
    rank = {c: r for r, c in enumerate(chosen)}
    U = []
    for r, c in enumerate(chosen[: upto if upto is not None else len(chosen)]):
        mem = arr["members"][arr["mem_off"][c]: arr["mem_off"][c + 1]].astype(np.int64)
        h = _popcounts(codes[mem] ^ qb[None, :])
        for slot, hh in zip(mem.tolist(), h.tolist()):
            if filt is not None and not (filt[0] <= tags[slot] <= filt[1]):
                continue
            if any(x != 0xFFFFFFFF and x != c and x in rank and rank[x] < r for x in sc[slot].tolist()):
                continue
            U.append((hh, slot))
    hs = np.array([h for h, _ in U], np.int64)
    cnt = np.bincount(hs, minlength=dp + 1).cumsum() if len(hs) else np.zeros(dp + 1, np.int64)
    reach = np.nonzero(cnt >= target)[0]
    tau = int(reach[0]) if len(reach) else dp
    kept = [s for h, s in U if h <= tau]
    vecs = arr["vecs_f32"].reshape(-1, arr["dim"]).astype(np.float64)
    ex = sorted(((float(vecs[s] @ q.astype(np.float64)), s) for s in kept), key=lambda t: (-t[0], t[1]))
    return tau, int(cnt[tau]), ex


@pytest.mark.parametrize("nprobe,rf,filt", [(8, 8, None), (24, 4, None), (156, 2, None), (16, 8, (0, 99))])
def test_search_one_hamming_branch_closed_form(churned_uncompacted, mix50k, nprobe, rf, filt):
    """With adaptive stopping off, the oracle's Hamming branch equals the closed form over every
    probed cell: the same reranked survivors, ties at tau included."""
    _, queries, _ = mix50k
    ix = churned_uncompacted
    ix.set_rerank_factor(rf)
    ix.set_adaptive(False, 0.02)
    ext = ix._ext_ids()
    tags = np.random.RandomState(502).randint(0, 1000, len(ext)).astype(np.uint32)
    if filt is not None:
        # every slot is live here (the inserts reused the deleted slots): slot i gets tags[i]
        ix.set_tags([int(e) for e in ext], [int(t) for t in tags])
        ix.set_filter(*filt)
    try:
        p = _params(ix, 10, nprobe)
        qs = queries[:12]
        slots, scores = oracle.search_one(ix._arena_desc(), qs, p, nthreads=4)
        ch, _, nch = oracle.route_query(ix._arena_desc(), qs, p, nthreads=4)
        for i, q in enumerate(qs):
            chosen = [int(c) for c in ch[i, : nch[i]]]
            _, _, ex = _hamming_branch_closed_form(ix, q, p, chosen, tags, filt)
            kk = min(10, len(ex))
            got = [int(s) for s in slots[i] if s != 0xFFFFFFFF]
            assert len(got) == kk and len(set(got)) == kk
            assert np.allclose([e for e, _ in ex[:kk]], scores[i][:kk], rtol=1e-5, atol=1e-6)
            if kk == len(ex) or ex[kk - 1][0] - ex[kk][0] > 1e-5:
                assert set(got) == {s for _, s in ex[:kk]}, i
            if filt is not None:
                assert all(filt[0] <= tags[s] <= filt[1] for s in got)
    finally:
        ix.set_rerank_factor(32)
        ix.set_adaptive(True, 0.02)
        ix.set_filter()


def tight_clusters(n=12000, d=64, n_clusters=16, seed=5):
    """Unit vectors in 16 tight clusters (noise 0.08 / sqrt(d)): cells cut from one cluster have
    small radii, so the reachability bounds of the other clusters' cells fall far below the
    Hamming branch's stop threshold and its adaptive stop fires after a cluster's cells."""
    rs = np.random.RandomState(seed)
    cent = rs.standard_normal((n_clusters, d))
    cent /= np.linalg.norm(cent, axis=1, keepdims=True)
    x = cent[rs.randint(0, n_clusters, n)] + 0.08 * rs.standard_normal((n, d)) / np.sqrt(d)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    return x.astype(np.float32)


@pytest.fixture(scope="module")
def tight_uncompacted():
    """10k tight-cluster vectors in 128 cells, 300 deletes and 2,000 inserts, no compact()."""
    x = tight_clusters()
    ix = M.preset(64, 10000)
    ix.train_centroids(x[:10000], 128)
    ix.add_batch(list(range(10000)), x[:10000])
    ix.compact()
    for i in range(300):
        assert ix.remove(i)
    ix.add_batch(list(range(10000, 12000)), x[10000:])
    return ix, x


def test_search_one_hamming_branch_adaptive_stop(tight_uncompacted):
    """With adaptive stopping on, the oracle's answer is the closed form over the first L probed
    cells, where L is the first prefix whose stop test fires: kept >= target and the best remaining
    reachability bound below cos(pi * tau / dp) - margin (src/index.rs:1779-1788), evaluated here in
    float64 (prefixes within 1e-5 of the threshold are skipped as libm-dependent)."""
    ix, x = tight_uncompacted
    queries = x[:64] + 0.0
    ix.set_rerank_factor(2)
    p = _params(ix, 10, 64)
    assert p.adaptive == 1
    arr = ix._arena_arrays()
    dp = arr["n_words"] * 64
    qs = queries[:16]
    slots, _ = oracle.search_one(ix._arena_desc(), qs, p, nthreads=4)
    ch, cs, nch = oracle.route_query(ix._arena_desc(), qs, p, nthreads=4)
    stopped_early = 0
    try:
        for i, q in enumerate(qs):
            chosen = [int(c) for c in ch[i, : nch[i]]]
            n = len(chosen)
            b = np.cos(np.maximum(np.arccos(np.clip(cs[i, :n].astype(np.float64), -1, 1))
                                  - arr["r_bound"][chosen].astype(np.float64), 0.0))
            suffix = np.append(np.maximum.accumulate(b[::-1])[::-1], -np.inf)
            L, ambiguous = n, False
            for upto in range(1, n + 1):
                tau, kept, _ = _hamming_branch_closed_form(ix, q, p, chosen, upto=upto)
                if kept >= p.k * p.rerank_factor:
                    thr = np.cos(np.pi * tau / dp) - p.at_margin
                    if abs(suffix[upto] - thr) <= 1e-5:
                        ambiguous = True
                        break
                    if suffix[upto] < thr:
                        L = upto
                        break
            if ambiguous:
                continue
            stopped_early += L < n
            _, _, ex = _hamming_branch_closed_form(ix, q, p, chosen, upto=L)
            got = [int(s) for s in slots[i] if s != 0xFFFFFFFF]
            kk = min(10, len(ex))
            if kk == len(ex) or ex[kk - 1][0] - ex[kk][0] > 1e-5:
                assert set(got) == {s for _, s in ex[:kk]}, i
        assert stopped_early > 0  # the stop is exercised
    finally:
        ix.set_rerank_factor(32)
