"""GPU parity through the C ABI (libmaivs_gpu.so) against the oracle, on the same seeded
inputs and the same arena: FastScan tables and sums, routed cell lists, seed cut-offs,
adaptive cuts, candidate sets and final top-k must be bit-exact; recall identical.
"""
import numpy as np
import pytest

import oracle
from maivs_amd import capi, mixture

pytestmark = pytest.mark.gpu


def _params(ix, k, nprobe, tc=1.0, beta=8.0):
    return capi.params_from_bytes(ix._search_params(k, nprobe, tc, beta))


@pytest.fixture(scope="module")
def ctx():
    c = capi.Context(0)
    yield c
    c.close()


def _upload(ctx, ix):
    ctx.upload(ix._arena_desc())


def test_query_prep_matches_oracle(ctx, quality50k, mix50k):
    _, queries, _ = mix50k
    ix = quality50k
    _upload(ctx, ix)
    q = queries[:257]
    bits, lut, delta, bias = ctx.query_prep(q, 8)
    signs = ix._rot_signs()
    for i in range(len(q)):
        rq = oracle.rotate(q[i], signs, 512)
        ob = oracle.pack_signs(rq, 8)
        olut, od, obias = oracle.fs_query(rq, 8)
        assert np.array_equal(bits[i], ob), i
        assert np.array_equal(lut[i], olut), i
        assert delta[i].tobytes() == od.tobytes(), i
        assert bias[i].tobytes() == obias.tobytes(), i


def test_block_sums_match_oracle(ctx):
    rs = np.random.RandomState(7)
    nb = 64
    blocks = rs.randint(0, 256, size=(nb, 2048)).astype(np.uint8)
    luts = rs.randint(0, 256, size=(nb, 2048)).astype(np.uint8)
    luts[0] = 255  # the maximum sum, 32640
    blocks[1] = 0
    out = ctx.block_sums(blocks, luts, 8)
    for b in range(nb):
        assert np.array_equal(out[b], oracle.fs_block_sums(blocks[b], luts[b])), b
    assert out[0].max() == 32640


@pytest.mark.parametrize("nprobe,tc", [(1, 1.0), (8, 1.0), (16, 1.0), (64, 1.0), (390, 1.0), (16, 0.95), (64, 0.5)])
def test_route_matches_oracle(ctx, quality50k, mix50k, nprobe, tc):
    _, queries, _ = mix50k
    ix = quality50k
    _upload(ctx, ix)
    p = _params(ix, 10, nprobe, tc)
    ch, cs, nch = ctx.route(queries, p)
    _, och, ocs, onch = oracle.route_batch(ix._arena_desc(), queries, p, 8)
    assert np.array_equal(nch, onch)
    for i in range(len(queries)):
        n = onch[i]
        assert np.array_equal(ch[i, :n], och[i, :n]), i
        assert cs[i, :n].tobytes() == ocs[i, :n].tobytes(), i


def _compare_search(ctx, ix, queries, p, gt=None):
    _upload(ctx, ix)
    st = capi.GpuStats()
    slots, scores = ctx.search(queries, p, st)
    desc = ix._arena_desc()
    oslots, oscores = oracle.search_batch(desc, queries, p, 8)
    nq = len(queries)
    otau, ore, ocut, onc, ocs, ocd = oracle.last_candidates(nq)
    tau, re, cut, nc, cs, cd = ctx.last_candidates(nq, int(onc.sum()) + 1024)
    assert np.array_equal(tau, otau)
    assert np.array_equal(re, ore)
    assert np.array_equal(cut, ocut)
    assert np.array_equal(nc, onc)
    n = int(onc.sum())
    assert np.array_equal(cs[:n], ocs) and np.array_equal(cd[:n], ocd)
    assert np.array_equal(slots, oslots)
    assert scores.tobytes() == oscores.tobytes()
    # work counters agree with the oracle's routed lists
    ctx.last_counters(st)
    arr = ix._arena_arrays()
    blocks = (np.diff(arr["mem_off"]) + 31) // 32
    _, och, _, onch = oracle.route_batch(desc, queries, p, arr["n_words"])
    seed_b = scan_b = pairs = 0
    for i in range(nq):
        ns = min(8, int(onch[i]))
        seed_b += int(blocks[och[i, :ns]].sum())
        scan_b += int(blocks[och[i, ns:ore[i]]].sum())
        pairs += max(int(ore[i]) - ns, 0)
    assert (st.seed_blocks, st.scan_blocks, st.scan_pairs, st.rerank_rows) == (seed_b, scan_b, pairs, n)
    if gt is not None:
        ext = ix._ext_ids()
        ids = np.where(slots == 0xFFFFFFFF, -1, ext[np.minimum(slots, len(ext) - 1)].astype(np.int64))
        oids = np.where(oslots == 0xFFFFFFFF, -1, ext[np.minimum(oslots, len(ext) - 1)].astype(np.int64))
        assert mixture.recall_at(ids, gt) == mixture.recall_at(oids, gt)
    return st


@pytest.mark.parametrize("nprobe,rf", [(1, 8), (8, 8), (16, 32), (64, 16), (390, 4)])
def test_search_quality_matches_oracle(ctx, quality50k, mix50k, nprobe, rf):
    _, queries, gt = mix50k
    ix = quality50k
    ix.set_rerank_factor(rf)
    try:
        _compare_search(ctx, ix, queries, _params(ix, 10, nprobe), gt)
    finally:
        ix.set_rerank_factor(32)


@pytest.mark.parametrize("nprobe", [8, 32])
def test_search_memory_matches_oracle(ctx, memory50k, mix50k, nprobe):
    _, queries, gt = mix50k
    _compare_search(ctx, memory50k, queries, _params(memory50k, 10, nprobe), gt)


def test_search_nucleus_matches_oracle(ctx, quality50k, mix50k):
    _, queries, gt = mix50k
    _compare_search(ctx, quality50k, queries, _params(quality50k, 10, 32, tc=0.95), gt)


def test_search_small_batches_and_k(ctx, quality50k, mix50k):
    _, queries, _ = mix50k
    ix = quality50k
    for nq, k in [(1, 10), (3, 1), (17, 100)]:
        _compare_search(ctx, ix, queries[:nq], _params(ix, k, 16))


def test_binding_search_batch(quality50k, mix50k):
    """The Python drop-in (FlatCellIndex.search_batch) returns the oracle's answer as ids."""
    _, queries, gt = mix50k
    ix = quality50k
    ids, scores = ix.search_batch(queries, 10, 16, 1.0, 8.0, True)
    p = _params(ix, 10, 16)
    check = oracle.search_batch if ix.takes_cellmajor(len(queries), True) else oracle.search_one
    oslots, oscores = check(ix._arena_desc(), queries, p, 8)
    ext = ix._ext_ids()
    oids = np.where(oslots == 0xFFFFFFFF, np.iinfo(np.uint64).max, ext[np.minimum(oslots, len(ext) - 1)])
    assert np.array_equal(np.array(ids, dtype=np.uint64).reshape(oids.shape), oids)
    assert np.array(scores, np.float32).tobytes() == oscores.tobytes()


def test_graph_replays_match_eager(quality50k, mix50k, monkeypatch):
    """The main pass replayed as one captured HIP graph returns the eager result on every replay,
    with other eager GPU work and synchronisations between the replays, and after re-captures."""
    _, queries, _ = mix50k
    ix = quality50k
    monkeypatch.setenv("MAIVS_GPU_GRAPH", "0")
    eager = capi.Context(0)
    monkeypatch.setenv("MAIVS_GPU_GRAPH", "1")
    graph = capi.Context(0)
    try:
        eager.upload(ix._arena_desc())
        graph.upload(ix._arena_desc())
        for npb in (16, 48, 16):
            p = _params(ix, 10, npb)
            ref_s, ref_v = eager.search(queries, p)
            for rep in range(4):
                st = capi.GpuStats()
                s, v = graph.search(queries, p, st)
                assert np.array_equal(s, ref_s), (npb, rep)
                assert v.tobytes() == ref_v.tobytes(), (npb, rep)
                assert st.ms_total > 0
                eager.search(queries[: 97 + rep], p)  # unrelated eager work between replays
            # a different batch size re-captures; the original shape then re-captures again
            s2, _ = graph.search(queries[:33], p)
            e2, _ = eager.search(queries[:33], p)
            assert np.array_equal(s2, e2)
    finally:
        eager.close()
        graph.close()


def test_search_bucket_overflow_falls_back(ctx, quality50k, mix50k):
    """Many queries probing the same cells overflow the per-cell query buckets; the pass then runs
    the counting-sort inversion and still matches the oracle."""
    _, queries, _ = mix50k
    ix = quality50k
    q = np.repeat(queries[:3], 150, axis=0)  # 450 queries, three distinct probe lists
    _compare_search(ctx, ix, q, _params(ix, 10, 40))


@pytest.mark.parametrize("t,nprobe", [(500, 16), (100, 64), (10, 128), (1, 312)])
def test_search_churned_filtered_matches_oracle(ctx, churn50k, mix50k, t, nprobe):
    """Churned index (deletes, inserts, compact), tag filter tag <= t - 1 applied inside the seed and
    cell-major scans: bit-exact with the oracle's filtered restatement; every result passes."""
    _, queries, _ = mix50k
    ix, tags, _ = churn50k
    ix.set_filter(0, t - 1)
    try:
        p = _params(ix, 10, nprobe)
        assert p.filter == 1 and (p.tag_lo, p.tag_hi) == (0, t - 1)
        _compare_search(ctx, ix, queries, p)
        ids, _ = ix.search_batch(queries, 10, nprobe, 1.0, 8.0, True)
        got = [i for i in ids if i != 2 ** 64 - 1]
        assert got and all(tags[i] <= t - 1 for i in got)
    finally:
        ix.set_filter()


def test_search_churned_unfiltered_matches_oracle(ctx, churn50k, mix50k):
    _, queries, _ = mix50k
    ix, _, _ = churn50k
    _compare_search(ctx, ix, queries, _params(ix, 10, 16))


@pytest.fixture(scope="module")
def dead20k(mix50k):
    """20k vectors in 156 cells with every member of four cells removed, then compact(): the
    emptied (dead) cells must leave the Hamming histogram and never be routed."""
    import maivs_amd as M
    base, _, _ = mix50k
    x = np.ascontiguousarray(base[:20000])
    ix = M.preset(384, len(x))
    ix.train_centroids(x, 156)
    ix.add_batch(list(range(len(x))), x)
    ix.compact()
    arr = ix._arena_arrays()
    ext = ix._ext_ids()
    gone = set()
    for c in (5, 17, 42, 99):
        for slot in arr["members"][arr["mem_off"][c]: arr["mem_off"][c + 1]].tolist():
            gone.add(int(ext[slot]))
    for v in sorted(gone):
        assert ix.remove(v)
    ix.compact()
    mo = ix._arena_arrays()["mem_off"]
    assert int((np.diff(mo) == 0).sum()) >= 4
    return ix


@pytest.mark.parametrize("nprobe", [8, 40, 152])
def test_dead_cells_match_oracle(ctx, dead20k, mix50k, nprobe):
    _, queries, _ = mix50k
    ix = dead20k
    _upload(ctx, ix)
    p = _params(ix, 10, nprobe)
    ch, cs, nch = ctx.route(queries, p)
    _, och, ocs, onch = oracle.route_batch(ix._arena_desc(), queries, p, 8)
    assert np.array_equal(nch, onch)
    dead = set(np.nonzero(np.diff(ix._arena_arrays()["mem_off"]) == 0)[0].tolist())
    for i in range(len(queries)):
        n = onch[i]
        assert np.array_equal(ch[i, :n], och[i, :n]), i
        assert not dead & set(ch[i, :n].tolist()), i
    _compare_search(ctx, ix, queries, p)
    s, v = ctx.search_queries(queries[:200], p)
    os_, ov = oracle.search_one(ix._arena_desc(), queries[:200], p, 8)
    assert np.array_equal(s, os_)
    assert v.tobytes() == ov.tobytes()


@pytest.fixture(scope="module")
def cells9k(mix50k):
    """50k vectors in 9,000 cells: more cells than the route keeps in LDS (8,192), so every query's
    Hamming row goes through its global-memory row instead."""
    import maivs_amd as M
    base, _, _ = mix50k
    x = np.ascontiguousarray(base)
    ix = M.preset(384, len(x))
    ix.train_centroids(x, 9000)
    ix.add_batch(list(range(len(x))), x)
    ix.compact()
    assert ix.stats()["n_cells"] == 9000
    return ix


@pytest.mark.parametrize("nprobe", [10, 40])
def test_global_hamming_rows_match_oracle(ctx, cells9k, mix50k, nprobe):
    _, queries, gt = mix50k
    ix = cells9k
    _upload(ctx, ix)
    p = _params(ix, 10, nprobe)
    ch, cs, nch = ctx.route(queries, p)
    _, och, ocs, onch = oracle.route_batch(ix._arena_desc(), queries, p, 8)
    assert np.array_equal(nch, onch)
    for i in range(len(queries)):
        n = onch[i]
        assert np.array_equal(ch[i, :n], och[i, :n]), i
        assert cs[i, :n].tobytes() == ocs[i, :n].tobytes(), i
    _compare_search(ctx, ix, queries, p, gt)


@pytest.mark.parametrize("mma", ["1", "0"])
def test_hamming_rows_both_kernels_match_oracle(cells9k, mix50k, monkeypatch, mma):
    """The query-tiled Hamming rows on the matrix cores (popc(q) + popc(c) - 2 q.c over int8 bits,
    MAIVS_GPU_HAM_MMA=1) and by popcounts (0): the routing built from them equals the oracle's, probe
    lists and score bits, for 1,000 queries (not a multiple of the 128-query tile) and 9,000 cells."""
    monkeypatch.setenv("MAIVS_GPU_HAM_MMA", mma)
    _, queries, gt = mix50k
    ix = cells9k
    c = capi.Context(0)
    try:
        _upload(c, ix)
        for nprobe in (5, 40):
            p = _params(ix, 10, nprobe)
            ch, cs, nch = c.route(queries, p)
            _, och, ocs, onch = oracle.route_batch(ix._arena_desc(), queries, p, 8)
            assert np.array_equal(nch, onch)
            for i in range(len(queries)):
                n = onch[i]
                assert np.array_equal(ch[i, :n], och[i, :n]), i
                assert cs[i, :n].tobytes() == ocs[i, :n].tobytes(), i
        _compare_search(c, ix, queries[:333], _params(ix, 10, 40), None)
    finally:
        c.close()


@pytest.mark.parametrize("mma", ["1", "0"])
def test_rows_pass_at_few_cells_matches_oracle(quality50k, churn50k, mix50k, monkeypatch, mma):
    """The batched pass by Hamming rows (prep, the rows kernel, route + seed from the rows) forced
    on indexes whose rows would fit in LDS (MAIVS_GPU_ROWS=1): the shortlist and the dead-cell
    fix-up read the written rows, and the search equals the oracle's, with both rows kernels."""
    monkeypatch.setenv("MAIVS_GPU_ROWS", "1")
    monkeypatch.setenv("MAIVS_GPU_HAM_MMA", mma)
    _, queries, gt = mix50k
    c = capi.Context(0)
    try:
        for nprobe in (10, 40):
            _compare_search(c, quality50k, queries, _params(quality50k, 10, nprobe), gt)
        ix, _, _ = churn50k
        _compare_search(c, ix, queries[:500], _params(ix, 10, 24))
    finally:
        c.close()


@pytest.mark.parametrize("mode", ["1", "0", "12"])
def test_scan_paths_match_oracle(quality50k, memory50k, churn50k, mix50k, monkeypatch, mode):
    """The cell-major scan with every bucket work item on the matrix cores (MAIVS_GPU_MMA_MIN=1:
    one-hot int8 products, even for items of one query), every item on the table lookups (0), or
    split by size (12: items of fewer queries go to the lookups, screened per workgroup): all
    bit-exact with the oracle, for both presets and with the tag filter."""
    monkeypatch.setenv("MAIVS_GPU_MMA_MIN", mode)
    _, queries, gt = mix50k
    c = capi.Context(0)
    try:
        for nprobe in (24, 64):
            _compare_search(c, quality50k, queries, _params(quality50k, 10, nprobe), gt)
        _compare_search(c, memory50k, queries, _params(memory50k, 10, 40), gt)
        ix, _, _ = churn50k
        ix.set_filter(0, 99)
        try:
            _compare_search(c, ix, queries, _params(ix, 10, 64))
        finally:
            ix.set_filter()
    finally:
        c.close()


@pytest.mark.parametrize("d", [64, 128, 200, 768])
def test_other_code_widths_match_oracle(monkeypatch, d):
    """The batched pass at other dimensions, so that every code width the kernels are built for
    runs (padded dims 64, 128, 256, 1024: 1, 2, 4 and 16 words): seed, rest and cell-major scans on
    the lookups and on the matrix cores, and the per-query scan on pair tables, bit-exact with the
    oracle."""
    import maivs_amd as M
    from .conftest import small_clustered
    x = small_clustered(12400, d, 60, seed=31 + d)
    base, queries = np.ascontiguousarray(x[:12000]), np.ascontiguousarray(x[12000:])
    ix = M.build_preset(base, "quality")
    for mode in ("0", "1"):
        monkeypatch.setenv("MAIVS_GPU_MMA_MIN", mode)
        c = capi.Context(0)
        try:
            for nprobe in (10, 40):
                p = _params(ix, 10, nprobe)
                _compare_search(c, ix, queries, p)
                # the per-query path at this width (pair tables: at most 256 queries)
                s, v = c.search_queries(queries[:100], p)
                os_, ov = oracle.search_one(ix._arena_desc(), queries[:100], p, 8)
                assert np.array_equal(s, os_) and v.tobytes() == ov.tobytes()
        finally:
            c.close()


def test_candidate_overflow_regrows(quality50k, mix50k, monkeypatch):
    """A candidate buffer of 16 per query overflows: the pass's end reports the largest count
    through the control block's host mirror, the buffer grows to it and the scan re-runs; the
    answer is the oracle's, and a second pass on the grown buffer needs no re-run."""
    _, queries, _ = mix50k
    ix = quality50k
    monkeypatch.setenv("MAIVS_GPU_CAND_CAP", "16")
    c = capi.Context(0)
    try:
        c.upload(ix._arena_desc())
        for nprobe in (12, 40):
            p = _params(ix, 10, nprobe)
            st = capi.GpuStats()
            s, v = c.search(queries, p, st)
            assert st.reruns >= 1, nprobe  # the 16-candidate buffer overflowed
            o_s, o_v = oracle.search_batch(ix._arena_desc(), queries, p, 8)
            assert np.array_equal(s, o_s) and v.tobytes() == o_v.tobytes()
            st2 = capi.GpuStats()
            s2, _ = c.search(queries, p, st2)
            assert np.array_equal(s2, s)
            assert st2.reruns == 0
    finally:
        c.close()


def test_counters_after_a_per_query_call(quality50k, mix50k):
    """After a per-query search the batched pass's seed cut-offs and work counters do not exist:
    last_counters / last_candidates report that instead of reading stale per-batch state, and a
    batched search afterwards reports its own counters again."""
    _, queries, _ = mix50k
    ix = quality50k
    c = capi.Context(0)
    try:
        c.upload(ix._arena_desc())
        p = _params(ix, 10, 16)
        c.search(queries[:200], p)          # batched: sets rest_end and the counters
        c.search_queries(queries[:7], _params(ix, 10, 600))  # per-query, a longer probe list
        with pytest.raises(capi.GpuError) as e:
            c.last_counters(capi.GpuStats())
        assert e.value.status == capi.ERR_UNSUPPORTED
        with pytest.raises(capi.GpuError):
            c.last_candidates(7, 1024)
        st = capi.GpuStats()
        c.search(queries[:200], p)
        c.last_counters(st)
        assert st.seed_blocks > 0 and st.rerank_rows > 0
    finally:
        c.close()


def test_small_arena_upload_keeps_larger_lds_limits(mix50k):
    """Uploading an arena with a small dimension on a second context must not lower the kernels'
    LDS limits that a larger arena's searches rely on: index A (d = 768) searched, index B (d = 64)
    uploaded elsewhere, then A searched again without a re-upload, equal to the oracle."""
    import maivs_amd as M
    from .conftest import small_clustered
    base, queries, _ = mix50k
    xa = np.ascontiguousarray(np.concatenate([base[:6000], base[6000:12000]], axis=1))
    xa /= np.linalg.norm(xa, axis=1, keepdims=True)
    qa = np.ascontiguousarray(np.concatenate([queries[:300], queries[300:600]], axis=1))
    qa /= np.linalg.norm(qa, axis=1, keepdims=True)
    ia = M.build_preset(xa.astype(np.float32), "quality")
    ib = M.build_preset(small_clustered(3000, 64), "quality")
    ca, cb = capi.Context(0), capi.Context(0)
    try:
        ca.upload(ia._arena_desc())
        p = _params(ia, 10, 24)
        s1, v1 = ca.search(qa, p)
        cb.upload(ib._arena_desc())
        cb.search(small_clustered(64, 64, seed=3), _params(ib, 10, 8))
        s2, v2 = ca.search(qa, p)
        o_s, o_v = oracle.search_batch(ia._arena_desc(), qa, p, 8)
        assert np.array_equal(s1, o_s) and v1.tobytes() == o_v.tobytes()
        assert np.array_equal(s2, o_s) and v2.tobytes() == o_v.tobytes()
    finally:
        ca.close()
        cb.close()


def test_upload_refuses_an_arena_without_cells(quality50k, mix50k):
    """An arena description with no cells is refused at upload with an argument error (every kernel
    indexes cell 0's code), and the context still uploads and searches a good arena afterwards."""
    import ctypes as C
    _, queries, _ = mix50k
    ix = quality50k
    bad = capi.ArenaDesc.from_buffer_copy(capi.ArenaDesc.from_address(ix._arena_desc()))
    bad.n_cells = 0
    c = capi.Context(0)
    try:
        with pytest.raises(capi.GpuError, match="no cells"):
            c.upload(C.addressof(bad))
        c.upload(ix._arena_desc())
        p = _params(ix, 10, 8)
        s, v = c.search(queries[:64], p)
        o_s, o_v = oracle.search_batch(ix._arena_desc(), queries[:64], p, 8)
        assert np.array_equal(s, o_s) and v.tobytes() == o_v.tobytes()
    finally:
        c.close()


def test_host_buffer_calls_grow_the_staging(quality50k, mix50k):
    """The host-buffer entry points stage queries and results through one pinned buffer that grows
    with the call: batches of rising and falling size on one context, through both entry points,
    each equal to the oracle."""
    _, queries, _ = mix50k
    ix = quality50k
    c = capi.Context(0)
    try:
        c.upload(ix._arena_desc())
        p = _params(ix, 10, 8)
        for n in (3, 64, 700, 5, 1000, 2):
            q = np.ascontiguousarray(queries[:n])
            s, v = c.search(q, p)
            o_s, o_v = oracle.search_batch(ix._arena_desc(), q, p, 8)
            assert np.array_equal(s, o_s) and v.tobytes() == o_v.tobytes(), n
            s, v = c.search_queries(q, p)
            o_s, o_v = oracle.search_one(ix._arena_desc(), q, p, nthreads=8)
            assert np.array_equal(s, o_s) and v.tobytes() == o_v.tobytes(), n
    finally:
        c.close()
