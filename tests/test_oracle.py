"""Pins for the oracle (CPU restatement of the reference search path), checked against what the
mathematics fixes rather than against a retyped formula:

* splitmix64 signs: the published splitmix64 test vector, then bit-for-bit low bits;
* FWHT / rotation: the explicit Sylvester Hadamard matrix in float64, orthonormality,
  inner-product preservation (src/quantize.rs:449-472);
* sign codes, Hamming, FastScan layout and sums: brute force from the definitions, starting
  from the u64 codes (a different path than the oracle's packed blocks);
* the FastScan table: the estimator bound |sum*delta + bias - <Rq, s(x)>| <= 128*delta/2;
* the 8-lane FMA dots: an exact-rational emulation (every FMA rounded once from the exact
  value), which fixes the hsum association and where the FMA sits;
* routing, the candidate set and the rerank: brute-force enumeration on real indexes.
"""
from fractions import Fraction

import numpy as np
import pytest
from scipy.linalg import hadamard

import oracle
from maivs_amd import capi

M64 = (1 << 64) - 1


def splitmix64(seed, n):
    s, out = seed, []
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & M64
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        out.append(z ^ (z >> 31))
    return out


def test_splitmix64_published_vector():
    # Vigna's splitmix64 reference output for seed 1234567
    assert splitmix64(1234567, 5) == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                                      4593380528125082431, 16408922859458223821]


@pytest.mark.parametrize("seed", [0x5EED, 42, 1234567, 0])
@pytest.mark.parametrize("dim_pad", [64, 512])
def test_make_signs(seed, dim_pad):
    got = oracle.make_signs(dim_pad, seed)
    want = np.array([1.0 if (z & 1) == 0 else -1.0 for z in splitmix64(seed, 2 * dim_pad)], np.float32)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n", [8, 64, 512, 1024])
def test_fht_is_normalised_hadamard(n):
    rs = np.random.RandomState(n)
    x = rs.standard_normal(n).astype(np.float32)
    want = hadamard(n).astype(np.float64) @ x.astype(np.float64) / np.sqrt(n)
    got = oracle.fht(x)
    assert np.allclose(got, want, atol=1e-5, rtol=0)
    # orthonormal and self-inverse
    assert abs(float(np.dot(got, got)) - float(np.dot(x, x))) < 1e-3
    assert np.allclose(oracle.fht(got), x, atol=1e-5)


def test_rotate_matches_dense_operator_and_preserves_inner_products():
    dim, dim_pad = 384, 512
    signs = oracle.make_signs(dim_pad, 0x5EED)
    H = hadamard(dim_pad).astype(np.float64) / np.sqrt(dim_pad)
    D1, D2 = np.diag(signs[:dim_pad].astype(np.float64)), np.diag(signs[dim_pad:].astype(np.float64))
    R = H @ D2 @ H @ D1
    rs = np.random.RandomState(3)
    a = rs.standard_normal(dim).astype(np.float32)
    b = rs.standard_normal(dim).astype(np.float32)
    pa = np.zeros(dim_pad)
    pa[:dim] = a
    ra, rb = oracle.rotate(a, signs, dim_pad), oracle.rotate(b, signs, dim_pad)
    assert np.allclose(ra, R @ pa, atol=1e-5)
    assert abs(float(np.dot(ra, rb)) - float(np.dot(a, b))) < 1e-3


def test_pack_signs_and_hamming_bruteforce():
    rs = np.random.RandomState(5)
    for nw in (1, 4, 8):
        x = rs.standard_normal(nw * 64).astype(np.float32)
        x[::17] = 0.0
        x[1::23] = -0.0  # -0.0 < 0 is false: bit stays 0
        bits = oracle.pack_signs(x, nw)
        want = np.zeros(nw, np.uint64)
        for i in range(nw * 64):
            if x[i] < 0:
                want[i >> 6] |= np.uint64(1) << np.uint64(i & 63)
        assert np.array_equal(bits, want)
        y = oracle.pack_signs(rs.standard_normal(nw * 64).astype(np.float32), nw)
        naive = sum(bin(int(p) ^ int(q)).count("1") for p, q in zip(bits, y))
        assert oracle.hamming(bits, y) == naive


def _nibbles(code_words):
    """128 nibbles of a 512-bit code from the u64 words (nibble j at word j>>4, bits 4(j&15))."""
    out = []
    for j in range(len(code_words) * 16):
        out.append((int(code_words[j >> 4]) >> (4 * (j & 15))) & 0xF)
    return out


def test_fs_pack_unpack_roundtrip_and_sums_bruteforce():
    rs = np.random.RandomState(11)
    nw = 8
    for ncodes in (32, 17, 1):
        codes = rs.randint(0, 2 ** 63, size=(ncodes, nw), dtype=np.int64).astype(np.uint64)
        codes ^= rs.randint(0, 2, size=(ncodes, nw)).astype(np.uint64) << np.uint64(63)
        blk = oracle.fs_pack_block(codes, nw)
        for lane in range(32):
            got = oracle.fs_unpack(blk, lane, nw)
            want = codes[lane] if lane < ncodes else np.zeros(nw, np.uint64)
            assert np.array_equal(got, want)
        lut = rs.randint(0, 256, size=nw * 256).astype(np.uint8)
        avx = oracle.fs_block_sums(blk, lut)
        scalar = oracle.fs_block_sums(blk, lut, scalar=True)
        want = np.zeros(32, np.int64)
        for lane in range(ncodes):
            want[lane] = sum(int(lut[j * 16 + nb]) for j, nb in enumerate(_nibbles(codes[lane])))
        want[ncodes:] = sum(int(lut[j * 16]) for j in range(nw * 16))  # missing lanes are code 0
        assert np.array_equal(avx.astype(np.int64), want)
        assert np.array_equal(scalar, avx)
    # the largest possible sum, 255 * 128, fits in u16
    blk = np.zeros(2048, np.uint8)
    assert oracle.fs_block_sums(blk, np.full(2048, 255, np.uint8)).max() == 32640


def test_fs_query_estimator_bound():
    rs = np.random.RandomState(13)
    signs = oracle.make_signs(512, 0x5EED)
    for _ in range(20):
        q = rs.standard_normal(384).astype(np.float32)
        q /= np.linalg.norm(q)
        rq = oracle.rotate(q, signs, 512)
        lut, delta, bias = oracle.fs_query(rq, 8)
        assert delta > 0
        tab = lut.reshape(128, 16)
        assert tab.min(axis=1).max() == 0  # every position's minimum entry quantises to 0
        assert tab.max() == 255  # the widest position spans the full u8 range
        for _ in range(10):
            x = rs.standard_normal(384).astype(np.float32)
            code = oracle.pack_signs(oracle.rotate(x, signs, 512), 8)
            nibs = _nibbles(code)
            ssum = sum(int(tab[j, nb]) for j, nb in enumerate(nibs))
            s = np.array([-1.0 if (int(code[i >> 6]) >> (i & 63)) & 1 else 1.0 for i in range(512)])
            exact = float(np.dot(rq.astype(np.float64), s))
            est = float(oracle.lib().orc_fs_estimate(float(delta), float(bias), ssum))
            assert abs(est - exact) <= 64.0 * float(delta) + 1e-4


def _fwht_textbook_f32(x):
    """The textbook iterative FWHT in float32: levels h = 1, 2, 4, ..., n/2 in ascending order,
    butterflies (u + v, u - v), then one multiply by 1/sqrt(n) computed in f32. Butterflies of one
    level are independent, so only the level order fixes the rounding; the reference states its
    8-block form is bit-identical to this loop (src/quantize.rs:73-75, 103-121)."""
    a = np.array(x, np.float32).copy()
    n = len(a)
    h = 1
    while h < n:
        v = a.reshape(-1, 2, h)
        u, w = v[:, 0, :].copy(), v[:, 1, :].copy()
        v[:, 0, :] = u + w
        v[:, 1, :] = u - w
        h *= 2
    s = np.float32(1.0) / np.sqrt(np.float32(n))
    return a * s


def _fwht_descending_f32(x):
    a = np.array(x, np.float32).copy()
    n = len(a)
    h = n // 2
    while h >= 1:
        v = a.reshape(-1, 2, h)
        u, w = v[:, 0, :].copy(), v[:, 1, :].copy()
        v[:, 0, :] = u + w
        v[:, 1, :] = u - w
        h //= 2
    return a * (np.float32(1.0) / np.sqrt(np.float32(n)))


@pytest.mark.parametrize("n", [8, 16, 64, 512, 1024])
def test_fht_bit_identical_to_textbook_level_order(n):
    rs = np.random.RandomState(100 + n)
    for trial in range(8):
        x = (rs.standard_normal(n) * (10.0 ** rs.randint(-3, 4))).astype(np.float32)
        got = oracle.fht(x)
        want = _fwht_textbook_f32(x)
        assert got.tobytes() == want.tobytes(), (n, trial)
    # the check can tell level orders apart: on these inputs a descending-level transform,
    # equal in exact arithmetic, rounds differently somewhere
    if n >= 64:
        x = rs.standard_normal(n).astype(np.float32)
        assert _fwht_descending_f32(x).tobytes() != oracle.fht(x).tobytes()


def test_rotate_is_two_rounds_of_textbook_fwht():
    """rotate = copy + zero-pad, then twice (multiply by the round's signs, FWHT)
    (src/quantize.rs:152-163), bit for bit."""
    signs = oracle.make_signs(512, 0x5EED)
    rs = np.random.RandomState(17)
    for _ in range(4):
        q = rs.standard_normal(384).astype(np.float32)
        x = np.zeros(512, np.float32)
        x[:384] = q
        for r in range(2):
            x = _fwht_textbook_f32(x * signs[r * 512:(r + 1) * 512])
        assert oracle.rotate(q, signs, 512).tobytes() == x.tobytes()


def test_fs_query_every_entry_within_half_a_step():
    """Every table entry is the nearest integer to (raw - min_j) / delta: |lut * delta - (raw - min_j)|
    <= delta / 2 (with the division's own rounding as slack), raw being the 4-term sign sum of the
    position (src/quantize.rs:279-308), recomputed here in float64 from rq."""
    rs = np.random.RandomState(19)
    signs = oracle.make_signs(512, 0x5EED)
    for _ in range(10):
        q = rs.standard_normal(384).astype(np.float32)
        rq = oracle.rotate(q, signs, 512)
        lut, delta, bias = oracle.fs_query(rq, 8)
        d = float(delta)
        tab = lut.reshape(128, 16).astype(np.float64)
        x = rq.astype(np.float64).reshape(128, 4)
        e = np.arange(16)
        sgn = np.where(((e[:, None] >> np.arange(4)[None, :]) & 1) == 1, -1.0, 1.0)  # (16, 4)
        raw = x @ sgn.T  # (128, 16)
        mins = raw.min(axis=1, keepdims=True)
        err = np.abs(tab * d - (raw - mins))
        assert err.max() <= 0.5 * d * (1 + 1e-5) + 1e-6
        # bias = the sum of the per-position minima, to within an f32 running sum's error bound
        bound = 128 * np.finfo(np.float32).eps * float(np.abs(mins).sum())
        assert abs(float(bias) - float(mins.sum())) <= bound


def test_fs_query_rounds_half_away_from_zero():
    """(raw - min) / delta exactly k + 1/2 rounds up (Rust's f32::round, src/quantize.rs:302), which
    a round-half-to-even (rint) slip would not. Position 0 spans 255 (x = 127.5), so delta = 1.0
    exactly; position 1 holds x = (1.25, 0.25), whose raw - min values are 0, 0.5, 2.5 and 3.0."""
    rq = np.zeros(64, np.float32)
    rq[0] = 127.5
    rq[4], rq[5] = 1.25, 0.25
    lut, delta, bias = oracle.fs_query(rq, 1)
    assert float(delta) == 1.0
    tab = lut.reshape(16, 16)  # nw = 1: 16 positions; position j = 2p + half at p*32 + half*16
    # position 0: raw = +-127.5 -> entries 0 / 255
    assert tab[0, 0] == 255 and tab[0, 1] == 0
    # position 1, e = bits of (t0, t1): raw = (+-1.25) + (+-0.25), min = -1.5
    want = {0: 3, 1: 1, 2: 3, 3: 0}  # 3.0 -> 3, 0.5 -> 1 (rint: 0), 2.5 -> 3 (rint: 2), 0 -> 0
    for e_lo, v in want.items():
        for hi in range(4):  # t2, t3 carry x = 0
            assert tab[1, e_lo | (hi << 2)] == v, (e_lo, hi)
    assert float(bias) == -127.5 - 1.5


def test_product_signs_are_the_splitmix64_stream():
    """The index's own rotation signs (what the product uploads and the GPU rotates with) are
    splitmix64's stream from the index seed: +1 for an even output, -1 for an odd one, two rounds
    of dim_pad (src/quantize.rs:132-148)."""
    import maivs_amd as M
    for seed, dim, pad in ((0x5EED, 384, 512), (7, 64, 64), (123456789, 100, 128)):
        ix = M.FlatCellIndex(dim, "binary", 8, seed)
        got = np.asarray(ix._rot_signs(), np.float32)
        want = np.array([1.0 if (z & 1) == 0 else -1.0 for z in splitmix64(seed, 2 * pad)], np.float32)
        assert got.shape == want.shape and np.array_equal(got, want), seed


# ---- exact-rational emulation of the 8-lane FMA dots ----

def _f32_round(v: Fraction) -> np.float32:
    f = np.float32(float(v))
    best = None
    for c in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        err = abs(Fraction(float(c)) - v)
        key = (err, int(np.array(c, np.float32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return np.float32(best[1])


def _fma(a, b, c):
    return _f32_round(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def _dot8_exact(a, b):
    n = len(a)
    acc = [np.float32(0.0)] * 8
    n8 = n - n % 8
    for i in range(0, n8, 8):
        for lane in range(8):
            acc[lane] = _fma(a[i + lane], b[i + lane], acc[lane])
    f = np.float32
    r = f(f(f(acc[0] + acc[4]) + f(acc[2] + acc[6])) + f(f(acc[1] + acc[5]) + f(acc[3] + acc[7])))
    for i in range(n8, n):
        r = f(r + f(f(a[i]) * f(b[i])))
    return r


@pytest.mark.parametrize("n", [384, 64, 13])
def test_dot_f32_exact_emulation(n):
    rs = np.random.RandomState(n)
    for t in range(25):
        a = rs.standard_normal(n).astype(np.float32)
        b = rs.standard_normal(n).astype(np.float32)
        if t % 5 == 0:  # heavy cancellation makes the association visible
            a[: n // 2] *= 1e4
            b[n // 2:] *= -1e4
        got = oracle.dot_f32(a, b)
        assert got.tobytes() == _dot8_exact(a, b).tobytes()


def test_dot_f32_u8_exact_emulation():
    rs = np.random.RandomState(99)
    for _ in range(25):
        qs = (rs.standard_normal(384) * 1e-3).astype(np.float32)
        v = rs.randint(0, 256, 384).astype(np.uint8)
        got = oracle.dot_f32_u8(qs, v)
        assert got.tobytes() == _dot8_exact(qs, v.astype(np.float32)).tobytes()


def test_hamming_cutoff_bruteforce():
    rs = np.random.RandomState(1)
    for _ in range(50):
        n = rs.randint(1, 300)
        hs = rs.randint(0, 40, n).astype(np.uint16)
        keep = (rs.rand(n) < 0.8).astype(np.uint8)
        live = np.sort(hs[keep == 1])
        want = int(rs.randint(0, max(len(live), 1) + 1))
        got = oracle.hamming_cutoff(hs, keep, want, 512)
        if want == 0:
            assert got == 0
        elif want > len(live):
            assert got == 512
        else:
            assert got == live[want - 1]


# ---- routing, candidate set and rerank by brute force on a real index ----

def _route_bruteforce(arr, q, nprobe, mult, tc, beta):
    nw, M, d = arr["n_words"], arr["n_cells"], arr["dim"]
    live = np.diff(arr["mem_off"]) > 0
    rq = oracle.rotate(q, arr["rot_signs"], arr["dim_pad"])
    qb = oracle.pack_signs(rq, nw)
    cb = arr["cent_bits"].reshape(M, nw)
    h = np.array([sum(bin(int(x) ^ int(y)).count("1") for x, y in zip(qb, cb[c])) for c in range(M)])
    want_c = min(nprobe * max(mult, 2), int(live.sum()))
    lh = np.sort(h[live])
    cut = lh[want_c - 1]
    sl = [c for c in range(M) if live[c] and h[c] <= cut]
    cqs = (q * arr["csq_step"]).astype(np.float32)
    base = np.float32(0.0)
    for j in range(d):
        base = np.float32(base + np.float32(q[j] * arr["csq_min"][j]))
    sq8 = arr["cent_sq8"].reshape(M, d)
    sc = [np.float32(oracle.dot_f32_u8(cqs, sq8[c]) + base) for c in sl]
    order = sorted(range(len(sl)), key=lambda i: (-float(sc[i]), sl[i]))[: min(nprobe, len(sl))]
    chosen = [sl[i] for i in order]
    scores = [sc[i] for i in order]
    if tc < 1.0 and chosen:
        mx = scores[0]
        ex = [np.float32(np.exp(np.float32((s - mx) * np.float32(beta)))) for s in scores]
        z = np.float32(-0.0)
        for e in ex:
            z = np.float32(z + e)
        cum, n = np.float32(0.0), len(chosen)
        for i, e in enumerate(ex):
            cum = np.float32(cum + np.float32(e / np.float32(z + np.float32(1e-9))))
            if cum >= tc:
                n = i + 1
                break
        chosen, scores = chosen[:n], scores[:n]
    return qb, chosen, scores


@pytest.mark.parametrize("nprobe,tc", [(16, 1.0), (3, 1.0), (64, 1.0), (16, 0.9)])
def test_route_batch_bruteforce(quality50k, mix50k, nprobe, tc):
    _, queries, _ = mix50k
    ix = quality50k
    arr = ix._arena_arrays()
    p = capi.params_from_bytes(ix._search_params(10, nprobe, tc, 8.0))
    qs = queries[:40]
    qbits, ch, cs, nch = oracle.route_batch(ix._arena_desc(), qs, p, arr["n_words"], nthreads=4)
    for i, q in enumerate(qs):
        qb, chosen, scores = _route_bruteforce(arr, q, nprobe, p.shortlist_mult, tc, 8.0)
        assert np.array_equal(qbits[i], qb)
        assert int(nch[i]) == len(chosen), i
        assert list(ch[i, : nch[i]]) == chosen, i
        assert cs[i, : nch[i]].tobytes() == np.array(scores, np.float32).tobytes(), i


def _all_nibbles(codes_u64):
    """(N, 16*W) nibbles of N codes: nibble j = byte j//2 of the little-endian code, low half if j even."""
    by = np.ascontiguousarray(codes_u64).view(np.uint8).reshape(codes_u64.shape[0], -1)
    nib = np.empty((by.shape[0], by.shape[1] * 2), np.uint8)
    nib[:, 0::2] = by & 0xF
    nib[:, 1::2] = by >> 4
    return nib


@pytest.mark.parametrize("nprobe,rf,filt", [(16, 8, None), (4, 32, None), (64, 4, None), (16, 8, (0, 99)),
                                             (32, 8, (0, 9)), (8, 16, (250, 749))])
def test_candidate_set_and_rerank_bruteforce(quality50k, mix50k, nprobe, rf, filt):
    """U(q) = canonical members of the scanned cells that pass the tag filter (keep!); candidates
    = {d <= G}, G the target-th smallest d; top-k = best exact scores (src/index.rs:1428-1439,
    2036-2045, 2155-2160, 2277-2311)."""
    _, queries, _ = mix50k
    ix = quality50k
    ix.set_rerank_factor(rf)
    ext = ix._ext_ids()
    tags = np.random.RandomState(502).randint(0, 1000, len(ext)).astype(np.uint32)
    if filt is not None:
        ix.set_tags([int(x) for x in ext], [int(t) for t in tags])
        ix.set_filter(*filt)
    try:
        arr = ix._arena_arrays()
        nibs = _all_nibbles(ix._codes().reshape(-1, arr["n_words"]))
        npos = nibs.shape[1]
        p = capi.params_from_bytes(ix._search_params(10, nprobe, 1.0, 8.0))
        qs = queries[:12]
        slots, scores = oracle.search_batch(ix._arena_desc(), qs, p, nthreads=4)
        tau, rest_end, cut, ncand, cs, cd = oracle.last_candidates(len(qs))
        _, ch, _, nch = oracle.route_batch(ix._arena_desc(), qs, p, arr["n_words"], nthreads=4)
        target = 10 * rf
        maxk = 255 * npos
        sc = arr["slot_cells"].reshape(-1, arr["max_assign"])
        vecs = arr["vecs_f32"].reshape(-1, arr["dim"])
        pos = 0
        for i, q in enumerate(qs):
            chosen = [int(c) for c in ch[i, : nch[i]]]
            probed = set(chosen)
            ns = min(8, len(chosen))
            rq = oracle.rotate(q, arr["rot_signs"], arr["dim_pad"])
            tab = oracle.fs_query(rq, arr["n_words"])[0].reshape(npos, 16).astype(np.int64)
            U, seed = [], []
            for rank, c in enumerate(chosen[: rest_end[i]]):
                mem = arr["members"][arr["mem_off"][c]: arr["mem_off"][c + 1]].astype(np.int64)
                dd = maxk - tab[np.arange(npos)[None, :], nibs[mem]].sum(axis=1)
                for slot, d in zip(mem.tolist(), dd.tolist()):
                    if filt is not None and not (filt[0] <= tags[slot] <= filt[1]):
                        continue  # keep!: tag outside the filter range
                    if any(h != 0xFFFFFFFF and h < c and h in probed for h in sc[slot].tolist()):
                        continue  # scored at a lower-id probed home
                    U.append((d, slot))
                    if rank < ns:
                        seed.append(d)
            seed.sort()
            assert tau[i] == (seed[target - 1] if len(seed) >= target else maxk)
            ds = sorted(d for d, _ in U)
            G = ds[target - 1] if len(ds) >= target else maxk
            want = sorted(x for x in U if x[0] <= G)
            got = [(int(a), int(b)) for a, b in zip(cd[pos: pos + ncand[i]], cs[pos: pos + ncand[i]])]
            pos += ncand[i]
            assert got == want, i
            assert cut[i] == G
            # rerank: exact f64 scores of the candidates; the oracle's top-k are the best ones
            ex = sorted(((float(np.dot(q.astype(np.float64), vecs[s].astype(np.float64))), s) for _, s in want),
                        key=lambda t: (-t[0], t[1]))
            kk = min(10, len(ex))
            assert np.allclose([e for e, _ in ex[:kk]], scores[i][:kk], rtol=1e-5, atol=1e-6)
            clear = kk == len(ex) or ex[kk - 1][0] - ex[kk][0] > 1e-5
            if clear:
                assert sorted(s for _, s in ex[:kk]) == sorted(int(s) for s in slots[i][:kk])
            if filt is not None:
                got_slots = [int(s) for s in slots[i] if s != 0xFFFFFFFF]
                assert all(filt[0] <= tags[s] <= filt[1] for s in got_slots)
    finally:
        ix.set_rerank_factor(32)
        ix.set_filter()


def test_adaptive_cut_matches_double_precision(quality50k, mix50k):
    """rest_end from f64 acos/cos agrees with the oracle's libm f32 wherever no suffix bound
    lies within 1e-5 of the threshold (src/index.rs:2166-2188)."""
    import math
    _, queries, _ = mix50k
    ix = quality50k
    arr = ix._arena_arrays()
    p = capi.params_from_bytes(ix._search_params(10, 64, 1.0, 8.0))
    qs = queries[:200]
    oracle.search_batch(ix._arena_desc(), qs, p, nthreads=4)
    tau, rest_end, _, _, _, _ = oracle.last_candidates(len(qs))
    _, ch, cs, nch = oracle.route_batch(ix._arena_desc(), qs, p, arr["n_words"], nthreads=4)
    norm = np.float32(np.sqrt(np.float32(2.0 * arr["dim_pad"]) / np.float32(math.pi)))
    checked = 0
    for i, q in enumerate(qs):
        rq = oracle.rotate(q, arr["rot_signs"], arr["dim_pad"])
        _, delta, bias = oracle.fs_query(rq, arr["n_words"])
        n = int(nch[i])
        ns = min(8, n)
        if tau[i] == 255 * 128 or ns >= n:
            assert rest_end[i] == n
            continue
        est = np.float32(np.float32(delta * np.float32(255 * 128 - int(tau[i]))) + bias)
        thr = np.float32(min(max(np.float32(est / norm), -1.0), 1.0))
        T = float(np.float32(thr - np.float32(p.at_margin)))
        suffix, best, rest = [], -np.inf, n
        for j in range(n - 1, ns - 1, -1):
            c = float(np.clip(cs[i, j], -1, 1))
            b = math.cos(max(math.acos(c) - float(arr["r_bound"][ch[i, j]]), 0.0))
            best = max(best, b)
            suffix.append((j, best))
        near = any(abs(s - T) < 1e-5 for _, s in suffix)
        for j, s in sorted(suffix):
            if s < T:
                rest = j
                break
        if not near:
            assert rest_end[i] == rest, i
            checked += 1
    assert checked > 100


def test_host_acosf_is_non_increasing_on_every_f32_in_unit_interval():
    """The GPU build's radii select the p99-th largest member dot on the device and take acos of it
    on the host; that equals the reference's p99-th smallest angle exactly when the host's acosf is
    non-increasing on [-1, 1]. Checked for every f32 there (2.1e9 inputs)."""
    n, first = oracle.acosf_violations(8)
    assert n == 0, hex(first)
