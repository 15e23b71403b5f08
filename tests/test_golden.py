"""Known-answer vectors (tests/golden/kat.npz, written by tests/golden/make_kat.py): the oracle
must keep reproducing them, and the GPU stage entry points must match them bit for bit."""
import os

import numpy as np
import pytest

import oracle

KAT = np.load(os.path.join(os.path.dirname(__file__), "golden", "kat.npz"))


def test_oracle_reproduces_kat():
    assert np.array_equal(oracle.make_signs(512, 0x5EED), KAT["signs"])
    for i, v in enumerate(KAT["q"]):
        r = oracle.rotate(v, KAT["signs"], 512)
        assert r.tobytes() == KAT["rot"][i].tobytes()
        assert np.array_equal(oracle.pack_signs(r, 8), KAT["bits"][i])
        lut, d, b = oracle.fs_query(r, 8)
        assert np.array_equal(lut, KAT["lut"][i])
        assert d.tobytes() == KAT["delta"][i].tobytes() and b.tobytes() == KAT["bias"][i].tobytes()
        assert np.array_equal(oracle.fs_block_sums(KAT["block"], lut), KAT["sums"][i])
    assert np.array_equal(oracle.fs_pack_block(KAT["codes"], 8), KAT["block"])
    for i in range(8):
        assert oracle.dot_f32(KAT["a"][i], KAT["q"][i % 4]).tobytes() == KAT["dots"][i].tobytes()
        assert oracle.dot_f32_u8(KAT["a"][i], KAT["u"][i]).tobytes() == KAT["dots_u8"][i].tobytes()


@pytest.mark.gpu
def test_gpu_block_sums_match_kat():
    from maivs_amd import capi
    ctx = capi.Context(0)
    try:
        blocks = np.repeat(KAT["block"][None, :], 4, axis=0)
        out = ctx.block_sums(blocks, KAT["lut"], 8)
        assert np.array_equal(out, KAT["sums"])
    finally:
        ctx.close()
