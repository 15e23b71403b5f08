"""Writes tests/golden/kat.npz: small known-answer vectors for the search path's arithmetic.

The reference ships no golden vectors for this path (its FastScan tests need an external corpus),
so these are produced by the oracle and accepted only after the independent checks below pass:
the published splitmix64 vector, the dense Hadamard operator in float64, the FastScan estimator
bound and a brute-force nibble sum. Re-run: python tests/golden/make_kat.py
"""
import os
import sys

import numpy as np
from scipy.linalg import hadamard

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle  # noqa: E402


def main():
    rs = np.random.RandomState(20261201)
    dim, P, nw = 384, 512, 8
    signs = oracle.make_signs(P, 0x5EED)
    q = rs.standard_normal((4, dim)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    H = hadamard(P) / np.sqrt(P)
    R = H @ np.diag(signs[P:].astype(np.float64)) @ H @ np.diag(signs[:P].astype(np.float64))
    rot, bits, lut, delta, bias = [], [], [], [], []
    for v in q:
        r = oracle.rotate(v, signs, P)
        pv = np.zeros(P)
        pv[:dim] = v
        assert np.allclose(r, R @ pv, atol=1e-5)
        b = oracle.pack_signs(r, nw)
        t, dl, bs = oracle.fs_query(r, nw)
        rot.append(r), bits.append(b), lut.append(t), delta.append(dl), bias.append(bs)
    codes = rs.randint(0, 2 ** 62, size=(32, nw), dtype=np.int64).astype(np.uint64)
    block = oracle.fs_pack_block(codes, nw)
    sums = np.stack([oracle.fs_block_sums(block, t) for t in lut])
    for t, s in zip(lut, sums):
        for lane in range(32):
            nib = [(int(codes[lane][j >> 4]) >> (4 * (j & 15))) & 0xF for j in range(128)]
            assert s[lane] == sum(int(t[j * 16 + n]) for j, n in enumerate(nib))
    a = rs.standard_normal((8, dim)).astype(np.float32)
    u = rs.randint(0, 256, (8, dim)).astype(np.uint8)
    dots = np.array([oracle.dot_f32(a[i], q[i % 4]) for i in range(8)], np.float32)
    dots_u8 = np.array([oracle.dot_f32_u8(a[i], u[i]) for i in range(8)], np.float32)
    np.savez_compressed(os.path.join(HERE, "kat.npz"), signs=signs, q=q, rot=np.array(rot), bits=np.array(bits),
                        lut=np.array(lut), delta=np.array(delta, np.float32), bias=np.array(bias, np.float32),
                        codes=codes, block=block, sums=sums, a=a, u=u, dots=dots, dots_u8=dots_u8)
    print("wrote", os.path.join(HERE, "kat.npz"))


if __name__ == "__main__":
    main()
