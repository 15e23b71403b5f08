"""The oracle (test infrastructure only): ctypes access to oracle/liboracle.so, the CPU
restatement of MAIVS's batched cell-major search. Imported by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the product.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from maivs_amd.capi import SearchParams

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
_lib = None

P, U32, U64, F32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_float
_SIGS = {
    "orc_make_signs": (None, [U32, U64, P]),
    "orc_fht": (None, [P, U32]),
    "orc_rotate": (None, [P, U32, P, U32, P]),
    "orc_pack_signs": (None, [P, U32, P, U32]),
    "orc_hamming": (U32, [P, P, U32]),
    "orc_fs_query": (None, [P, U32, U32, P, P, P]),
    "orc_fs_estimate": (F32, [F32, F32, U32]),
    "orc_fs_pack_block": (None, [P, U32, U32, P]),
    "orc_fs_unpack": (None, [P, U32, U32, P]),
    "orc_fs_block_sums": (None, [P, P, U32, P]),
    "orc_fs_block_sums_scalar": (None, [P, P, U32, P]),
    "orc_dot_f32": (F32, [P, P, U32]),
    "orc_dot_f32_u8": (F32, [P, P, U32]),
    "orc_hamming_cutoff": (U32, [P, P, U32, U32, U32]),
    "orc_route_batch": (C.c_int, [P, P, U32, C.POINTER(SearchParams), U32, P, P, P, P]),
    "orc_search_batch": (C.c_int, [P, P, U32, C.POINTER(SearchParams), U32, P, P]),
    "orc_last_candidates": (C.c_int, [P, P, P, P, P, P, U64]),
    "orc_last_total_candidates": (U64, []),
    "orc_set_record": (None, [C.c_int]),
    "orc_search_one": (C.c_int, [P, P, U32, C.POINTER(SearchParams), U32, P, P]),
    "orc_route_query": (C.c_int, [P, P, U32, C.POINTER(SearchParams), U32, P, P, P]),
    "orc_acosf_violations": (U64, [U32, P]),
}


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            from . import build_oracle
            build_oracle.build()
        L = C.CDLL(LIB_PATH)
        for n, (r, a) in _SIGS.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data


def make_signs(dim_pad: int, seed: int) -> np.ndarray:
    out = np.empty(2 * dim_pad, np.float32)
    lib().orc_make_signs(dim_pad, seed, _p(out))
    return out


def fht(a: np.ndarray) -> np.ndarray:
    a = np.array(a, np.float32, copy=True)
    lib().orc_fht(_p(a), len(a))
    return a


def rotate(v: np.ndarray, signs: np.ndarray, dim_pad: int) -> np.ndarray:
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty(dim_pad, np.float32)
    lib().orc_rotate(_p(v), len(v), _p(np.ascontiguousarray(signs, np.float32)), dim_pad, _p(out))
    return out


def pack_signs(rot: np.ndarray, nw: int) -> np.ndarray:
    rot = np.ascontiguousarray(rot, np.float32)
    out = np.empty(nw, np.uint64)
    lib().orc_pack_signs(_p(rot), len(rot), _p(out), nw)
    return out


def hamming(a: np.ndarray, b: np.ndarray) -> int:
    a = np.ascontiguousarray(a, np.uint64)
    b = np.ascontiguousarray(b, np.uint64)
    return lib().orc_hamming(_p(a), _p(b), len(a))


def fs_query(rq: np.ndarray, nw: int):
    rq = np.ascontiguousarray(rq, np.float32)
    lut = np.empty(nw * 256, np.uint8)
    delta, bias = C.c_float(), C.c_float()
    lib().orc_fs_query(_p(rq), len(rq), nw, _p(lut), C.addressof(delta), C.addressof(bias))
    return lut, np.float32(delta.value), np.float32(bias.value)


def fs_pack_block(codes: np.ndarray, nw: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.uint64).reshape(-1, nw)
    out = np.empty(nw * 256, np.uint8)
    lib().orc_fs_pack_block(_p(codes), codes.shape[0], nw, _p(out))
    return out


def fs_unpack(block: np.ndarray, lane: int, nw: int) -> np.ndarray:
    out = np.empty(nw, np.uint64)
    lib().orc_fs_unpack(_p(np.ascontiguousarray(block, np.uint8)), lane, nw, _p(out))
    return out


def fs_block_sums(block: np.ndarray, lut: np.ndarray, scalar: bool = False) -> np.ndarray:
    block = np.ascontiguousarray(block, np.uint8)
    lut = np.ascontiguousarray(lut, np.uint8)
    out = np.empty(32, np.uint16)
    f = lib().orc_fs_block_sums_scalar if scalar else lib().orc_fs_block_sums
    f(_p(block), _p(lut), len(block) // 32, _p(out))
    return out


def dot_f32(a, b) -> np.float32:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return np.float32(lib().orc_dot_f32(_p(a), _p(b), len(a)))


def dot_f32_u8(qs, v) -> np.float32:
    qs = np.ascontiguousarray(qs, np.float32)
    v = np.ascontiguousarray(v, np.uint8)
    return np.float32(lib().orc_dot_f32_u8(_p(qs), _p(v), len(qs)))


def hamming_cutoff(hs: np.ndarray, keep: np.ndarray, want: int, bits: int) -> int:
    hs = np.ascontiguousarray(hs, np.uint16)
    keep = np.ascontiguousarray(keep, np.uint8)
    return lib().orc_hamming_cutoff(_p(hs), _p(keep), len(hs), want, bits)


def route_batch(desc_addr: int, q: np.ndarray, params: SearchParams, n_words: int, nthreads: int = 8):
    q = np.ascontiguousarray(q, np.float32)
    nq = q.shape[0]
    qbits = np.empty((nq, n_words), np.uint64)
    chosen = np.empty((nq, params.nprobe), np.uint32)
    cscore = np.empty((nq, params.nprobe), np.float32)
    nchosen = np.empty(nq, np.uint32)
    rc = lib().orc_route_batch(C.c_void_p(desc_addr), _p(q), nq, C.byref(params), nthreads, _p(qbits), _p(chosen),
                               _p(cscore), _p(nchosen))
    if rc != 0:
        raise RuntimeError(f"orc_route_batch failed ({rc})")
    return qbits, chosen, cscore, nchosen


def search_batch(desc_addr: int, q: np.ndarray, params: SearchParams, nthreads: int = 8):
    q = np.ascontiguousarray(q, np.float32)
    nq = q.shape[0]
    slots = np.empty((nq, params.k), np.uint32)
    scores = np.empty((nq, params.k), np.float32)
    rc = lib().orc_search_batch(C.c_void_p(desc_addr), _p(q), nq, C.byref(params), nthreads, _p(slots), _p(scores))
    if rc != 0:
        raise RuntimeError(f"orc_search_batch failed ({rc})")
    return slots, scores


def search_one(desc_addr: int, q: np.ndarray, params: SearchParams, nthreads: int = 8):
    """The per-query path (route_query + search_one + rerank_exact) for every query."""
    q = np.ascontiguousarray(q, np.float32)
    nq = q.shape[0]
    slots = np.empty((nq, params.k), np.uint32)
    scores = np.empty((nq, params.k), np.float32)
    rc = lib().orc_search_one(C.c_void_p(desc_addr), _p(q), nq, C.byref(params), nthreads, _p(slots), _p(scores))
    if rc != 0:
        raise RuntimeError(f"orc_search_one failed ({rc})")
    return slots, scores


def route_query(desc_addr: int, q: np.ndarray, params: SearchParams, nthreads: int = 8):
    q = np.ascontiguousarray(q, np.float32)
    nq = q.shape[0]
    chosen = np.empty((nq, params.nprobe), np.uint32)
    cscore = np.empty((nq, params.nprobe), np.float32)
    nchosen = np.empty(nq, np.uint32)
    rc = lib().orc_route_query(C.c_void_p(desc_addr), _p(q), nq, C.byref(params), nthreads, _p(chosen), _p(cscore),
                               _p(nchosen))
    if rc != 0:
        raise RuntimeError(f"orc_route_query failed ({rc})")
    return chosen, cscore, nchosen


def last_candidates(nq: int):
    total = lib().orc_last_total_candidates()
    tau, rest_end, cut, ncand = (np.empty(nq, np.uint32) for _ in range(4))
    slots = np.empty(max(total, 1), np.uint32)
    dd = np.empty(max(total, 1), np.uint32)
    rc = lib().orc_last_candidates(_p(tau), _p(rest_end), _p(cut), _p(ncand), _p(slots), _p(dd), total)
    if rc != 0:
        raise RuntimeError("orc_last_candidates failed")
    return tau, rest_end, cut, ncand, slots[:total], dd[:total]


def set_record(on: bool) -> None:
    """Keep (True, the default) or skip each query's candidate list for last_candidates; the CPU
    baseline's timing runs skip it, as the reference keeps nothing of the kind."""
    lib().orc_set_record(1 if on else 0)


def acosf_violations(nthreads: int = 8):
    """(count, first x) of the f32 inputs in [-1, 1] where the host libm's acosf increases from one
    input to the next (none expected: the GPU radii rely on acosf being non-increasing)."""
    first = C.c_uint64(0)
    n = lib().orc_acosf_violations(nthreads, C.byref(first))
    return int(n), int(first.value)
