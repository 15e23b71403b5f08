"""ctypes mirror of the C ABI in ``include/maivs_gpu.h`` (libmaivs_gpu.so).

This is the binding a maintainer would write on the reference side (the Rust equivalent is
in the integration notes); tests and the benchmark use it to call the boundary directly.
Loading fails loudly when the library is missing: there is no CPU path behind it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("MAIVS_GPU_LIB", os.path.join(HERE, "libmaivs_gpu.so"))

MAIVS_OK = 0
OK, ERR_ARG, ERR_NOT_UPLOADED, ERR_HIP, ERR_OOM, ERR_UNSUPPORTED = 0, -1, -2, -3, -4, -5
STATUS = {0: "ok", -1: "bad argument", -2: "arena not uploaded", -3: "HIP error", -4: "out of memory",
          -5: "unsupported"}
RERANK_F32, RERANK_SQ8 = 0, 1


class ArenaDesc(C.Structure):
    _fields_ = [
        ("dim", C.c_uint32), ("dim_pad", C.c_uint32), ("n_words", C.c_uint32), ("n_cells", C.c_uint32),
        ("n_slots", C.c_uint32), ("max_assign", C.c_uint32), ("rerank_mode", C.c_uint32),
        ("reserved0", C.c_uint32),
        ("fs_codes", C.c_void_p), ("fs_off", C.c_void_p), ("mem_off", C.c_void_p), ("members", C.c_void_p),
        ("slot_cells", C.c_void_p), ("cent_bits", C.c_void_p), ("cent_sq8", C.c_void_p),
        ("centroids", C.c_void_p), ("csq_min", C.c_void_p), ("csq_step", C.c_void_p), ("r_bound", C.c_void_p),
        ("rot_signs", C.c_void_p), ("vecs_f32", C.c_void_p), ("sq8_codes", C.c_void_p), ("sq_min", C.c_void_p),
        ("sq_step", C.c_void_p), ("tags", C.c_void_p), ("tree", C.c_void_p), ("slot_codes", C.c_void_p),
        ("store_token", C.c_uint64),
    ]


class SearchParams(C.Structure):
    _fields_ = [
        ("k", C.c_uint32), ("nprobe", C.c_uint32), ("target_confidence", C.c_float), ("beta", C.c_float),
        ("rerank_factor", C.c_uint32), ("shortlist_mult", C.c_uint32), ("adaptive", C.c_uint32),
        ("at_margin", C.c_float), ("filter", C.c_uint32), ("tag_lo", C.c_uint32), ("tag_hi", C.c_uint32),
        ("route_mode", C.c_uint32),
    ]


class GpuStats(C.Structure):
    _fields_ = [
        ("ms_total", C.c_float), ("ms_prep", C.c_float), ("ms_route", C.c_float), ("ms_seed", C.c_float),
        ("ms_invert", C.c_float), ("ms_scan", C.c_float), ("ms_select", C.c_float), ("ms_rerank", C.c_float),
        ("scan_pairs", C.c_uint64), ("scan_blocks", C.c_uint64), ("seed_blocks", C.c_uint64),
        ("survivors", C.c_uint64), ("rerank_rows", C.c_uint64), ("host_checks", C.c_uint32),
        ("host_fixes", C.c_uint32), ("reruns", C.c_uint32), ("reserved", C.c_uint32),
    ]

    def as_dict(self) -> dict:
        return {f: getattr(self, f) for f, _ in self._fields_ if f != "reserved"}


# every entry point the header declares, with its ctypes signature
P = C.c_void_p
U32, U64, F32, I32 = C.c_uint32, C.c_uint64, C.c_float, C.c_int
SIGNATURES = {
    "maivs_gpu_create": (I32, [I32, C.POINTER(P)]),
    "maivs_gpu_destroy": (None, [P]),
    "maivs_gpu_last_error": (C.c_char_p, [P]),
    "maivs_gpu_upload_arena": (I32, [P, P]),
    "maivs_gpu_search_batch": (I32, [P, P, U32, C.POINTER(SearchParams), P, P, C.POINTER(GpuStats)]),
    "maivs_gpu_search_batch_device": (I32, [P, P, U32, C.POINTER(SearchParams), P, P, C.POINTER(GpuStats)]),
    "maivs_gpu_search_batch_device_noalloc": (I32, [P, P, U32, C.POINTER(SearchParams), P, P, C.POINTER(GpuStats)]),
    "maivs_gpu_query_prep": (I32, [P, P, U32, P, P, P, P]),
    "maivs_gpu_block_sums": (I32, [P, U32, P, P, U32, P]),
    "maivs_gpu_route": (I32, [P, P, U32, C.POINTER(SearchParams), P, P, P]),
    "maivs_gpu_last_candidates": (I32, [P, P, P, P, P, P, P, U64]),
    "maivs_gpu_last_counters": (I32, [P, C.POINTER(GpuStats)]),
    "maivs_gpu_search_queries": (I32, [P, P, U32, C.POINTER(SearchParams), P, P, C.POINTER(GpuStats)]),
    "maivs_gpu_search_queries_device": (I32, [P, P, U32, C.POINTER(SearchParams), P, P, C.POINTER(GpuStats)]),
    "maivs_gpu_kmeans": (I32, [P, P, U64, U32, P, P, U32, P, P]),
    "maivs_gpu_place": (I32, [P, P, P, U32, P, P, P]),
    "maivs_gpu_store_reset": (I32, [P, U32, U32, U32]),
    "maivs_gpu_store_info": (I32, [P, P, P]),
    "maivs_gpu_store_radii": (I32, [P, P, P, P]),
    "maivs_gpu_store_compact": (I32, [P, P, U32, U32, P, P, P, P, P, P, P]),
}

_lib = None


def load() -> C.CDLL:
    """Load libmaivs_gpu.so (RuntimeError with the reason when it cannot be loaded)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run python -m maivs_amd.build)")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def ptr(a: np.ndarray) -> int:
    return a.ctypes.data if a is not None else 0


class GpuError(RuntimeError):
    def __init__(self, status: int, what: str, msg: str):
        super().__init__(f"{what} failed ({STATUS.get(status, status)}): {msg}")
        self.status = status


class Context:
    """One maivs_gpu_ctx (device, arena)."""

    def __init__(self, device: int = 0):
        self.lib = load()
        h = C.c_void_p()
        rc = self.lib.maivs_gpu_create(device, C.byref(h))
        if rc != 0:
            raise GpuError(rc, "maivs_gpu_create", "")
        self.h = h

    def _check(self, rc: int, what: str) -> None:
        if rc != 0:
            raise GpuError(rc, what, (self.lib.maivs_gpu_last_error(self.h) or b"").decode())

    def close(self) -> None:
        if getattr(self, "h", None):
            self.lib.maivs_gpu_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def upload(self, desc_addr: int) -> None:
        self._check(self.lib.maivs_gpu_upload_arena(self.h, C.c_void_p(desc_addr)), "maivs_gpu_upload_arena")

    def search(self, q: np.ndarray, params: SearchParams, stats: GpuStats | None = None):
        q = np.ascontiguousarray(q, np.float32)
        nq = q.shape[0]
        slots = np.empty((nq, params.k), np.uint32)
        scores = np.empty((nq, params.k), np.float32)
        self._check(self.lib.maivs_gpu_search_batch(self.h, ptr(q), nq, C.byref(params), ptr(slots), ptr(scores),
                                                    C.byref(stats) if stats is not None else None),
                    "maivs_gpu_search_batch")
        return slots, scores

    def search_device(self, q_ptr: int, nq: int, params: SearchParams, slots_ptr: int, scores_ptr: int,
                      stats: GpuStats | None = None) -> None:
        self._check(self.lib.maivs_gpu_search_batch_device(self.h, C.c_void_p(q_ptr), nq, C.byref(params),
                                                           C.c_void_p(slots_ptr), C.c_void_p(scores_ptr),
                                                           C.byref(stats) if stats is not None else None),
                    "maivs_gpu_search_batch_device")

    def search_device_noalloc(self, q_ptr: int, nq: int, params: SearchParams, slots_ptr: int, scores_ptr: int,
                              stats: GpuStats | None = None) -> None:
        """maivs_gpu_search_batch_device_noalloc: device buffers, no device allocation."""
        self._check(self.lib.maivs_gpu_search_batch_device_noalloc(self.h, C.c_void_p(q_ptr), nq, C.byref(params),
                                                                   C.c_void_p(slots_ptr), C.c_void_p(scores_ptr),
                                                                   C.byref(stats) if stats is not None else None),
                    "maivs_gpu_search_batch_device_noalloc")

    def search_queries(self, q: np.ndarray, params: SearchParams, stats: GpuStats | None = None):
        """The per-query path (maivs_gpu_search_queries)."""
        q = np.ascontiguousarray(q, np.float32)
        nq = q.shape[0]
        slots = np.empty((nq, params.k), np.uint32)
        scores = np.empty((nq, params.k), np.float32)
        self._check(self.lib.maivs_gpu_search_queries(self.h, ptr(q), nq, C.byref(params), ptr(slots), ptr(scores),
                                                      C.byref(stats) if stats is not None else None),
                    "maivs_gpu_search_queries")
        return slots, scores

    def search_queries_device(self, q_ptr: int, nq: int, params: SearchParams, slots_ptr: int, scores_ptr: int,
                              stats: GpuStats | None = None) -> None:
        self._check(self.lib.maivs_gpu_search_queries_device(self.h, C.c_void_p(q_ptr), nq, C.byref(params),
                                                             C.c_void_p(slots_ptr), C.c_void_p(scores_ptr),
                                                             C.byref(stats) if stats is not None else None),
                    "maivs_gpu_search_queries_device")

    def query_prep(self, q: np.ndarray, n_words: int):
        q = np.ascontiguousarray(q, np.float32)
        nq = q.shape[0]
        bits = np.empty((nq, n_words), np.uint64)
        lut = np.empty((nq, n_words * 256), np.uint8)
        delta = np.empty(nq, np.float32)
        bias = np.empty(nq, np.float32)
        self._check(self.lib.maivs_gpu_query_prep(self.h, ptr(q), nq, ptr(bits), ptr(lut), ptr(delta), ptr(bias)),
                    "maivs_gpu_query_prep")
        return bits, lut, delta, bias

    def block_sums(self, blocks: np.ndarray, luts: np.ndarray, n_words: int) -> np.ndarray:
        blocks = np.ascontiguousarray(blocks, np.uint8)
        luts = np.ascontiguousarray(luts, np.uint8)
        nb = blocks.shape[0]
        out = np.empty((nb, 32), np.uint16)
        self._check(self.lib.maivs_gpu_block_sums(self.h, n_words, ptr(blocks), ptr(luts), nb, ptr(out)),
                    "maivs_gpu_block_sums")
        return out

    def route(self, q: np.ndarray, params: SearchParams):
        q = np.ascontiguousarray(q, np.float32)
        nq = q.shape[0]
        chosen = np.empty((nq, params.nprobe), np.uint32)
        cscore = np.empty((nq, params.nprobe), np.float32)
        nchosen = np.empty(nq, np.uint32)
        self._check(self.lib.maivs_gpu_route(self.h, ptr(q), nq, C.byref(params), ptr(chosen), ptr(cscore),
                                             ptr(nchosen)), "maivs_gpu_route")
        return chosen, cscore, nchosen

    def last_counters(self, stats: GpuStats) -> GpuStats:
        self._check(self.lib.maivs_gpu_last_counters(self.h, C.byref(stats)), "maivs_gpu_last_counters")
        return stats

    def last_candidates(self, nq: int, cap: int):
        tau, rest_end, cut, ncand = (np.empty(nq, np.uint32) for _ in range(4))
        slots = np.empty(cap, np.uint32)
        dd = np.empty(cap, np.uint32)
        self._check(self.lib.maivs_gpu_last_candidates(self.h, ptr(tau), ptr(rest_end), ptr(cut), ptr(ncand),
                                                       ptr(slots), ptr(dd), cap), "maivs_gpu_last_candidates")
        return tau, rest_end, cut, ncand, slots, dd


def params_from_bytes(b: bytes) -> SearchParams:
    p = SearchParams()
    C.memmove(C.byref(p), b, C.sizeof(p))
    return p
