"""maivs_gpu_search_batch_device_noalloc (no device allocation; work buffers carved from a fixed
per-GPU array) against maivs_gpu_search_batch_device on the same device buffers: slots and score
bits identical, on two calls in a row, the second with a smaller input, and the context's own
entry point unchanged afterwards."""
import numpy as np
import pytest

import oracle
from maivs_amd import capi

pytestmark = pytest.mark.gpu


def _params(ix, k, nprobe, tc=1.0, beta=8.0):
    return capi.params_from_bytes(ix._search_params(k, nprobe, tc, beta))


def _run(ctx, fn, q_dev, p):
    import torch
    nq = q_dev.shape[0]
    slots = torch.empty((nq, p.k), dtype=torch.int32, device="cuda:0")
    scores = torch.empty((nq, p.k), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    st = capi.GpuStats()
    fn(q_dev.data_ptr(), nq, p, slots.data_ptr(), scores.data_ptr(), st)
    return slots.cpu().numpy().view(np.uint32), scores.cpu().numpy(), st


def test_noalloc_matches_device_entry_point(quality50k, mix50k):
    import torch
    _, queries, _ = mix50k
    ix = quality50k
    c = capi.Context(0)
    try:
        c.upload(ix._arena_desc())
        # call 1: 1,000 queries at nprobe 40 (the cell-major scan runs; the batch is larger than the
        # array holds at this index, so it runs in chunks); call 2: 300 queries at nprobe 12
        for nq, nprobe, rf in ((1000, 40, 16), (300, 12, 8)):
            ix.set_rerank_factor(rf)
            p = _params(ix, 10, nprobe)
            q = torch.from_numpy(np.ascontiguousarray(queries[:nq])).to("cuda:0")
            s_ref, v_ref, _ = _run(c, c.search_device, q, p)
            s_na, v_na, st = _run(c, c.search_device_noalloc, q, p)
            assert np.array_equal(s_na, s_ref), (nq, nprobe)
            assert v_na.tobytes() == v_ref.tobytes(), (nq, nprobe)
            assert st.ms_total > 0
            # and both equal the oracle
            o_s, o_v = oracle.search_batch(ix._arena_desc(), queries[:nq], p, 8)
            assert np.array_equal(s_na, o_s) and v_na.tobytes() == o_v.tobytes()
            # the context's own buffers were left alone: its entry point gives the same again
            s_again, v_again, _ = _run(c, c.search_device, q, p)
            assert np.array_equal(s_again, s_ref) and v_again.tobytes() == v_ref.tobytes()
    finally:
        ix.set_rerank_factor(32)
        c.close()
