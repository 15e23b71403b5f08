import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmaivs_gpu.so's C ABI)")
    config.addinivalue_line("markers", "slow: builds the 500k-vector workload")


def pytest_collection_modifyitems(config, items):
    # GPU tests need a visible device; on a CPU-only machine they are skipped, not failed.
    try:
        import torch
        have = torch.cuda.device_count() > 0
    except Exception:
        have = False
    if have:
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def mix50k():
    """The 50k x 384 mixture (512 components) with 1,000 held-out queries and exact top-10."""
    from maivs_amd import mixture
    base, queries = mixture.workload("mix50k")
    gt = mixture.exact_topk(base, queries, 10)
    return base, queries, gt


@pytest.fixture(scope="session")
def quality50k(mix50k):
    import maivs_amd as M
    base, _, _ = mix50k
    return M.build_preset(base, "quality")


@pytest.fixture(scope="session")
def memory50k(mix50k):
    import maivs_amd as M
    base, _, _ = mix50k
    return M.build_preset(base, "memory")


@pytest.fixture(scope="session")
def churn50k(mix50k):
    """The update-and-filter workload at 50k (the 400k churn + filter workload's shape): 40k initial
    vectors, 5 rounds of (delete 2k random initial ids, insert 2k new vectors), compact(), then a
    tag in [0, 1000) per id (bench/fair/churn.py:29,47-61; bench/fair/filtered.py:33).
    Returns (index, tag of every id, live ids)."""
    import maivs_amd as M
    base, _, _ = mix50k
    n0, nnew, rounds = 40_000, 10_000, 5
    ix = M.build_preset(base[:n0], "quality")
    dele = np.random.RandomState(501).choice(n0, nnew, replace=False)
    per = nnew // rounds
    for r in range(rounds):
        for i in dele[r * per:(r + 1) * per]:
            assert ix.remove(int(i))
        lo = n0 + r * per
        ix.add_batch(list(range(lo, lo + per)), np.ascontiguousarray(base[lo:lo + per]))
    ix.compact()
    gone = set(dele.tolist())
    live = [i for i in range(n0 + nnew) if i not in gone]
    tags = np.random.RandomState(502).randint(0, 1000, n0 + nnew).astype(np.uint32)
    ix.set_tags(live, [int(tags[i]) for i in live])
    return ix, tags, live


def small_clustered(n=4000, d=64, n_clusters=40, seed=0):
    """Small clustered unit vectors (tests/test_index.py:51-95 style: Gaussian centres, noise)."""
    rs = np.random.RandomState(seed)
    cent = rs.standard_normal((n_clusters, d))
    cent /= np.linalg.norm(cent, axis=1, keepdims=True)
    lab = rs.randint(0, n_clusters, n)
    x = cent[lab] + 0.7 / np.sqrt(d) * rs.standard_normal((n, d))
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    return x.astype(np.float32)
