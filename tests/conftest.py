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


def small_clustered(n=4000, d=64, n_clusters=40, seed=0):
    """Small clustered unit vectors (tests/test_index.py:51-95 style: Gaussian centres, noise)."""
    rs = np.random.RandomState(seed)
    cent = rs.standard_normal((n_clusters, d))
    cent /= np.linalg.norm(cent, axis=1, keepdims=True)
    lab = rs.randint(0, n_clusters, n)
    x = cent[lab] + 0.7 / np.sqrt(d) * rs.standard_normal((n, d))
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    return x.astype(np.float32)
