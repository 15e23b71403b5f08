"""Seeded anisotropic Gaussian-mixture workloads for the batched cell-major search.

The reference ships no generator for these mixtures (its test generator is
``tests/test_index.py:51-95``, an isotropic clustered set); the workloads below are the
ones the benchmark configurations name, built with ``numpy.random.RandomState`` because
numpy freezes that stream across versions.

A mixture with ``n_comp`` components in ``dim`` dimensions:

* component means ``mu_c = normalise(N(0, I))``;
* a per-dimension spectrum ``sigma_i = 1/sqrt(i+1)``, its order permuted per component;
* a draw ``x = normalise(mu_c + scale * (sigma_c * z) / ||sigma||)`` with ``z ~ N(0, I)``,
  ``c`` uniform over the components and ``scale = 0.35``.

Held-out queries are fresh draws from the same mixture with another seed. Shifted
queries (``memory``-preset workload) rotate the means by a Givens rotation of ``angle``
degrees in a random orthonormal plane, then add ``noise * g / sqrt(dim)`` and renormalise.

Ground truth is the exact top-k by float32 inner product, ties broken by the lower id
(the reference's ``bench/fair/prep_data.py:58-72`` computes the same top-k with numpy).
"""
from __future__ import annotations

import dataclasses

import numpy as np

SCALE = 0.35


@dataclasses.dataclass
class Mixture:
    means: np.ndarray  # (n_comp, dim) float64, unit rows
    sig: np.ndarray  # (n_comp, dim) float64, per-component permuted spectrum / ||sigma||


def make_mixture(n_comp: int, dim: int, seed: int) -> Mixture:
    rs = np.random.RandomState(seed)
    means = rs.standard_normal((n_comp, dim))
    means /= np.linalg.norm(means, axis=1, keepdims=True)
    spec = 1.0 / np.sqrt(np.arange(dim, dtype=np.float64) + 1.0)
    spec = spec / np.linalg.norm(spec)
    sig = np.empty((n_comp, dim))
    for c in range(n_comp):
        sig[c] = spec[rs.permutation(dim)]
    return Mixture(means, sig)


def draw(mix: Mixture, n: int, seed: int, *, means: np.ndarray | None = None,
         noise: float = 0.0, chunk: int = 65536) -> np.ndarray:
    """n unit-norm float32 vectors from the mixture (optionally with substituted means)."""
    rs = np.random.RandomState(seed)
    mu = mix.means if means is None else means
    n_comp, dim = mu.shape
    comp = rs.randint(0, n_comp, size=n)
    out = np.empty((n, dim), np.float32)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        c = comp[s:e]
        z = rs.standard_normal((e - s, dim))
        x = mu[c] + SCALE * mix.sig[c] * z
        if noise > 0.0:
            x += noise * rs.standard_normal((e - s, dim)) / np.sqrt(dim)
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        out[s:e] = x
    return out


def givens_rotated_means(mix: Mixture, angle_deg: float, seed: int) -> np.ndarray:
    """Means rotated by ``angle_deg`` in a random orthonormal plane (u, v)."""
    rs = np.random.RandomState(seed)
    dim = mix.means.shape[1]
    u = rs.standard_normal(dim)
    u /= np.linalg.norm(u)
    v = rs.standard_normal(dim)
    v -= u * (u @ v)
    v /= np.linalg.norm(v)
    th = np.deg2rad(angle_deg)
    m = mix.means
    a = m @ u
    b = m @ v
    ca, sa = np.cos(th), np.sin(th)
    rot = m + np.outer(a * (ca - 1.0) - b * sa, u) + np.outer(a * sa + b * (ca - 1.0), v)
    return rot / np.linalg.norm(rot, axis=1, keepdims=True)


# name -> (n_comp, n_base, n_query, mixture seed, base seed, query seed, shifted?)
WORKLOADS = {
    # 50k x 384, 512 components, 1,000 held-out queries (CPU-runnable case)
    "mix50k": dict(n_comp=512, n=50_000, nq=1_000, seeds=(101, 101, 102), shifted=False),
    # 500k x 384, 4,096 components, 1,000 in-distribution queries
    "mix500k": dict(n_comp=4096, n=500_000, nq=1_000, seeds=(201, 202, 203), shifted=False),
    # same base, 1,000 shifted queries (20 degree Givens rotation of the means + 0.15 noise)
    "mix500k-shift": dict(n_comp=4096, n=500_000, nq=1_000, seeds=(201, 202, 301), shifted=True),
    # 5.2M x 384, 16,384 components, 10,000 queries
    "mix5m": dict(n_comp=16384, n=5_200_000, nq=10_000, seeds=(401, 402, 403), shifted=False),
}


def workload(name: str, dim: int = 384, n: int | None = None, nq: int | None = None):
    """(base, queries) for a named workload; ``n``/``nq`` override the sizes (prefixes)."""
    w = WORKLOADS[name]
    n = w["n"] if n is None else n
    nq = w["nq"] if nq is None else nq
    sm, sb, sq = w["seeds"]
    mix = make_mixture(w["n_comp"], dim, sm)
    if sm == sb:
        # one stream for means and base: continue the mixture RNG past the spectra draws
        base = draw(mix, n, sm + 1_000_003)
    else:
        base = draw(mix, n, sb)
    if w["shifted"]:
        means = givens_rotated_means(mix, 20.0, 302)
        queries = draw(mix, nq, sq, means=means, noise=0.15)
    else:
        queries = draw(mix, nq, sq)
    return base, queries


def exact_topk(base: np.ndarray, queries: np.ndarray, k: int = 10, chunk: int = 131072,
               device: str | None = None) -> np.ndarray:
    """Exact top-k ids by float32 inner product, ties to the lower id.

    Uses torch on ``device`` when given (the GPU on the bench box), numpy otherwise.
    """
    nq = len(queries)
    if device is not None and nq * len(base) > 2_000_000_000:
        return _exact_topk_on_device(base, queries, k, device)
    best_s = np.full((nq, k), -np.inf, np.float32)
    best_i = np.full((nq, k), np.iinfo(np.int64).max, np.int64)
    if device is not None:
        import torch
        qt = torch.from_numpy(np.ascontiguousarray(queries)).to(device)
    for s in range(0, len(base), chunk):
        b = base[s:s + chunk]
        if device is not None:
            bt = torch.from_numpy(np.ascontiguousarray(b)).to(device)
            S = (qt @ bt.T).float().cpu().numpy()
        else:
            S = queries @ b.T
        kk = min(k, S.shape[1])
        idx = np.argpartition(-S, kk - 1, axis=1)[:, :kk]
        # widen to every column tied with the kk-th best so the lower id wins ties
        kth = np.take_along_axis(S, idx, 1).min(axis=1, keepdims=True)
        for qi in range(nq):
            cols = np.nonzero(S[qi] >= kth[qi])[0]
            cs = np.concatenate([best_s[qi], S[qi, cols]])
            ci = np.concatenate([best_i[qi], cols.astype(np.int64) + s])
            o = np.lexsort((ci, -cs))[:k]
            best_s[qi] = cs[o]
            best_i[qi] = ci[o]
    return best_i


def _exact_topk_on_device(base, queries, k, device, chunk=262144, qblk=2048):
    """exact_topk for large products, entirely on the device: per base chunk the k best of every
    query (torch.topk), merged with the running best by (score desc, id asc). An exact score tie
    that straddles a chunk's k-th place may keep either id (ties elsewhere go to the lower id)."""
    import torch
    nq = len(queries)
    qt = torch.from_numpy(np.ascontiguousarray(queries, np.float32)).to(device)
    bs = torch.full((nq, k), float("-inf"), device=device)
    bi = torch.full((nq, k), np.iinfo(np.int64).max, dtype=torch.int64, device=device)
    for s in range(0, len(base), chunk):
        bt = torch.from_numpy(np.ascontiguousarray(base[s:s + chunk], np.float32)).to(device)
        kk = min(k, bt.shape[0])
        for q0 in range(0, nq, qblk):
            q1 = min(nq, q0 + qblk)
            v, i = torch.topk(qt[q0:q1] @ bt.T, kk, dim=1)
            cs = torch.cat([bs[q0:q1], v], 1)
            ci = torch.cat([bi[q0:q1], i.to(torch.int64) + s], 1)
            o = torch.argsort(ci, dim=1, stable=True)
            cs, ci = torch.gather(cs, 1, o), torch.gather(ci, 1, o)
            o = torch.argsort(-cs, dim=1, stable=True)[:, :k]
            bs[q0:q1] = torch.gather(cs, 1, o)
            bi[q0:q1] = torch.gather(ci, 1, o)
        del bt
    return bi.cpu().numpy()


def recall_at(ids: np.ndarray, gt: np.ndarray, k: int = 10) -> float:
    """Mean |top-k ∩ gt-k| / k, as ``bench/fair/fairbench.py:46-48``."""
    ids = np.asarray(ids).reshape(len(gt), -1)[:, :k]
    hits = 0
    for a, b in zip(ids.tolist(), gt[:, :k].tolist()):
        hits += len(set(a) & set(b))
    return hits / (k * len(gt))
