"""Seeded synthetic layers for the benchmark configurations.

numpy ``Generator(PCG64(seed))``; FP16 values by IEEE round-to-nearest-even.
Shapes, densities and distributions follow the five configurations the
benchmark is quoted on (in_features K -> out_features N, tokens M):

  c1  4096 -> 4096,  M=1, per-row scales, ortho 1 % uniform, alpha in {0, 1}
  c2  4096 -> 11008, M in {1,2,4,8,16}, group-128 scales, ortho 1 % uniform
  c3  4096 -> 4096,  M=2048, group-128, ortho 1 % uniform, alpha in {0, .5, 1}
  c4  4096 -> 14336, M=8, group-128, ortho 0.5 % in 41 outlier columns with
      Zipf(1.2) nonzeros per row (capped at 41), values N(0, 0.2)
  c5  Llama-2-7B block: q,k,v,o 4096->4096; gate,up 4096->11008;
      down 11008->4096; group-128, ortho 2 % uniform, M in {1, 32}

q is drawn directly as uniform integers in [-8, 7] (every packed byte
uniform in 0..255), scales |N(0, 0.02)|, ortho positions uniform without
replacement (exactly round(density*N*K) of them), ortho values N(0, 0.05)
with exact zeros redrawn, x N(0, 1).  Inputs are numpy arrays in the API
layout; ``to_device`` moves a layer to torch tensors.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np


@dataclass
class Layer:
    K: int
    N: int
    q: np.ndarray                 # uint8 [N, K/2]
    scales: np.ndarray            # float16 [N] or [N, K/G]
    row_ptr: np.ndarray           # int32 [N+1]
    col: np.ndarray               # int32 [nnz]
    vals: np.ndarray              # float16 [nnz]
    name: str = ""
    meta: Dict = field(default_factory=dict)

    @property
    def nnz(self) -> int:
        return int(self.vals.size)

    @property
    def groups(self) -> int:
        return 1 if self.scales.ndim == 1 else int(self.scales.shape[1])


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _f16_nonzero(rng, n: int, sigma: float) -> np.ndarray:
    v = rng.normal(0.0, sigma, size=n).astype(np.float16)
    bad = v == 0
    while bad.any():
        v[bad] = rng.normal(0.0, sigma, size=int(bad.sum())).astype(np.float16)
        bad = v == 0
    return v


def _csr_from_flat(flat: np.ndarray, N: int, K: int):
    flat = np.sort(flat.astype(np.int64))
    rows = flat // K
    cols = (flat % K).astype(np.int32)
    counts = np.bincount(rows, minlength=N)
    row_ptr = np.zeros(N + 1, np.int32)
    row_ptr[1:] = np.cumsum(counts)
    return row_ptr, cols


def make_layer(K: int, N: int, group: Optional[int], density: float, seed: int,
               val_sigma: float = 0.05, name: str = "") -> Layer:
    """Uniform-random ortho layer (configs c1, c2, c3, c5)."""
    rng = _rng(seed)
    q = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    sshape = (N,) if group is None else (N, K // group)
    scales = np.abs(rng.normal(0.0, 0.02, size=sshape)).astype(np.float16)
    nnz = int(round(density * N * K))
    flat = rng.choice(N * K, size=nnz, replace=False) if nnz else np.zeros(0, np.int64)
    row_ptr, col = _csr_from_flat(flat, N, K)
    vals = _f16_nonzero(rng, nnz, val_sigma)
    return Layer(K, N, q, scales, row_ptr, col, vals, name=name,
                 meta=dict(seed=seed, density=density, group=group or K))


def zipf_row_counts(rng, N: int, total: int, cap: int, s: float = 1.2) -> np.ndarray:
    """Per-row nonzero counts with a Zipf(s) profile, summing to ``total``,
    none above ``cap`` (overflow goes to uncapped rows)."""
    if total > N * cap:
        raise ValueError("total exceeds N * cap")
    raw = rng.zipf(s, size=N).astype(np.float64)
    lo, hi = 0.0, float(total) / raw.min() + 1.0
    for _ in range(200):  # bisection on the scale factor
        mid = 0.5 * (lo + hi)
        if np.minimum(cap, np.floor(raw * mid)).sum() > total:
            hi = mid
        else:
            lo = mid
    counts = np.minimum(cap, np.floor(raw * lo)).astype(np.int64)
    rem = total - int(counts.sum())
    frac = raw * lo - np.floor(raw * lo)
    order = np.lexsort((np.arange(N), -frac))
    i = 0
    while rem > 0:
        r = order[i % N]
        if counts[r] < cap:
            counts[r] += 1
            rem -= 1
        i += 1
    return counts


def make_skewed_layer(K: int, N: int, group: int, density: float, outlier_frac: float,
                      seed: int, val_sigma: float = 0.2, name: str = "") -> Layer:
    """Hessian-sieve-like ortho (config c4): all nonzeros in a few outlier
    input columns, Zipf-distributed per row."""
    rng = _rng(seed)
    q = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    scales = np.abs(rng.normal(0.0, 0.02, size=(N, K // group))).astype(np.float16)
    n_out = int(round(outlier_frac * K))
    outliers = np.sort(rng.choice(K, size=n_out, replace=False)).astype(np.int64)
    total = int(round(density * N * K))
    counts = zipf_row_counts(rng, N, total, n_out)
    flat = np.empty(total, np.int64)
    pos = 0
    for r in range(N):
        c = int(counts[r])
        if c:
            flat[pos:pos + c] = r * K + rng.choice(outliers, size=c, replace=False)
            pos += c
    row_ptr, col = _csr_from_flat(flat, N, K)
    vals = _f16_nonzero(rng, total, val_sigma)
    return Layer(K, N, q, scales, row_ptr, col, vals, name=name,
                 meta=dict(seed=seed, density=density, group=group, outliers=n_out))


def make_x(M: int, K: int, seed: int) -> np.ndarray:
    return _rng(seed).normal(0.0, 1.0, size=(M, K)).astype(np.float16)


# ----------------------------------------------------------------- configs

def config_layer(cfg: str, case: int = 0) -> Layer:
    """The layer of a benchmark configuration; seed = 1000*config + case."""
    c = int(cfg[1:])
    seed = 1000 * c + case
    if cfg == "c1":
        return make_layer(4096, 4096, None, 0.01, seed, name="c1")
    if cfg == "c2":
        return make_layer(4096, 11008, 128, 0.01, seed, name="c2")
    if cfg == "c3":
        return make_layer(4096, 4096, 128, 0.01, seed, name="c3")
    if cfg == "c4":
        return make_skewed_layer(4096, 14336, 128, 0.005, 0.01, seed, name="c4")
    raise ValueError(cfg)


LLAMA_BLOCK = [("q_proj", 4096, 4096), ("k_proj", 4096, 4096), ("v_proj", 4096, 4096),
               ("o_proj", 4096, 4096), ("gate_proj", 4096, 11008), ("up_proj", 4096, 11008),
               ("down_proj", 11008, 4096)]


def llama_block(case: int = 0) -> List[Layer]:
    """Config c5: the seven projections of one Llama-2-7B decoder block."""
    return [make_layer(K, N, 128, 0.02, 5000 + 10 * case + i, name=nm)
            for i, (nm, K, N) in enumerate(LLAMA_BLOCK)]


def algorithmic_bytes(layer: Layer, M: int, alpha: float, io_bytes: int = 2) -> int:
    """HBM bytes one forward must move at minimum, in the API layout:
    N*K/2 (packed q) + 2*N*K/G (fp16 scales) + [ortho on] (6*nnz + 4*(N+1))
    + io_bytes*M*K (x) + io_bytes*M*N (y)."""
    N, K = layer.N, layer.K
    b = N * K // 2 + layer.scales.size * 2 + io_bytes * M * K + io_bytes * M * N
    if alpha > 0 and layer.nnz > 0:
        b += 6 * layer.nnz + 4 * (N + 1)
    return int(b)


def algorithmic_flops(layer: Layer, M: int, alpha: float) -> int:
    f = 2 * M * layer.N * layer.K
    if alpha > 0 and layer.nnz > 0:
        f += 2 * M * layer.nnz
    return int(f)


def to_device(layer: Layer, device="cuda"):
    """torch tensors (q, scales, vals, col, row_ptr) on ``device``."""
    import torch
    return dict(
        q=torch.from_numpy(layer.q).to(device),
        scales=torch.from_numpy(layer.scales).to(device),
        vals=torch.from_numpy(layer.vals).to(device),
        col=torch.from_numpy(layer.col).to(device),
        row_ptr=torch.from_numpy(layer.row_ptr).to(device),
    )
