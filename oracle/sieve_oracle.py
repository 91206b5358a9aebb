"""CPU oracle for the offline Base/Ortho sieve (numpy).

TEST INFRASTRUCTURE ONLY.  The product path (``libortho_amd``) never imports
this module; only ``tests/`` may, as the checker of the device sieve.

Restates, element by element in numpy, /root/reference/tools/sieve.py:

* ``quantize_int4`` (:13-23): m = max|w| per row (NaN propagates),
  clamp(m, min=1e-8) in w's dtype, s = m / 7, r = clamp(round(w / s), -8, 7)
  * s with round-half-even, non-finite results replaced by 0.
* ``hessian_sieve`` (:25-76): residual = w - w_base, score = residual^2 /
  (H_inv + 1e-6) (H_inv's diagonal when it is a matrix), threshold = the
  k-th largest score for ``sparsity_target`` (NaN largest, as torch.topk;
  k = 0 keeps nothing) or ``curvature_thresh`` (compared in the score's dtype,
  as torch compares a tensor with a host scalar); w_ortho = residual * (score
  > threshold).
* ``compute_hessian_diag_approx`` (:79-95): diag(X^T X) / n + 1e-6, the
  diagonal as FP64 column sums of squares rounded to X's dtype.

Dtype semantics are those of torch's elementwise ops: arithmetic in FP32
rounded to the tensor's dtype.  ``m / 7.0`` and ``d / n`` divide by a host
scalar, which torch computes on a GPU tensor as a multiplication by the FP32
reciprocal (``scalar_div="reciprocal"``) and on a CPU tensor as an IEEE
division (``scalar_div="ieee"``).  Arrays hold FP32 values that are exact in
the stated dtype (FP16/BF16 values widened).
"""
from __future__ import annotations

import numpy as np

from .pack_oracle import round_to

_PROMOTE = {("f32", "f32"): "f32", ("f16", "f16"): "f16", ("bf16", "bf16"): "bf16"}


def promote(a: str, b: str) -> str:
    """torch.promote_types for the three float dtypes."""
    return _PROMOTE.get((a, b), "f32")


def _scalar_div(dtype: str, v: np.ndarray, d: float, scalar_div: str) -> np.ndarray:
    if scalar_div == "reciprocal":
        return round_to(dtype, v * (np.float32(1.0) / np.float32(d)))
    return round_to(dtype, v / np.float32(d))


def quantize_int4(w: np.ndarray, dtype: str, scalar_div: str = "reciprocal") -> np.ndarray:
    """FP32 values of quantize_int4(w) (each exactly representable in w's dtype)."""
    wf = np.asarray(w, np.float32)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        m = np.abs(wf).max(axis=1, keepdims=True)          # NaN propagates
        lo = round_to(dtype, np.float32(1e-8))
        m = np.where(np.isnan(m), m, np.maximum(m, lo)).astype(np.float32)
        s = _scalar_div(dtype, m, 7.0, scalar_div)
        t = np.rint(round_to(dtype, wf / s))
        t = np.where(np.isnan(t), t, np.clip(t, -8.0, 7.0)).astype(np.float32)
        r = round_to(dtype, t * s)
    return np.where(np.isfinite(r), r, np.float32(0.0)).astype(np.float32)


def _kth_largest(score: np.ndarray, k: int) -> np.float32:
    flat = score.reshape(-1)
    nan = np.isnan(flat)
    n_nan = int(nan.sum())
    if k <= n_nan:
        return np.float32(np.nan)
    rest = np.sort(flat[~nan])[::-1]
    return rest[k - n_nan - 1]


def hessian_sieve(w: np.ndarray, dtype: str, h_inv: np.ndarray, h_dtype: str, curvature_thresh: float = 10.0,
                  sparsity_target: float | None = None, scalar_div: str = "reciprocal"):
    """(w_base, w_ortho) as FP32 arrays of values in w's dtype."""
    wf = np.asarray(w, np.float32)
    wb = quantize_int4(w, dtype, scalar_div)
    h = np.asarray(h_inv, np.float32)
    if h.ndim > 1:
        h = np.diag(h)
    sdt = promote(dtype, h_dtype)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        res = round_to(dtype, wf - wb)
        hs = round_to(h_dtype, h + np.float32(1e-6))
        score = round_to(sdt, round_to(dtype, res * res) / hs[None, :])
        if sparsity_target is not None:
            k = int(sparsity_target * score.size)
            thr = _kth_largest(score, k) if k > 0 else np.float32(np.nan)
        else:
            thr = round_to(sdt, np.float32(curvature_thresh))  # the host scalar in the score's dtype
        keep = score > thr
        wo = round_to(dtype, res * keep.astype(np.float32))
    return wb, wo, score


def compute_hessian_diag_approx(x: np.ndarray, dtype: str, scalar_div: str = "reciprocal") -> np.ndarray:
    xf = np.asarray(x, np.float32).astype(np.float64)
    n = xf.shape[0]
    d = round_to(dtype, (xf * xf).sum(axis=0).astype(np.float32))
    q = _scalar_div(dtype, d, float(n), scalar_div)
    return round_to(dtype, q + np.float32(1e-6))
