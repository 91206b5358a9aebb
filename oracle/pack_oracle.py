"""CPU oracle for the packing step in front of the dual GEMM (numpy).

TEST INFRASTRUCTURE ONLY.  The product path (``libortho_amd``) never imports
this module; only ``tests/`` may, as the checker of the device packer.

Restates, element by element in numpy:

* ``pack_base``: ``OrthoLinear.load_from_weights`` steps 1
  (/root/reference/torch_bind/ortho_linear.py:89-120): scales =
  clamp(max|W| / 7, min=1e-6) per row (or per group of ``group_size``
  columns), the FP16 copy stored, q = clamp(round(W / scales), -8, 7) with
  the scales as computed, nibbles of the flattened [N, K] array packed
  low = even index.
* ``pack_csr``: ``pack_ortho_sparse(W, "csr")``
  (/root/reference/tools/sieve.py:119-152): the entries W != 0 in row-major
  order, row_ptr = [0, cumsum(bincount(rows))], values in W's dtype.

Dtype semantics are those of torch's ops: arithmetic in FP32 rounded to the
tensor's dtype (FP16 or BF16, round to nearest even).  ``max|W| / 7.0``
divides by a Python scalar; torch computes that on a GPU tensor as a
multiplication by the FP32 reciprocal (``scale_div="reciprocal"``) and on a
CPU tensor as an IEEE division (``scale_div="ieee"``).  W / s promotes to
FP32 when W and given scales differ in dtype.  BF16 arrays are passed as
uint16 bit patterns with ``dtype="bf16"``.
"""
from __future__ import annotations

import numpy as np

DTYPES = ("f32", "f16", "bf16")


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """Round to nearest even (NaN kept as a quiet NaN)."""
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def as_f32(w: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_bits_to_f32(w)
    return np.asarray(w).astype(np.float32)


def round_to(dtype: str, v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, np.float32)
    if dtype == "f16":
        return v.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(v))
    return v


def pack_base(w: np.ndarray, dtype: str, group_size: int | None = None,
              scales: np.ndarray | None = None, scales_dtype: str | None = None,
              scale_div: str = "reciprocal"):
    """(q uint8 [N, K/2], scales float16 [N] or [N, K/G]) for dense w [N, K]."""
    assert dtype in DTYPES and scale_div in ("reciprocal", "ieee")
    N, K = w.shape
    G = K if not group_size else int(group_size)
    assert K % 2 == 0 and K % G == 0 and G % 2 == 0
    wf = as_f32(w, dtype)                      # exact values of w
    cells = wf.reshape(N, K // G, G)
    with np.errstate(invalid="ignore", over="ignore"):
        if scales is None:
            m = np.abs(cells).max(axis=2)          # NaN propagates
            if scale_div == "reciprocal":
                s = round_to(dtype, m * (np.float32(1.0) / np.float32(7.0)))
            else:
                s = round_to(dtype, m / np.float32(7.0))
            lo = round_to(dtype, np.float32(1e-6))
            s = np.where(s < lo, lo, s).astype(np.float32)
            prom = dtype
        else:
            sd = scales_dtype or dtype
            s = as_f32(np.asarray(scales).reshape(N, K // G), sd)
            prom = dtype if sd == dtype else "f32"
        v = round_to(prom, cells / s[:, :, None])  # IEEE FP32 division, then the dtype
        v = np.rint(v)
        v = np.clip(v, -8.0, 7.0)
        v = np.where(np.isnan(v), 0.0, v)          # (NaN weights: not a supported input)
    q = v.reshape(N, K).astype(np.int8).reshape(-1)
    packed = ((q[0::2].astype(np.uint8) & 0x0F) | ((q[1::2].astype(np.uint8) & 0x0F) << 4)).astype(np.uint8)
    s_out = s.astype(np.float16)
    if G == K:
        s_out = s_out.reshape(N)
    return packed.reshape(N, K // 2), s_out


def nonzero_mask(w: np.ndarray, dtype: str) -> np.ndarray:
    """w != 0 as the reference's mask: -0 is zero, NaN is not."""
    if dtype == "f32":
        return (np.asarray(w, np.float32).view(np.uint32) & 0x7FFFFFFF) != 0
    bits = np.asarray(w).view(np.uint16) if dtype == "f16" else np.asarray(w, np.uint16)
    return (bits & 0x7FFF) != 0


def pack_csr(w: np.ndarray, dtype: str):
    """(row_ptr int32 [N+1], col int32 [nnz], values [nnz] in w's dtype)."""
    N, K = w.shape
    mask = nonzero_mask(w, dtype)
    rows, cols = np.nonzero(mask)                  # row-major order
    row_ptr = np.zeros(N + 1, np.int64)
    row_ptr[1:] = np.cumsum(np.bincount(rows, minlength=N))
    return row_ptr.astype(np.int32), cols.astype(np.int32), np.asarray(w)[mask]
