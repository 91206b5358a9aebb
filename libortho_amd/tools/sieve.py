"""The reference's ``tools.sieve`` (/root/reference/tools/sieve.py): the
offline Base/Ortho split and the sparse packing of the Ortho component.

``pack_ortho_sparse`` has the contract of /root/reference/tools/sieve.py:98-177:

  format="csr" -> (row_ptr int32 [N+1], col_indices int32 [nnz], values [nnz])
      nonzeros of ``w_ortho`` (exact zeros dropped, :123) in row-major order,
      columns ascending within a row (:131-136), row_ptr = [0, cumsum of the
      per-row counts] (:140-146); values keep ``w_ortho``'s dtype.
  format="coo" -> (flat uint16 indices row*K+col, values, None), deprecated
      (:153-175).  Like the reference, the flat index is kept modulo 2**16,
      so it only addresses matrices of at most 65536 elements.
  anything else -> ValueError.

On a ROCm GPU the CSR is built by the library's packing kernels
(``_C_ops.pack_csr``, same result bit for bit); elsewhere by torch ops
(``torch.nonzero`` already lists coordinates in row-major order, so no sort
is needed).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch


def pack_ortho_sparse(w_ortho: torch.Tensor, format: str = "csr"
                      ) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    if w_ortho.dim() != 2:
        raise ValueError(f"w_ortho must be 2-D [out_features, in_features], got {tuple(w_ortho.shape)}")
    if format == "csr" and w_ortho.is_cuda and w_ortho.dtype in (torch.float16, torch.bfloat16, torch.float32):
        from .. import _C_ops
        return _C_ops.pack_csr(w_ortho)
    return pack_ortho_sparse_torch(w_ortho, format)


def pack_ortho_sparse_torch(w_ortho: torch.Tensor, format: str = "csr"):
    """The torch-op form of ``pack_ortho_sparse`` on any device."""
    out_features, in_features = w_ortho.shape
    mask = w_ortho != 0
    coords = torch.nonzero(mask, as_tuple=False)  # row-major order
    rows, cols = coords[:, 0], coords[:, 1]
    values = w_ortho[mask]
    if format == "csr":
        counts = torch.bincount(rows, minlength=out_features)
        row_ptr = torch.zeros(out_features + 1, dtype=torch.int32, device=w_ortho.device)
        row_ptr[1:] = torch.cumsum(counts, dim=0).to(torch.int32)
        return row_ptr, cols.to(torch.int32), values
    if format == "coo":
        flat = (rows * in_features + cols) & 0xFFFF
        return flat.to(torch.int32).to(torch.uint16), values, None
    raise ValueError(f"Unsupported format: {format}. Use 'csr' or 'coo'")


# ------------------------------------------------------------ offline sieve

def quantize_int4_torch(weight: torch.Tensor) -> torch.Tensor:
    """The torch-op form of ``quantize_int4`` (/root/reference/tools/sieve.py:13-23):
    per-row scale max|w| (clamped at 1e-8) / 7, round-half-even of w / s
    clamped to [-8, 7], times s; non-finite results become 0."""
    max_vals = weight.abs().max(dim=1, keepdim=True)[0].clamp(min=1e-8)
    scales = max_vals / 7.0
    result = (weight / scales).round().clamp(-8, 7) * scales
    return torch.where(torch.isfinite(result), result, torch.zeros_like(result))


def hessian_sieve_torch(weight: torch.Tensor, H_inv: torch.Tensor, curvature_thresh: float = 10.0,
                        sparsity_target: Optional[float] = None):
    """The torch-op form of ``hessian_sieve`` (/root/reference/tools/sieve.py:25-76)."""
    w_base = quantize_int4_torch(weight)
    residual = weight - w_base
    if H_inv.dim() > 1:
        H_inv = torch.diag(H_inv)
    score = (residual ** 2) / (H_inv + 1e-6).unsqueeze(0)
    if sparsity_target is not None:
        k = int(sparsity_target * score.numel())
        threshold = torch.topk(score.flatten(), k, largest=True).values[-1] if k > 0 else score.max() + 1.0
    else:
        threshold = curvature_thresh
    return w_base, residual * (score > threshold)


def compute_hessian_diag_approx_torch(inputs: torch.Tensor, outputs: Optional[torch.Tensor] = None):
    """The torch-op form of ``compute_hessian_diag_approx``
    (/root/reference/tools/sieve.py:79-95): diag(X^T X) / n + 1e-6."""
    n = inputs.shape[0]
    return torch.diag(torch.matmul(inputs.T, inputs)) / n + 1e-6


def _sieve_on_device(t: torch.Tensor) -> bool:
    return t.is_cuda and t.dtype in (torch.float16, torch.bfloat16, torch.float32)


def quantize_int4(weight: torch.Tensor) -> torch.Tensor:
    """Per-row INT4 fake quantisation, /root/reference/tools/sieve.py:13-23."""
    if weight.dim() == 2 and _sieve_on_device(weight):
        from .. import _C_ops
        return _C_ops.sieve_quantize(weight)
    return quantize_int4_torch(weight)


def hessian_sieve(weight: torch.Tensor, H_inv: torch.Tensor, curvature_thresh: float = 10.0,
                  sparsity_target: Optional[float] = None):
    """Base/Ortho split, /root/reference/tools/sieve.py:25-76: (w_base,
    w_ortho) with w_base = quantize_int4(weight) and w_ortho the residual
    where residual^2 / (H_inv + 1e-6) exceeds the threshold (the k-th
    largest score for ``sparsity_target``, else ``curvature_thresh``)."""
    if weight.dim() == 2 and _sieve_on_device(weight) and H_inv.is_cuda and \
            H_inv.dtype in (torch.float16, torch.bfloat16, torch.float32) and H_inv.dim() in (1, 2):
        from .. import _C_ops
        return _C_ops.sieve_split(weight, H_inv, curvature_thresh, sparsity_target)
    return hessian_sieve_torch(weight, H_inv, curvature_thresh, sparsity_target)


def compute_hessian_diag_approx(inputs: torch.Tensor, outputs: Optional[torch.Tensor] = None):
    """diag(X^T X) / n + 1e-6, /root/reference/tools/sieve.py:79-95."""
    if inputs.dim() == 2 and _sieve_on_device(inputs):
        from .. import _C_ops
        return _C_ops.sieve_hdiag(inputs)
    return compute_hessian_diag_approx_torch(inputs, outputs)
