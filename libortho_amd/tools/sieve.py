"""Sparse packing of the Ortho component.

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
