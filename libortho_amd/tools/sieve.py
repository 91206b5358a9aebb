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

The offline sieve (``quantize_int4``, ``hessian_sieve``,
``compute_hessian_diag_approx``) always runs the library's kernels
(orth_sieve.hip).  A CPU tensor is copied to the current ROCm GPU, split
there with the arithmetic torch uses on CPU tensors (IEEE division by the
host scalars), and the results are copied back; without a ROCm GPU, or for
dtypes other than float16 / bfloat16 / float32, these functions raise.
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

_SIEVE_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _sieve_device(*tensors: torch.Tensor):
    """The GPU the sieve runs on and whether the inputs came from the CPU
    (then torch's CPU arithmetic is reproduced and results are copied back)."""
    for t in tensors:
        if t.dtype not in _SIEVE_DTYPES:
            raise TypeError(f"the sieve kernels take float16, bfloat16 or float32 tensors, got {t.dtype}")
    first = tensors[0]
    if first.is_cuda:
        return first.device, False
    if first.device.type != "cpu":
        raise RuntimeError(f"the sieve runs on a ROCm GPU; tensors on {first.device} are not supported")
    if not torch.cuda.is_available():
        raise RuntimeError("the sieve runs on the library's GPU kernels: a CPU tensor needs a ROCm GPU to be "
                           "split on (none is available)")
    return torch.device("cuda", torch.cuda.current_device()), True


def _require_2d(t: torch.Tensor, what: str) -> None:
    if t.dim() != 2:
        raise ValueError(f"{what} must be 2-D, got shape {tuple(t.shape)}")


def quantize_int4(weight: torch.Tensor) -> torch.Tensor:
    """Per-row INT4 fake quantisation, /root/reference/tools/sieve.py:13-23:
    s = clamp(max|w|, 1e-8) / 7 per row, clamp(round(w / s), -8, 7) * s,
    non-finite results 0; same dtype, shape and device as ``weight``."""
    from .. import _C_ops
    _require_2d(weight, "weight")
    dev, from_cpu = _sieve_device(weight)
    out = _C_ops.sieve_quantize(weight.to(dev), ieee_div=from_cpu)
    return out.cpu() if from_cpu else out


def hessian_sieve(weight: torch.Tensor, H_inv: torch.Tensor, curvature_thresh: float = 10.0,
                  sparsity_target: Optional[float] = None):
    """Base/Ortho split, /root/reference/tools/sieve.py:25-76: (w_base,
    w_ortho) with w_base = quantize_int4(weight) and w_ortho the residual
    where residual^2 / (H_inv + 1e-6) exceeds the threshold (the k-th
    largest score for ``sparsity_target``, else ``curvature_thresh``);
    H_inv is a vector or a matrix whose diagonal is used."""
    from .. import _C_ops
    _require_2d(weight, "weight")
    if H_inv.dim() not in (1, 2):
        raise ValueError(f"H_inv must be 1-D or 2-D, got shape {tuple(H_inv.shape)}")
    dev, from_cpu = _sieve_device(weight, H_inv)
    wb, wo = _C_ops.sieve_split(weight.to(dev), H_inv.to(dev), curvature_thresh, sparsity_target,
                                ieee_div=from_cpu)
    return (wb.cpu(), wo.cpu()) if from_cpu else (wb, wo)


def compute_hessian_diag_approx(inputs: torch.Tensor, outputs: Optional[torch.Tensor] = None):
    """diag(X^T X) / n + 1e-6 for X = ``inputs`` [n, in_features],
    /root/reference/tools/sieve.py:79-95 (``outputs`` is unused there too)."""
    from .. import _C_ops
    _require_2d(inputs, "inputs")
    dev, from_cpu = _sieve_device(inputs)
    out = _C_ops.sieve_hdiag(inputs.to(dev), ieee_div=from_cpu)
    return out.cpu() if from_cpu else out
