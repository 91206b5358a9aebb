"""Weight-packing tools on the dual-GEMM path (the reference's ``tools``
package, /root/reference/tools/__init__.py:5-7): the sparse packer and the
offline Hessian sieve that produces the Base/Ortho split."""
from .sieve import compute_hessian_diag_approx, hessian_sieve, pack_ortho_sparse, quantize_int4

__all__ = ["hessian_sieve", "quantize_int4", "compute_hessian_diag_approx", "pack_ortho_sparse"]
