"""Weight-packing tools on the dual-GEMM path (the reference's ``tools``
package, /root/reference/tools/__init__.py).  Only the sparse packer is on
the path; the offline Hessian sieve is out of scope."""
from .sieve import pack_ortho_sparse

__all__ = ["pack_ortho_sparse"]
