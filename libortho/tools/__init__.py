"""``libortho.tools``: the installed-package path of the reference's tools
(/root/reference/setup.py:189-195, /root/reference/tools/__init__.py:5-7)."""
from libortho_amd.tools.sieve import (  # noqa: F401
    compute_hessian_diag_approx, hessian_sieve, pack_ortho_sparse, quantize_int4)

__all__ = ["hessian_sieve", "quantize_int4", "compute_hessian_diag_approx", "pack_ortho_sparse"]
