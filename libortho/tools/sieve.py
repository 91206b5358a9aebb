"""``libortho.tools.sieve``: the sieve and sparse packer from libortho_amd."""
from libortho_amd.tools.sieve import (  # noqa: F401
    compute_hessian_diag_approx, hessian_sieve, pack_ortho_sparse, quantize_int4)
