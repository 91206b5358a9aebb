"""``tools`` / ``tools.sieve``: the reference's development-mode import path
(/root/reference/tools/__init__.py:5-7, used as ``from tools.sieve import
...`` by /root/reference/README.md:64, /root/reference/examples/basic_usage.py:16
and /root/reference/torch_bind/ortho_linear.py:123), resolved from the
repository root to libortho_amd's sieve module.  One file rather than a
package: ``tools.sieve`` is registered as a submodule when this module is
imported, which the import system honours for ``from tools.sieve import``."""
import sys

from libortho_amd.tools import sieve  # noqa: F401
from libortho_amd.tools.sieve import (  # noqa: F401
    compute_hessian_diag_approx, hessian_sieve, pack_ortho_sparse, quantize_int4)

sys.modules[__name__ + ".sieve"] = sieve

__all__ = ["hessian_sieve", "quantize_int4", "compute_hessian_diag_approx", "pack_ortho_sparse"]
