"""``libortho.torch_bind.ortho_linear``: OrthoLinear from libortho_amd."""
from libortho_amd.torch_bind.ortho_linear import (  # noqa: F401
    HAS_C_OPS, OrthoLinear, load_checkpoint, pack_base_torch)

__all__ = ["OrthoLinear"]
