"""``torch_bind.ortho_linear`` (/root/reference/torch_bind/ortho_linear.py):
OrthoLinear on MI355X, from libortho_amd."""
from libortho_amd.torch_bind.ortho_linear import (  # noqa: F401
    HAS_C_OPS, OrthoLinear, load_checkpoint, pack_base_torch)

__all__ = ["OrthoLinear"]
