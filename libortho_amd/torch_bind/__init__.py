"""PyTorch bindings (the reference's ``torch_bind`` package,
/root/reference/torch_bind/__init__.py)."""
from .ortho_linear import OrthoLinear, load_checkpoint

__all__ = ["OrthoLinear", "load_checkpoint"]
