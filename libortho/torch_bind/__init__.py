"""``libortho.torch_bind``: the installed-package path of the reference's
bindings (/root/reference/setup.py:189-195 maps it to torch_bind/)."""
from libortho_amd.torch_bind import OrthoLinear, load_checkpoint  # noqa: F401

__all__ = ["OrthoLinear"]
