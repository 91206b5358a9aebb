"""``torch_bind``: the reference's PyTorch-binding package
(/root/reference/torch_bind/__init__.py), importable from the repository
root as the reference's README (/root/reference/README.md:79) and examples
(/root/reference/examples/basic_usage.py:15) import it.  The module is
libortho_amd's OrthoLinear."""
from libortho_amd.torch_bind import OrthoLinear, load_checkpoint  # noqa: F401

__all__ = ["OrthoLinear"]
