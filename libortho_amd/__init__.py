"""libortho_amd: libortho's fused dual GEMM (dense INT4 base + sparse FP16
ortho correction) for AMD Instinct MI355X (gfx950).

  libortho_amd._C_ops             the operator boundary (``libortho._C_ops``)
  libortho_amd.torch_bind         OrthoLinear (``torch_bind.OrthoLinear``)
  libortho_amd.tools              pack_ortho_sparse (``tools.sieve``)
  libortho_amd.csrc / include/    HIP kernels and their C ABI (libortho_amd.so)

The package imports without a GPU; calls that reach the library fail
loudly if libortho_amd.so has not been built.
"""
from . import _C_ops
from ._lib import OrthoError
from .tools import pack_ortho_sparse
from .torch_bind import OrthoLinear

__all__ = ["OrthoLinear", "OrthoError", "pack_ortho_sparse", "_C_ops"]
