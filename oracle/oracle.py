"""CPU oracle for libortho's fused dual GEMM (numpy/ctypes front end).

TEST INFRASTRUCTURE ONLY.  The product path (``libortho_amd``) never imports
this module; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may, and only as the checker or the
timed CPU baseline.

Every function wraps a C routine in ``oracle/ortho_oracle.c`` or
``oracle/cpu_baseline.c``; those files cite the reference lines they restate
(``/root/reference/src/ortho.c:315-402`` for the nibble decode, loop order,
alpha gate and sparse update).  Inputs are numpy arrays in the API layout:

  q        uint8  [N, K/2]   packed signed INT4, low nibble = even k
  scales   float16|float32 [N] or [N, K/G]
  row_ptr  int32  [N+1], col int32 [nnz], vals float16|float32 [nnz]
  x        float16|float32 [M, K]
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_REF_LIB_PATH = os.path.join(_HERE, "_ref", "libortho_ref.so")

_lib = None


def build(quiet: bool = True) -> None:
    """Compile the oracle with gcc (oracle/Makefile)."""
    out = subprocess.run(["make", "-C", _HERE], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + out.stdout + out.stderr)
    if not quiet:
        print(out.stdout)


def build_ref() -> bool:
    """Compile the reference's own CPU path into oracle/_ref when the
    reference tree is present (this container only).  Returns success."""
    if not os.path.isdir("/root/reference/src"):
        return False
    out = subprocess.run(["make", "-C", _HERE, "ref"], capture_output=True, text=True)
    return out.returncode == 0


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        f32 = ctypes.c_float
        L.orc_unpack_int4.argtypes = [P, ctypes.c_size_t]
        L.orc_unpack_int4.restype = ctypes.c_int
        L.orc_dequant_f32.argtypes = [P, P, i64, i64, i64, P]
        L.orc_dequant_f32.restype = None
        fwd = [P, P, i64, P, P, P, i64, f32, P, P, i64, i64, i64]
        for name in ("orc_forward_ref_f32", "orc_forward_f64", "orc_baseline_forward_f32"):
            getattr(L, name).argtypes = fwd
            getattr(L, name).restype = ctypes.c_int
        L.orc_baseline_time.argtypes = fwd + [ctypes.c_int, ctypes.c_int]
        L.orc_baseline_time.restype = ctypes.c_double
        L.orc_forward_ref_coo_f32.argtypes = [P, P, P, P, i64, f32, P, P, i64, i64, i64]
        L.orc_forward_ref_coo_f32.restype = ctypes.c_int
        L.orc_f32_array_to_f16.argtypes = [P, P, i64]
        L.orc_f16_array_to_f32.argtypes = [P, P, i64]
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=np.float32)


def _prep(q, scales, row_ptr, col, vals, x):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    N = q.shape[0]
    sc = _f32(scales).reshape(N, -1)
    x = _f32(x)
    if x.ndim == 1:
        x = x[None, :]
    M, K = x.shape
    if q.shape[1] * 2 != K:
        raise ValueError(f"q {q.shape} does not match K={K}")
    nnz = 0 if vals is None else int(np.asarray(vals).size)
    if nnz:
        rp = np.ascontiguousarray(row_ptr, dtype=np.int32)
        cl = np.ascontiguousarray(col, dtype=np.int32)
        vv = _f32(vals)
    else:
        rp = np.zeros(N + 1, np.int32)
        cl = np.zeros(1, np.int32)
        vv = np.zeros(1, np.float32)
    return q, sc, rp, cl, vv, nnz, x, M, K, N


def unpack_int4(packed: np.ndarray, idx: int) -> int:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    return int(lib().orc_unpack_int4(_ptr(packed), idx))


def dequant_f32(q, scales) -> np.ndarray:
    """float(q[n,k]) * float(s[n, k/G]) for the whole matrix, FP32."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    N, K = q.shape[0], q.shape[1] * 2
    sc = _f32(scales).reshape(N, -1)
    out = np.empty((N, K), np.float32)
    lib().orc_dequant_f32(_ptr(q), _ptr(sc), N, K, sc.shape[1], _ptr(out))
    return out


def forward_ref_f32(q, scales, row_ptr, col, vals, x, alpha: float) -> np.ndarray:
    """Reference loop order, FP32 accumulation (ortho.c:327-402)."""
    q, sc, rp, cl, vv, nnz, x, M, K, N = _prep(q, scales, row_ptr, col, vals, x)
    y = np.empty((M, N), np.float32)
    rc = lib().orc_forward_ref_f32(_ptr(q), _ptr(sc), sc.shape[1], _ptr(rp), _ptr(cl),
                                   _ptr(vv), nnz, float(alpha), _ptr(x), _ptr(y), M, K, N)
    if rc != 0:
        raise ValueError("orc_forward_ref_f32 rejected its arguments")
    return y


def forward_f64(q, scales, row_ptr, col, vals, x, alpha: float) -> np.ndarray:
    """The same formula accumulated in FP64 (the tolerance reference)."""
    q, sc, rp, cl, vv, nnz, x, M, K, N = _prep(q, scales, row_ptr, col, vals, x)
    y = np.empty((M, N), np.float64)
    rc = lib().orc_forward_f64(_ptr(q), _ptr(sc), sc.shape[1], _ptr(rp), _ptr(cl),
                               _ptr(vv), nnz, float(alpha), _ptr(x), _ptr(y), M, K, N)
    if rc != 0:
        raise ValueError("orc_forward_f64 rejected its arguments")
    return y


def forward_ref_coo_f32(q, scales, idx_u16, vals, x, alpha: float) -> np.ndarray:
    """The reference's legacy COO path (per-row scales, uint16 flat index)."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    N, K = q.shape[0], q.shape[1] * 2
    sc = _f32(scales)
    x = _f32(x).reshape(-1, K)
    idx = np.ascontiguousarray(idx_u16, dtype=np.uint16)
    vv = _f32(vals)
    y = np.empty((x.shape[0], N), np.float32)
    lib().orc_forward_ref_coo_f32(_ptr(q), _ptr(sc), _ptr(idx), _ptr(vv), idx.size,
                                  float(alpha), _ptr(x), _ptr(y), x.shape[0], K, N)
    return y


def baseline_time(q, scales, row_ptr, col, vals, x, alpha: float, warmup: int,
                  iters: int):
    """Mean seconds per call of the reference-flag CPU restatement
    (oracle/cpu_baseline.c), single thread; returns (seconds, y)."""
    q, sc, rp, cl, vv, nnz, x, M, K, N = _prep(q, scales, row_ptr, col, vals, x)
    y = np.empty((M, N), np.float32)
    t = lib().orc_baseline_time(_ptr(q), _ptr(sc), sc.shape[1], _ptr(rp), _ptr(cl),
                                _ptr(vv), nnz, float(alpha), _ptr(x), _ptr(y), M, K, N,
                                int(warmup), int(iters))
    return t, y


def f32_to_f16_bits(a) -> np.ndarray:
    """Round-to-nearest-even binary16 via the oracle's own converter."""
    a = _f32(a)
    out = np.empty(a.shape, np.uint16)
    lib().orc_f32_array_to_f16(_ptr(a), _ptr(out), a.size)
    return out


# ---------------------------------------------------------------------------
# the reference's compiled CPU path (oracle/_ref), this container only

class OrthBaseRef(ctypes.Structure):
    """Mirror of orth_base_t, /root/reference/include/ortho.h:22-28."""
    _fields_ = [("q_weight", ctypes.c_void_p), ("q_scales", ctypes.c_void_p),
                ("q_bits", ctypes.c_int), ("in_features", ctypes.c_size_t),
                ("out_features", ctypes.c_size_t)]


class OrthOrthoRef(ctypes.Structure):
    """Mirror of orth_ortho_t, /root/reference/include/ortho.h:41-53."""
    _fields_ = [("row_ptr", ctypes.c_void_p), ("col_indices", ctypes.c_void_p),
                ("values", ctypes.c_void_p), ("indices", ctypes.c_void_p),
                ("count", ctypes.c_int), ("capacity", ctypes.c_size_t),
                ("format", ctypes.c_int)]


class OrthLayerRef(ctypes.Structure):
    """Mirror of orth_layer_t, /root/reference/include/ortho.h:63-71 (nested
    exactly as in C so the padding after each sub-struct matches)."""
    _fields_ = [("base", OrthBaseRef), ("ortho", OrthOrthoRef), ("alpha", ctypes.c_float)]


def ref_lib_available() -> bool:
    return os.path.exists(_REF_LIB_PATH)


def ref_forward_coo(q, scales, idx_u16, vals, x, alpha: float) -> np.ndarray:
    """Run the reference's own orth_layer_forward (src/ortho.c:327-402),
    compiled by oracle/Makefile, on a COO layer built from numpy buffers."""
    L = ctypes.CDLL(_REF_LIB_PATH)
    L.orth_layer_forward.argtypes = [ctypes.POINTER(OrthLayerRef), ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_size_t]
    L.orth_layer_forward.restype = ctypes.c_int
    q = np.ascontiguousarray(q, dtype=np.uint8)
    N, K = q.shape[0], q.shape[1] * 2
    sc = _f32(scales)
    x = _f32(x).reshape(-1, K)
    idx = np.ascontiguousarray(idx_u16, dtype=np.uint16)
    vv = _f32(vals)
    layer = OrthLayerRef()
    assert ctypes.sizeof(layer) == 104, "orth_layer_t mirror has the wrong size"
    layer.base.q_weight = q.ctypes.data
    layer.base.q_scales = sc.ctypes.data
    layer.base.q_bits = 4
    layer.base.in_features = K
    layer.base.out_features = N
    layer.ortho.indices = idx.ctypes.data if idx.size else None
    layer.ortho.values = vv.ctypes.data if vv.size else None
    layer.ortho.count = int(idx.size)
    layer.ortho.capacity = int(idx.size)
    layer.ortho.format = 0
    layer.alpha = float(alpha)
    y = np.empty((x.shape[0], N), np.float32)
    rc = L.orth_layer_forward(ctypes.byref(layer), x.ctypes.data, y.ctypes.data, x.shape[0])
    if rc != 0:
        raise RuntimeError("reference orth_layer_forward returned %d" % rc)
    return y
