"""ctypes binding of the C ABI in include/orth_hip.h (libortho_amd.so).

The structures below mirror the header field for field; they are the only
place Python touches the ABI.  Loading fails loudly: there is no CPU or
pure-Python substitute for the HIP library.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("LIBORTHO_AMD_LIB", os.path.join(_HERE, "libortho_amd.so"))

# orth_dtype_t
DT_F16, DT_BF16, DT_F32 = 0, 1, 2
# orth_status_t
OK, ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED, ERR_HIP, ERR_NO_DEVICE = 0, 1, 2, 3, 4
STATUS_NAMES = {OK: "ORTH_OK", ERR_INVALID_ARGUMENT: "ORTH_ERR_INVALID_ARGUMENT",
                ERR_UNSUPPORTED: "ORTH_ERR_UNSUPPORTED", ERR_HIP: "ORTH_ERR_HIP",
                ERR_NO_DEVICE: "ORTH_ERR_NO_DEVICE"}
# kernel ids (orth_hip_last_kernel) and policies (orth_hip_set_kernel_policy)
KERNEL_NAMES = {0: "none", 1: "decode", 2: "prefill", 3: "general", 4: "skinny", 5: "decode_group", 6: "mid", 7: "quarter",
                8: "split", 9: "split_group", 10: "prefill_wide"}
GROUP_MAX = 4
POLICIES = {"auto": 0, "decode": 1, "prefill": 2, "general": 3, "skinny": 4, "mid": 5, "quarter": 6, "split": 7, "prefill_wide": 8}


class OrthHipBase(ctypes.Structure):
    _fields_ = [("q_weight", ctypes.c_void_p), ("q_scales", ctypes.c_void_p),
                ("q_bits", ctypes.c_int32), ("scale_dtype", ctypes.c_int32),
                ("scale_groups", ctypes.c_int64), ("in_features", ctypes.c_int64),
                ("out_features", ctypes.c_int64)]


class OrthHipOrtho(ctypes.Structure):
    _fields_ = [("row_ptr", ctypes.c_void_p), ("col_indices", ctypes.c_void_p),
                ("values", ctypes.c_void_p), ("value_dtype", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("count", ctypes.c_int64)]


class OrthHipLayer(ctypes.Structure):
    _fields_ = [("base", OrthHipBase), ("ortho", OrthHipOrtho), ("alpha", ctypes.c_float)]


class OrthHipDeviceInfo(ctypes.Structure):
    _fields_ = [("arch", ctypes.c_char * 64), ("is_gfx950", ctypes.c_int32),
                ("compute_units", ctypes.c_int32), ("wavefront_size", ctypes.c_int32),
                ("lds_bytes_per_block", ctypes.c_int32), ("clock_khz", ctypes.c_int32),
                ("memory_clock_khz", ctypes.c_int32), ("memory_bus_width", ctypes.c_int32),
                ("l2_bytes", ctypes.c_int32), ("global_mem_bytes", ctypes.c_int64)]


# every function the header declares, with its ctypes signature
_P, _I32, _I64, _F32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
_LP = ctypes.POINTER(OrthHipLayer)
SIGNATURES = {
    "orth_layer_hip_set_alpha": (None, [_LP, _F32]),
    "orth_layer_check_hip": (ctypes.c_int, [_LP, _P, _P, _I64, _I32]),
    "orth_layer_forward_hip": (ctypes.c_int, [_LP, _P, _P, _I64, _I32, _P]),
    "orth_layer_forward_hip_planned": (ctypes.c_int, [_LP, _P, _I64, _P, _P, _I64, _I32, _P]),
    "orth_layer_forward_hip_ex": (ctypes.c_int, [_LP, _P, _I64, _P, _I32, _P, _P, _I64, _I32, _P]),
    "orth_layer_forward_hip_noalloc": (ctypes.c_int, [_LP, _P, _I64, _P, _I32, _P, _P, _I64, _I32, _P]),
    "orth_noalloc_scratch_bytes": (_I64, []),
    "orth_layers_forward_hip": (ctypes.c_int, [_P, _P, _P, _P, _P, _I32, _P, _P, _I64, _I32, _P]),
    "orth_ortho_plan_bytes": (_I64, [_LP]),
    "orth_ortho_plan_build": (ctypes.c_int, [_LP, _P, _I64, _P]),
    "orth_base_dequant_hip": (ctypes.c_int, [_LP, _P, _P]),
    "orth_pack_base_hip": (ctypes.c_int, [_P, _I32, _I64, _I64, _I64, _P, _I32, _P, _P, _P]),
    "orth_pack_base_path": (ctypes.c_int, [_P, _I32, _I64, _I64, _P]),
    "orth_pack_csr_mask_bytes": (_I64, [_P, _I32, _I64, _I64]),
    "orth_pack_csr_rows_hip": (ctypes.c_int, [_P, _I32, _I64, _I64, _P, _P, _I64, _P]),
    "orth_pack_csr_fill_hip": (ctypes.c_int, [_P, _I32, _I64, _I64, _P, _P, _I64, _P, _P, _I32, _P]),
    "orth_sieve_quantize_hip": (ctypes.c_int, [_P, _I32, _I64, _I64, _P, _I32, _P]),
    "orth_sieve_select_bytes": (_I64, []),
    "orth_sieve_split_hip": (ctypes.c_int, [_P, _I32, _I64, _I64, _P, _I32, _I64, _I32, _I32, _I64, _F32,
                                            _P, _P, _P, _P, _I32, _P]),
    "orth_sieve_hdiag_workspace": (_I64, [_I64, _I64]),
    "orth_sieve_hdiag_hip": (ctypes.c_int, [_P, _I32, _I64, _I64, _P, _I64, _P, _I32, _P]),
    "orth_hip_device_info": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(OrthHipDeviceInfo)]),
    "orth_hip_set_kernel_policy": (ctypes.c_int, [ctypes.c_int]),
    "orth_hip_get_kernel_policy": (ctypes.c_int, []),
    "orth_hip_last_kernel": (ctypes.c_int, []),
    "orth_hip_last_error": (ctypes.c_char_p, []),
    "orth_hip_abi_version": (ctypes.c_int, []),
    "orth_hip_clock_stamp": (ctypes.c_int, [_P, _P]),
}

_lib = None
_lock = threading.Lock()


class LibraryNotBuilt(RuntimeError):
    pass


def lib():
    """The loaded libortho_amd.so (raises LibraryNotBuilt if it is absent)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise LibraryNotBuilt(
                        f"libortho_amd HIP library not found at {LIB_PATH}; build it with "
                        "`python -m libortho_amd.build` (hipcc, gfx950)")
                L = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(L, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = L
    return _lib


_torch_ops = None
_torch_ops_tried = False


def torch_ops():
    """The compiled torch binding (libortho_amd/_torch_ops*.so, built by
    libortho_amd.build beside libortho_amd.so), or None when it is absent:
    the ctypes calls of this module then serve the same entry points."""
    global _torch_ops, _torch_ops_tried
    if not _torch_ops_tried:
        L = lib()  # the binding links libortho_amd.so: load (and check) it first, outside the lock
        with _lock:
            if not _torch_ops_tried:
                try:
                    from . import _torch_ops as T
                    _torch_ops = T if T.abi_version() == L.orth_hip_abi_version() else None
                except ImportError:
                    _torch_ops = None
                _torch_ops_tried = True
    return _torch_ops


class OrthoError(RuntimeError):
    """A C-ABI call returned a status other than ORTH_OK."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")


def check(status: int) -> None:
    if status != OK:
        msg = lib().orth_hip_last_error()
        raise OrthoError(status, msg.decode() if msg else "")


def last_error() -> str:
    msg = lib().orth_hip_last_error()
    return msg.decode() if msg else ""


def last_kernel() -> str:
    return KERNEL_NAMES.get(lib().orth_hip_last_kernel(), "?")


def set_kernel_policy(policy: str) -> None:
    check(lib().orth_hip_set_kernel_policy(POLICIES[policy]))


def get_kernel_policy() -> str:
    inv = {v: k for k, v in POLICIES.items()}
    return inv[lib().orth_hip_get_kernel_policy()]


def device_info(device: int = 0) -> dict:
    info = OrthHipDeviceInfo()
    check(lib().orth_hip_device_info(device, ctypes.byref(info)))
    out = {f: getattr(info, f) for f, _ in OrthHipDeviceInfo._fields_}
    out["arch"] = info.arch.decode()
    return out
