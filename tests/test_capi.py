"""The C ABI without a GPU: the library loads, exports exactly what
include/orth_hip.h declares, its structs match the header byte for byte,
and host-side validation returns the documented status codes (no device
access is needed for any of these)."""
import ctypes
import math
import os
import re
import subprocess

import pytest

from libortho_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "orth_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(orth_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libortho_amd.so not built (run __graft_entry__.build())")
    return _lib.lib()


def test_exports_every_declared_symbol(L):
    names = declared_functions()
    assert len(names) >= 13
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s+(orth_\w+)", out))
    missing = [n for n in names if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"
    for n in names:
        assert getattr(L, n) is not None


def test_struct_layout_matches_header(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(r'''
#include <stdio.h>
#include <stddef.h>
#include "orth_hip.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu %zu\n", sizeof(orth_hip_layer_t),
         offsetof(orth_hip_layer_t, ortho), offsetof(orth_hip_layer_t, alpha),
         offsetof(orth_hip_layer_t, ortho.count), offsetof(orth_hip_layer_t, base.scale_groups),
         sizeof(orth_hip_device_info_t), offsetof(orth_hip_device_info_t, global_mem_bytes));
  return 0;
}''')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    C = ctypes
    expect = [C.sizeof(_lib.OrthHipLayer), _lib.OrthHipLayer.ortho.offset,
              _lib.OrthHipLayer.alpha.offset,
              _lib.OrthHipLayer.ortho.offset + _lib.OrthHipOrtho.count.offset,
              _lib.OrthHipBase.scale_groups.offset, C.sizeof(_lib.OrthHipDeviceInfo),
              _lib.OrthHipDeviceInfo.global_mem_bytes.offset]
    assert got == expect


def fake_layer(K=4096, N=4096, groups=32, nnz=100):
    """A layer whose pointers are never dereferenced by host validation."""
    L = _lib.OrthHipLayer()
    L.base.q_weight = 0x1000
    L.base.q_scales = 0x2000
    L.base.q_bits = 4
    L.base.scale_dtype = _lib.DT_F16
    L.base.scale_groups = groups
    L.base.in_features = K
    L.base.out_features = N
    L.ortho.row_ptr = 0x3000 if nnz else None
    L.ortho.col_indices = 0x4000 if nnz else None
    L.ortho.values = 0x5000 if nnz else None
    L.ortho.value_dtype = _lib.DT_F16
    L.ortho.count = nnz
    L.alpha = 1.0
    return L


def check(L, layer, M=1, io=_lib.DT_F16, x=0x6000, y=0x7000):
    return L.orth_layer_check_hip(ctypes.byref(layer) if layer is not None else None, x, y, M, io)


def test_valid_call_passes_host_validation(L):
    assert check(L, fake_layer()) == _lib.OK
    assert check(L, fake_layer(nnz=0)) == _lib.OK
    assert check(L, fake_layer(groups=1)) == _lib.OK
    assert check(L, fake_layer(), M=0, x=None, y=None) == _lib.OK


@pytest.mark.parametrize("mutate,status,needle", [
    (lambda l: setattr(l.base, "in_features", 4095), _lib.ERR_INVALID_ARGUMENT, "even"),
    (lambda l: setattr(l.base, "in_features", 0), _lib.ERR_INVALID_ARGUMENT, "even"),
    (lambda l: setattr(l.base, "out_features", 0), _lib.ERR_INVALID_ARGUMENT, "out_features"),
    (lambda l: setattr(l.base, "q_bits", 8), _lib.ERR_UNSUPPORTED, "q_bits"),
    (lambda l: setattr(l.base, "scale_groups", 3), _lib.ERR_INVALID_ARGUMENT, "scale_groups"),
    (lambda l: setattr(l.base, "scale_groups", 0), _lib.ERR_INVALID_ARGUMENT, "scale_groups"),
    (lambda l: setattr(l.base, "scale_dtype", _lib.DT_BF16), _lib.ERR_INVALID_ARGUMENT, "scale_dtype"),
    (lambda l: setattr(l.base, "q_weight", None), _lib.ERR_INVALID_ARGUMENT, "q_weight"),
    (lambda l: setattr(l.base, "q_scales", None), _lib.ERR_INVALID_ARGUMENT, "q_scales"),
    (lambda l: setattr(l.ortho, "count", -1), _lib.ERR_INVALID_ARGUMENT, "negative"),
    (lambda l: setattr(l.ortho, "row_ptr", None), _lib.ERR_INVALID_ARGUMENT, "NULL CSR"),
    (lambda l: setattr(l.ortho, "values", None), _lib.ERR_INVALID_ARGUMENT, "NULL CSR"),
    (lambda l: setattr(l.ortho, "value_dtype", 9), _lib.ERR_INVALID_ARGUMENT, "value_dtype"),
    (lambda l: setattr(l.ortho, "count", 1 << 31), _lib.ERR_UNSUPPORTED, "int32"),
])
def test_layer_validation_errors(L, mutate, status, needle):
    layer = fake_layer()
    mutate(layer)
    assert check(L, layer) == status
    assert needle in _lib.last_error()


def test_io_validation_errors(L):
    assert check(L, None) == _lib.ERR_INVALID_ARGUMENT and "NULL" in _lib.last_error()
    assert check(L, fake_layer(), M=-1) == _lib.ERR_INVALID_ARGUMENT
    assert check(L, fake_layer(), io=7) == _lib.ERR_INVALID_ARGUMENT
    assert check(L, fake_layer(), x=None) == _lib.ERR_INVALID_ARGUMENT
    assert check(L, fake_layer(), M=1 << 40) == _lib.ERR_INVALID_ARGUMENT
    assert check(L, fake_layer(), io=_lib.DT_BF16) == _lib.OK
    assert check(L, fake_layer(), io=_lib.DT_F32) == _lib.OK


def test_forward_without_gpu_reports_no_device(L):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    layer = fake_layer()
    rc = L.orth_layer_forward_hip(ctypes.byref(layer), 0x6000, 0x7000, 1, _lib.DT_F16, None)
    assert rc == _lib.ERR_NO_DEVICE, _lib.last_error()
    # an empty batch never touches the device
    assert L.orth_layer_forward_hip(ctypes.byref(layer), None, None, 0, _lib.DT_F16, None) == _lib.OK
    with pytest.raises(_lib.OrthoError):
        _lib.device_info(0)


def cell_words(N, K, nnz, cols, max_words):
    # plan records of (16-row block, cols-column cell): 20 header words + the
    # mean entries of a cell + 4 (isqrt(mean) + 1), in 256-word units; 0 (no
    # records) above max_words
    mean = -(-16 * cols * nnz // (N * K))
    w = -(-(20 + mean + 4 * (math.isqrt(mean) + 1)) // 256) * 256
    return w if w <= max_words else 0


def qrec_words(N, K, nnz):
    # decode records: one per (16-row block, K quarter of cpw chunks)
    if K % 128:
        return 0
    c = (K // 128 + 3) // 4
    return cell_words(N, K, nnz, ((c + 1) & ~1) * 128, 2048)


def srec_words(N, K, nnz):
    # mid-batch records: one per (16-row block, 1024-column slice; the last
    # slice holds the rest of K)
    return 0 if K % 128 else cell_words(N, K, nnz, 1024, 512)


def test_plan_size(L):
    assert L.orth_ortho_plan_bytes(ctypes.byref(fake_layer(nnz=0))) == 0
    n = L.orth_ortho_plan_bytes(ctypes.byref(fake_layer(K=4096, N=4096, nnz=100)))
    offsets = ((4096 // 128) * (4096 // 64 + 1) * 4 + 15) // 16 * 16
    chunks = (4096 * (4096 // 128 + 1) * 2 + 15) // 16 * 16  # uint16 [N][K/128 + 1]
    qrecs = (4096 // 16) * 4 * qrec_words(4096, 4096, 100) * 4  # uint32 [N/16][4][Wq]
    assert qrec_words(4096, 4096, 100) == 256
    srecs = (4096 // 16) * (4096 // 1024) * srec_words(4096, 4096, 100) * 4
    assert srec_words(4096, 4096, 100) == 256
    assert n == (64 + offsets + 400 + 15) // 16 * 16 + chunks + qrecs + srecs
    # K % 128 != 0: no chunk table and no records
    n64 = L.orth_ortho_plan_bytes(ctypes.byref(fake_layer(K=4160, N=4100, nnz=100)))
    assert n64 == (64 + ((4100 + 127) // 128) * (4160 // 64 + 1) * 4 + 400 + 15) // 16 * 16
    # c2 (1 % of 4096 x 11008): 164 entries per (16-row, 1024-column) cell ->
    # 256 words; 2 % -> 512; 10 %: no records (the CSR paths)
    assert qrec_words(11008, 4096, 450888) == 256
    assert srec_words(11008, 4096, 450888) == 256
    assert srec_words(4096, 4096, 335544) == 512
    assert srec_words(4096, 4096, 4096 * 4096 // 10) == 0
    # down_proj shape (K = 11008: quarters of 22 chunks, 2816 columns) at 1 %
    assert qrec_words(4096, 11008, 450888) == 768
    # ... and its 11 slices (10 of 1024 columns, one of 768): 256 words each
    assert srec_words(4096, 11008, 450888) == 256
    n11 = L.orth_ortho_plan_bytes(ctypes.byref(fake_layer(K=11008, N=4096, nnz=450888)))
    off11 = ((4096 // 128) * (11008 // 64 + 1) * 4 + 15) // 16 * 16
    ch11 = (4096 * (11008 // 128 + 1) * 2 + 15) // 16 * 16
    assert n11 == ((64 + off11 + 4 * 450888 + 15) // 16 * 16 + ch11 + (4096 // 16) * 4 * 768 * 4
                   + (4096 // 16) * 11 * 256 * 4)
    assert qrec_words(4096, 11008, 2 * 450888) == 1280   # down_proj at 2 %
    assert qrec_words(4096, 4096, 4096 * 4096 // 10) == 2048
    assert qrec_words(4096, 4096, 4096 * 4096 // 5) == 0  # 20 %: the CSR path
    assert L.orth_ortho_plan_bytes(ctypes.byref(fake_layer(K=4000, nnz=5))) < 0  # K % 64 != 0
    assert L.orth_ortho_plan_bytes(ctypes.byref(fake_layer(K=4095))) == -_lib.ERR_INVALID_ARGUMENT


def test_policy_alpha_and_version(L):
    assert L.orth_hip_abi_version() == 103
    before = L.orth_hip_get_kernel_policy()
    for name, val in _lib.POLICIES.items():
        _lib.set_kernel_policy(name)
        assert L.orth_hip_get_kernel_policy() == val
    L.orth_hip_set_kernel_policy(before)
    assert L.orth_hip_set_kernel_policy(9) == _lib.ERR_INVALID_ARGUMENT
    layer = fake_layer()
    L.orth_layer_hip_set_alpha(ctypes.byref(layer), -0.25)
    assert layer.alpha == -0.25


def test_torch_binding_loads_first_in_a_fresh_process():
    """The compiled binding as the first thing a process loads (it loads the
    C library itself first): no lock re-entry, and it matches the ABI."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r); from libortho_amd import _lib; T = _lib.torch_ops(); "
            "print('binding', T is not None and T.abi_version() == _lib.lib().orth_hip_abi_version())" % ROOT)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    assert "binding True" in r.stdout
