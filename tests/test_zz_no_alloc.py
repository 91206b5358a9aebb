"""orth_layer_forward_hip_noalloc (no allocation: scratch from a static
device array) against orth_layer_forward_hip_ex (per-stream workspace and
stream-ordered allocations), through the C ABI: same bits, on two calls in
a row with the second smaller, for each kernel that uses scratch (the
mid-batch split-K partials; the prefill plan built for an unplanned
alpha > 0 call) and for decode; and a request beyond the scratch size is
refused before anything is launched."""
import ctypes

import numpy as np
import pytest
import torch

from libortho_amd import _C_ops, _lib
from libortho_amd import workloads as W

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def call(entry, desc, x, y):
    fn = getattr(_lib.lib(), entry)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return fn(ctypes.byref(desc), None, 0, None, 0, _p(x), _p(y), int(x.shape[0]), _lib.DT_F16, s)


def compare(layer, Ms, alpha, kernel, seed):
    d = W.to_device(layer)
    desc = _C_ops.make_layer(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], layer.K, layer.N, alpha,
                             torch.device("cuda:0"))
    for M in Ms:  # second call smaller than the first
        x = torch.from_numpy(W.make_x(M, layer.K, seed + M)).cuda()
        y_ref = torch.full((M, layer.N), float("nan"), dtype=torch.float16, device="cuda")
        y = torch.full_like(y_ref, float("nan"))
        _lib.check(call("orth_layer_forward_hip_ex", desc, x, y_ref))
        _lib.check(call("orth_layer_forward_hip_noalloc", desc, x, y))
        assert _C_ops.last_kernel() == kernel
        torch.cuda.synchronize()
        assert torch.isfinite(y).all().item()
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16)), f"{kernel} M={M}"


def test_scratch_size_is_exported(gpu):
    assert _lib.lib().orth_noalloc_scratch_bytes() == 32 << 20


def test_mid_batch_split_k_partials_in_scratch(gpu):
    compare(W.config_layer("c2"), (24, 12), 1.0, "skinny", 8100)


def test_prefill_plan_in_scratch(gpu):
    compare(W.config_layer("c3"), (2048, 600), 1.0, "prefill", 8200)


def test_one_launch_mid_batch_needs_no_scratch(gpu):
    compare(W.config_layer("c2"), (16, 8), 0.0, "mid", 8400)


def test_quarter_partials_in_scratch(gpu):
    compare(W.config_layer("c2"), (32, 20), 0.0, "quarter", 8500)


def test_decode_needs_no_scratch(gpu):
    compare(W.config_layer("c2"), (2, 1), 1.0, "decode", 8300)


def test_request_beyond_the_scratch_is_refused(gpu):
    # a dense "ortho" of 1024 x 8192: the prefill plan's entries alone take
    # 4 * 8,388,608 bytes, past the 32 MiB of scratch
    K, N, M = 1024, 8192, 64 * 5
    q = torch.zeros(N, K // 2, dtype=torch.uint8, device="cuda")
    scales = torch.ones(N, dtype=torch.float16, device="cuda")
    row_ptr = (torch.arange(N + 1, dtype=torch.int64, device="cuda") * K).to(torch.int32)
    col = torch.arange(K, dtype=torch.int32, device="cuda").repeat(N)
    vals = torch.full((N * K,), 0.5, dtype=torch.float16, device="cuda")
    desc = _C_ops.make_layer(q, scales, vals, col, row_ptr, K, N, 1.0, torch.device("cuda:0"))
    x = torch.ones(M, K, dtype=torch.float16, device="cuda")
    y = torch.full((M, N), 7.0, dtype=torch.float16, device="cuda")
    _lib.set_kernel_policy("prefill")
    try:
        rc = call("orth_layer_forward_hip_noalloc", desc, x, y)
    finally:
        _lib.set_kernel_policy("auto")
    assert rc == _lib.ERR_UNSUPPORTED
    assert "scratch" in _lib.last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all().item()), "nothing may be launched"
