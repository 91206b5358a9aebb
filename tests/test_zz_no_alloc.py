"""orth_layer_forward_hip_noalloc (no allocation: scratch from a static
device array) against orth_layer_forward_hip_ex (per-stream workspace and
stream-ordered allocations), through the C ABI: same bits, on two calls in
a row with the second smaller, for each kernel that uses scratch (the
mid-batch split-K partials; the prefill K split's partials; the prefill
plan built for an unplanned alpha > 0 call) and for decode; and a request beyond the scratch size is
refused before anything is launched.  Captured into a graph, a call of
either entry adds kernel nodes only (no allocation node), and a captured
call beyond the scratch size needs an eager call on its stream first; calls
on two streams of one GPU are ordered by the library, so they do not race on
the shared scratch."""
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


def test_prefill_k_split_partials_in_scratch(gpu):
    # no ortho term (no plan needed): c3's K in 4 slices at 512 tokens (32 MB
    # of FP32 partials, the whole scratch array) and at 300
    compare(W.config_layer("c3"), (512, 300), 0.0, "prefill", 8150)


def test_prefill_plan_in_scratch(gpu):
    compare(W.config_layer("c3"), (2048, 1024), 1.0, "prefill_wide", 8200)
    compare(W.config_layer("c3"), (600, 300), 1.0, "prefill", 8250)


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


# ------------------------------------------------------------ graph capture

_GRAPH_NODE_KERNEL, _GRAPH_NODE_MEM_ALLOC, _GRAPH_NODE_MEM_FREE = 0, 10, 11


def _hip():
    h = ctypes.CDLL("libamdhip64.so")
    V, P = ctypes.c_void_p, ctypes.POINTER
    for name, args in (("hipStreamCreate", [P(V)]), ("hipStreamDestroy", [V]),
                       ("hipStreamBeginCapture", [V, ctypes.c_int]), ("hipStreamEndCapture", [V, P(V)]),
                       ("hipGraphGetNodes", [V, P(V), P(ctypes.c_size_t)]),
                       ("hipGraphNodeGetType", [V, P(ctypes.c_int)]), ("hipGraphDestroy", [V]),
                       ("hipStreamSynchronize", [V]), ("hipGraphInstantiate", [P(V), V, V, ctypes.c_char_p, ctypes.c_size_t]),
                       ("hipGraphLaunch", [V, V]), ("hipGraphExecDestroy", [V])):
        getattr(h, name).argtypes = args
        getattr(h, name).restype = ctypes.c_int
    return h


def captured_node_types(entry, desc, x, y, warm=False, replay=None):
    """Types of the nodes one call of `entry` adds to a graph captured on a
    fresh stream (with ``warm``, after the same call made eagerly on that
    stream).  With ``replay`` (an output tensor like y), the graph is also
    instantiated and launched once with y as its output, then y is copied
    into ``replay``."""
    h = _hip()
    s = ctypes.c_void_p()
    assert h.hipStreamCreate(ctypes.byref(s)) == 0
    g = ctypes.c_void_p()
    ex = ctypes.c_void_p()
    try:
        if warm:
            _lib.check(getattr(_lib.lib(), entry)(ctypes.byref(desc), None, 0, None, 0, _p(x), _p(y),
                                                  int(x.shape[0]), _lib.DT_F16, s))
            assert h.hipStreamSynchronize(s) == 0
        assert h.hipStreamBeginCapture(s, 0) == 0  # global mode
        rc = getattr(_lib.lib(), entry)(ctypes.byref(desc), None, 0, None, 0, _p(x), _p(y), int(x.shape[0]),
                                        _lib.DT_F16, s)
        assert h.hipStreamEndCapture(s, ctypes.byref(g)) == 0
        _lib.check(rc)
        n = ctypes.c_size_t(0)
        assert h.hipGraphGetNodes(g, None, ctypes.byref(n)) == 0
        nodes = (ctypes.c_void_p * n.value)()
        assert h.hipGraphGetNodes(g, nodes, ctypes.byref(n)) == 0
        types = []
        for nd in nodes:
            t = ctypes.c_int(-1)
            assert h.hipGraphNodeGetType(ctypes.c_void_p(nd), ctypes.byref(t)) == 0
            types.append(t.value)
        if replay is not None:
            y.fill_(float("nan"))
            torch.cuda.synchronize()
            assert h.hipGraphInstantiate(ctypes.byref(ex), g, None, None, 0) == 0
            assert h.hipGraphLaunch(ex, s) == 0
            assert h.hipStreamSynchronize(s) == 0
            replay.copy_(y)
        return types
    finally:
        if ex.value:
            h.hipGraphExecDestroy(ex)
        if g.value:
            h.hipGraphDestroy(g)
        h.hipStreamDestroy(s)


@pytest.mark.parametrize("cfg,M,alpha,kernel", [("c2", 24, 1.0, "skinny"), ("c3", 600, 1.0, "prefill"),
                                                ("c3", 1024, 1.0, "prefill_wide"), ("c3", 512, 0.0, "prefill"),
                                                ("c2", 32, 0.0, "quarter"), ("c2", 1, 1.0, "decode")])
def test_noalloc_capture_has_kernel_nodes_only(gpu, cfg, M, alpha, kernel):
    layer = W.config_layer(cfg)
    d = W.to_device(layer)
    desc = _C_ops.make_layer(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], layer.K, layer.N, alpha,
                             torch.device("cuda:0"))
    x = torch.from_numpy(W.make_x(M, layer.K, 8600 + M)).cuda()
    y = torch.empty(M, layer.N, dtype=torch.float16, device="cuda")
    torch.cuda.synchronize()
    types = captured_node_types("orth_layer_forward_hip_noalloc", desc, x, y)
    assert _C_ops.last_kernel() == kernel
    assert types and all(t == _GRAPH_NODE_KERNEL for t in types), types
    # the allocating entry records no allocation under capture either: on a
    # fresh stream its partials (or temporary plan) go to the scratch array
    y_eager = torch.empty_like(y)
    _lib.check(call("orth_layer_forward_hip_ex", desc, x, y_eager))
    y_graph = torch.empty_like(y)
    ctl = captured_node_types("orth_layer_forward_hip_ex", desc, x, y, replay=y_graph)
    assert ctl and all(t == _GRAPH_NODE_KERNEL for t in ctl), ctl
    torch.cuda.synchronize()
    assert torch.equal(y_graph.view(torch.int16), y_eager.view(torch.int16))


def test_capture_beyond_the_scratch_needs_an_eager_call_first(gpu):
    """A captured call whose partials exceed the scratch array (quarter-split
    kernel, M = 32, N = 65600: 33.6 MB) is refused on a fresh stream; after
    one eager call on the capture stream (which sizes that stream's capture
    buffer) it captures as kernel nodes only, and the graph's output equals
    the eager one."""
    layer = W.make_layer(4096, 65600, 128, 0.0, seed=8800)
    d = W.to_device(layer)
    desc = _C_ops.make_layer(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], layer.K, layer.N, 0.0,
                             torch.device("cuda:0"))
    x = torch.from_numpy(W.make_x(32, layer.K, 8801)).cuda()
    y = torch.empty(32, layer.N, dtype=torch.float16, device="cuda")
    assert 4 * 32 * layer.N * 4 > _lib.lib().orth_noalloc_scratch_bytes()
    y_eager = torch.empty_like(y)
    _lib.check(call("orth_layer_forward_hip_ex", desc, x, y_eager))
    assert _C_ops.last_kernel() == "quarter"
    torch.cuda.synchronize()
    with pytest.raises(_lib.OrthoError, match="capture buffer"):
        captured_node_types("orth_layer_forward_hip_ex", desc, x, y)
    y_graph = torch.empty_like(y)
    types = captured_node_types("orth_layer_forward_hip_ex", desc, x, y, warm=True, replay=y_graph)
    assert types and all(t == _GRAPH_NODE_KERNEL for t in types), types
    torch.cuda.synchronize()
    assert torch.equal(y_graph.view(torch.int16), y_eager.view(torch.int16))


def test_noalloc_calls_on_two_streams_are_ordered(gpu):
    """Split-K calls (partials in the shared scratch) launched back to back on
    two streams with no synchronisation between them: each output equals
    that of the allocating entry on one stream, bit for bit."""
    layer = W.config_layer("c2")
    d = W.to_device(layer)
    desc = _C_ops.make_layer(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], layer.K, layer.N, 1.0,
                             torch.device("cuda:0"))
    xs = [torch.from_numpy(W.make_x(24, layer.K, 8700 + i)).cuda() for i in range(2)]
    refs = []
    for x in xs:
        y = torch.empty(24, layer.N, dtype=torch.float16, device="cuda")
        _lib.check(call("orth_layer_forward_hip_ex", desc, x, y))
        refs.append(y)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(8):
        outs = [torch.full((24, layer.N), float("nan"), dtype=torch.float16, device="cuda") for _ in xs]
        torch.cuda.synchronize()
        for i in (0, 1, 0, 1):
            with torch.cuda.stream(streams[i]):
                _lib.check(call("orth_layer_forward_hip_noalloc", desc, xs[i], outs[i]))
                assert _C_ops.last_kernel() == "skinny"
        torch.cuda.synchronize()
        for i in (0, 1):
            assert torch.equal(outs[i].view(torch.int16), refs[i].view(torch.int16)), f"rep {rep} stream {i}"
