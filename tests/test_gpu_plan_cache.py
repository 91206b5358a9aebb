"""The reference's 8-argument ``libortho._C_ops.forward`` keeps an ortho plan
per weight set (``_C_ops._PlanCache``): from the first call on a set it takes
the planned kernels, with the bits of ``forward_planned`` given the same plan,
and it never uses a plan of other or changed weights."""
import gc

import numpy as np
import pytest
import torch

from libortho_amd import _C_ops, _lib
from libortho_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _fresh(gpu):
    torch.cuda.set_device(0)
    _lib.set_kernel_policy("auto")
    _C_ops._PLANS.clear()
    yield
    _C_ops._PLANS.clear()


def args(d):
    return d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"]


def planned(d, x, alpha, K):
    """The same call with an explicitly built plan."""
    y = torch.full((x.shape[0], d["q"].shape[0]), float("nan"), dtype=x.dtype, device="cuda")
    p = _C_ops.build_plan(*args(d), K)
    _C_ops.forward_planned(*args(d), x, y, alpha, p)
    return y, _C_ops.last_kernel()


def ref_forward(d, x, alpha):
    y = torch.full((x.shape[0], d["q"].shape[0]), float("nan"), dtype=x.dtype, device="cuda")
    _C_ops.forward(*args(d), x, y, alpha)
    return y, _C_ops.last_kernel()


@pytest.mark.parametrize("M,kernel", [(1, "decode"), (8, "mid"), (300, "prefill")])
def test_reference_forward_takes_the_planned_kernels(M, kernel):
    lay = W.config_layer("c2")
    d = W.to_device(lay)
    x = torch.from_numpy(W.make_x(M, lay.K, 6100 + M)).cuda()
    want, kw = planned(d, x, 1.0, lay.K)
    assert kw == kernel
    for _ in range(2):
        y, k = ref_forward(d, x, 1.0)
        assert k == kernel
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))
    assert len(_C_ops._PLANS) == 1


def test_unplanned_and_planned_kernels_differ_at_8_tokens():
    """What the cache changes for the 8-argument entry: at 8 tokens the call
    without a plan takes the decode kernel, with one the mid-batch kernel."""
    lay = W.config_layer("c2")
    d = W.to_device(lay)
    x = torch.from_numpy(W.make_x(8, lay.K, 6200)).cuda()
    y = torch.empty(8, lay.N, dtype=torch.float16, device="cuda")
    _C_ops.forward_planned(*args(d), x, y, 1.0, None)
    assert _C_ops.last_kernel() == "decode"
    _, k = ref_forward(d, x, 1.0)
    assert k == "mid"


def test_in_place_writes_and_new_tensors_rebuild_the_plan(oracle_mod):
    lay = W.make_layer(4096, 1040, 128, 0.02, 6300)
    d = W.to_device(lay)
    x = torch.from_numpy(W.make_x(1, 4096, 6301)).cuda()
    y0, _ = ref_forward(d, x, 1.0)
    d["vals"].mul_(-2.0)  # same tensor object, new contents (the plan records hold the values)
    y1, _ = ref_forward(d, x, 1.0)
    want, _ = planned(d, x, 1.0, 4096)
    assert torch.equal(y1.view(torch.int16), want.view(torch.int16))
    vals = lay.vals.astype(np.float32) * -2.0
    ref = oracle_mod.forward_f64(lay.q, lay.scales, lay.row_ptr, lay.col, vals.astype(np.float16),
                                 x.float().cpu().numpy(), 1.0)
    err = float(np.abs(y1.float().cpu().numpy() - ref).max())
    assert err <= 2e-3 * float(np.abs(ref).max())
    assert not torch.equal(y0, y1)
    # a different CSR tensor with the other contents: its own entry
    d2 = dict(d)
    d2["vals"] = d["vals"].clone().mul_(-0.5)
    y2, _ = ref_forward(d2, x, 1.0)
    assert torch.equal(y2.view(torch.int16), y0.view(torch.int16))


def test_freed_tensors_drop_their_plans():
    lay = W.make_layer(4096, 520, 128, 0.02, 6400)
    x = torch.from_numpy(W.make_x(2, 4096, 6401)).cuda()
    d = W.to_device(lay)
    ref_forward(d, x, 1.0)
    assert len(_C_ops._PLANS) == 1
    del d
    gc.collect()
    assert len(_C_ops._PLANS) == 0


def test_no_plan_without_the_ortho_term():
    lay = W.make_layer(4096, 520, 128, 0.02, 6500)
    d = W.to_device(lay)
    x = torch.from_numpy(W.make_x(1, 4096, 6501)).cuda()
    for alpha in (0.0, -1.0):
        ref_forward(d, x, alpha)
    assert len(_C_ops._PLANS) == 0


def test_plan_built_on_one_stream_used_on_another():
    lay = W.config_layer("c2")
    d = W.to_device(lay)
    x = torch.from_numpy(W.make_x(1, lay.K, 6600)).cuda()
    want, _ = planned(d, x, 1.0, lay.K)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    y = torch.full((1, lay.N), float("nan"), dtype=torch.float16, device="cuda")
    with torch.cuda.stream(s):
        _C_ops.forward(*args(d), x, y, 1.0)  # builds on s
    out = []
    for _ in range(3):  # used on the default stream
        yy, k = ref_forward(d, x, 1.0)
        out.append(yy)
        assert k == "decode"
    torch.cuda.synchronize()
    for yy in [y] + out:
        assert torch.equal(yy.view(torch.int16), want.view(torch.int16))


def test_graph_capture_reads_the_csr_and_builds_no_plan():
    """A captured graph would keep the pointer of a plan the cache may free,
    so captured calls take no plan (cached or new) and read the CSR."""
    lay = W.config_layer("c2")
    d = W.to_device(lay)
    fresh = W.to_device(W.make_layer(4096, 1040, 128, 0.02, 6700))
    x = torch.from_numpy(W.make_x(1, lay.K, 6701)).cuda()
    ref_forward(d, x, 1.0)  # cached eagerly
    assert len(_C_ops._PLANS) == 1
    want = torch.empty(1, lay.N, dtype=torch.float16, device="cuda")
    _C_ops.forward_planned(*args(d), x, want, 1.0, None)
    want2 = torch.empty(1, 1040, dtype=torch.float16, device="cuda")
    _C_ops.forward_planned(*args(fresh), x, want2, 1.0, None)
    y = torch.full((1, lay.N), float("nan"), dtype=torch.float16, device="cuda")
    y2 = torch.full((1, 1040), float("nan"), dtype=torch.float16, device="cuda")
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _C_ops.forward(*args(d), x, y, 1.0)  # eager warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g, stream=s):
        _C_ops.forward(*args(d), x, y, 1.0)
        _C_ops.forward(*args(fresh), x, y2, 1.0)
    assert len(_C_ops._PLANS) == 1
    _C_ops._PLANS.clear()  # the graph holds no plan pointer: replays are unaffected
    for _ in range(3):
        y.fill_(float("nan"))
        y2.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))
        assert torch.equal(y2.view(torch.int16), want2.view(torch.int16))


def _ortholinear(K, N, seed):
    from libortho_amd import OrthoLinear
    rng = np.random.default_rng(seed)
    m = OrthoLinear(K, N, group_size=128).cuda()
    m.load_from_weights(torch.from_numpy((rng.standard_normal((N, K)) * 0.02).astype(np.float32)).cuda(),
                        torch.from_numpy(np.where(rng.random((N, K)) < 0.02, rng.standard_normal((N, K)), 0.0)
                                         .astype(np.float32)).cuda())
    return m


@torch.no_grad()
def test_ortholinear_captured_without_warm_up_reads_the_csr():
    """A freshly loaded OrthoLinear captured with no eager call first: the
    plan cannot be built under capture (the build reads its flags back), so
    the captured forward reads the CSR; every replay equals an eager
    unplanned call, and the module builds its plan on its next eager call."""
    m = _ortholinear(4096, 1040, 6800)
    x = torch.from_numpy(W.make_x(1, 4096, 6801)).cuda()
    want = torch.empty(1, 1040, dtype=torch.float16, device="cuda")
    _C_ops.forward_planned(m.base_weight, m.base_scales, m.ortho_values, m.ortho_col_indices, m.ortho_row_ptr,
                           x, want, 1.0, None)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=s):
        y = m(x)
    assert m._plan is None
    for _ in range(3):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))
    m(x)
    assert m._plan is not None


@torch.no_grad()
def test_ortholinear_plan_used_on_another_stream_and_by_a_copy():
    """OrthoLinear's own plan: a second stream waits on its build before the
    first use there; a deep copy of a module that has run a forward rebuilds
    its own descriptor and plan, with the same outputs."""
    import copy
    m = _ortholinear(4096, 1040, 6800)
    x = torch.from_numpy(W.make_x(8, 4096, 6801)).cuda()
    want = m(x)
    assert _C_ops.last_kernel() == "mid"  # planned
    torch.cuda.synchronize()
    m.ortho_values.mul_(1.0)  # new version: the next call rebuilds the plan
    first = m(x)  # rebuilt on the default stream
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):  # no wait on the default stream: only the plan's build event orders s
        x.record_stream(s)
        got = m(x)
    torch.cuda.current_stream().wait_stream(s)
    c = copy.deepcopy(m)
    got2 = c(x)
    torch.cuda.synchronize()
    for y in (first, got, got2):
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))


def test_bounds_evict_the_least_recently_used_plans():
    """At most max_entries and max_bytes of plans (here set to 2 entries,
    then to one plan's bytes, through the public plan_cache_limit); the byte
    count follows every drop."""
    sets = [W.to_device(W.make_layer(4096, 520, 128, 0.02, 6900 + i)) for i in range(3)]
    x = torch.from_numpy(W.make_x(1, 4096, 6910)).cuda()
    saved = _C_ops.plan_cache_limit()
    _C_ops.plan_cache_clear()
    try:
        _C_ops.plan_cache_limit(entries=2)
        for d in sets:
            ref_forward(d, x, 1.0)
        assert len(_C_ops._PLANS) == 2
        plans = [e["plan"] for e in _C_ops._PLANS._d.values()]
        assert _C_ops._PLANS._bytes == sum(p.numel() for p in plans)
        assert _C_ops.plan_cache_info()["bytes"] == _C_ops._PLANS._bytes
        ref_forward(sets[1], x, 1.0)  # most recent: sets 2, 1
        ref_forward(sets[0], x, 1.0)  # rebuilt; evicts set 2
        keys = [k[2] for k in _C_ops._PLANS._d]
        assert keys == [id(sets[1]["vals"]), id(sets[0]["vals"])]
        _C_ops.plan_cache_limit(max_bytes=plans[0].numel())  # trims at once to the newest
        assert len(_C_ops._PLANS) == 1 and [k[2] for k in _C_ops._PLANS._d] == [id(sets[0]["vals"])]
        ref_forward(sets[2], x, 1.0)  # over the byte bound: only the newest stays
        assert len(_C_ops._PLANS) == 1 and [k[2] for k in _C_ops._PLANS._d] == [id(sets[2]["vals"])]
        del sets, d  # (the loop variable holds the last set too)
        gc.collect()
        assert len(_C_ops._PLANS) == 0 and _C_ops._PLANS._bytes == 0
    finally:
        _C_ops.plan_cache_limit(*saved)


def test_cache_off_and_clear():
    """entries=0 turns the cache off (calls read the CSR, same results as
    a planned call within one FP16 step); plan_cache_clear drops every plan."""
    d = W.to_device(W.make_layer(4096, 520, 128, 0.02, 6950))
    x = torch.from_numpy(W.make_x(1, 4096, 6951)).cuda()
    saved = _C_ops.plan_cache_limit()
    try:
        ref_forward(d, x, 1.0)
        assert _C_ops.plan_cache_info()["entries"] >= 1
        _C_ops.plan_cache_clear()
        assert _C_ops.plan_cache_info() == {"entries": 0, "bytes": 0, "max_entries": saved[0],
                                            "max_bytes": saved[1]}
        _C_ops.plan_cache_limit(entries=0)
        y, _ = ref_forward(d, x, 1.0)
        assert len(_C_ops._PLANS) == 0
        _C_ops.plan_cache_limit(entries=saved[0])
        y2, _ = ref_forward(d, x, 1.0)
        torch.cuda.synchronize()
        diff = (y.float() - y2.float()).abs()
        assert float(diff.max()) <= float(y.float().abs().max()) * 2e-3
    finally:
        _C_ops.plan_cache_limit(*saved)
