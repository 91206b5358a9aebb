"""The one-launch mid-batch kernel (orth_mid.hip, 5..16 tokens, K = 4096)
and the quarter-split kernel (orth_quarter.hip, 17..32 tokens) against the
FP64 oracle, forced through the kernel policy: group-128 and per-row
scales, alpha in {0, 0.5, 1}, ragged N (a partial last row block, fewer
blocks than workgroups), the c2, c4 and c5 shapes, records that overflow
(skewed rows read from the CSR), the fused bias; and against the split-K
mid-batch kernel on the same inputs."""
import numpy as np
import pytest
import torch

from libortho_amd import _C_ops, _lib
from libortho_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL = 1e-2  # max |err| <= TOL * ||y||_inf (the achieved error is far below)


@pytest.fixture(scope="module", autouse=True)
def _dev(gpu):
    torch.cuda.set_device(0)
    yield
    _lib.set_kernel_policy("auto")


def run(layer, x_np, alpha, policy, bias=None, plan=True):
    d = W.to_device(layer)
    x = torch.from_numpy(np.asarray(x_np)).cuda()
    y = torch.full((x.shape[0], layer.N), float("nan"), dtype=torch.float16, device="cuda")
    p = _C_ops.build_plan(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], layer.K) if plan else None
    _lib.set_kernel_policy(policy)
    try:
        _C_ops.forward_planned(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], x, y, alpha, p, bias)
        kernel = _C_ops.last_kernel()
    finally:
        _lib.set_kernel_policy("auto")
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), kernel


def check(oracle_mod, layer, x_np, alpha, y, what):
    ref = oracle_mod.forward_f64(layer.q, layer.scales, layer.row_ptr, layer.col, layer.vals, x_np, alpha)
    assert np.isfinite(y).all(), what
    err = float(np.abs(y - ref).max())
    assert err <= TOL * float(np.abs(ref).max()), f"{what}: max|err| {err} vs ||y|| {np.abs(ref).max()}"
    return err / float(np.abs(ref).max())


@pytest.mark.parametrize("M", [5, 8, 9, 12, 16])
@pytest.mark.parametrize("alpha", [1.0, 0.0])
def test_mid_c2(oracle_mod, M, alpha):
    lay = W.config_layer("c2")
    x = W.make_x(M, lay.K, 4000 + M)
    y, k = run(lay, x, alpha, "mid")
    assert k == "mid"
    check(oracle_mod, lay, x, alpha, y, f"c2 M={M} alpha={alpha}")
    # the split-K kernel on the same inputs agrees to FP32 summation order
    y2, k2 = run(lay, x, alpha, "skinny")
    assert k2 == "skinny"
    assert float(np.abs(y - y2).max()) <= 2e-3 * float(np.abs(y2).max())


@pytest.mark.parametrize("N,group,M,alpha", [(1000, 128, 7, 0.5), (1000, None, 16, 1.0), (4096, None, 6, 1.0),
                                             (40, 128, 16, 1.0), (3000, 128, 13, 0.0)])
def test_mid_shapes(oracle_mod, N, group, M, alpha):
    lay = W.make_layer(4096, N, group, 0.01, 77 + N)
    x = W.make_x(M, 4096, 78 + M)
    y, k = run(lay, x, alpha, "mid")
    assert k == "mid"
    check(oracle_mod, lay, x, alpha, y, f"N={N} G={group} M={M}")


def test_mid_c4_skewed(oracle_mod):
    lay = W.config_layer("c4")
    x = W.make_x(8, lay.K, 4400)
    y, k = run(lay, x, 1.0, "mid")
    assert k == "mid"
    check(oracle_mod, lay, x, 1.0, y, "c4")


def test_mid_bias_matches_the_unfused_add(oracle_mod):
    lay = W.config_layer("c2")
    x = W.make_x(8, lay.K, 4500)
    g = torch.Generator(device="cpu").manual_seed(9)
    for dt in (torch.float16, torch.bfloat16, torch.float32):
        b = (torch.randn(lay.N, generator=g) * 0.5).to(dt).cuda()
        y, k = run(lay, x, 1.0, "mid", bias=b)
        y0, _ = run(lay, x, 1.0, "mid")
        assert k == "mid"
        want = (torch.from_numpy(y0).half().float() + b.float().cpu()).half().float().numpy()
        assert np.array_equal(y, want)


def test_mid_refuses_what_it_cannot_take():
    lay = W.make_layer(2048, 512, 128, 0.01, 5)  # K != 4096
    with pytest.raises(RuntimeError, match="mid-batch"):
        run(lay, W.make_x(8, 2048, 1), 1.0, "mid")
    lay = W.config_layer("c2")
    with pytest.raises(RuntimeError, match="mid-batch"):  # ortho term without a plan
        run(lay, W.make_x(8, lay.K, 1), 1.0, "mid", plan=False)


@pytest.mark.parametrize("M", [17, 24, 32])
@pytest.mark.parametrize("alpha", [1.0, 0.0, 0.5])
def test_quarter_c2(oracle_mod, M, alpha):
    lay = W.config_layer("c2")
    x = W.make_x(M, lay.K, 4600 + M)
    y, k = run(lay, x, alpha, "quarter")
    assert k == "quarter"
    rows = np.unique(np.linspace(0, M - 1, 9).astype(int))
    check(oracle_mod, lay, x[rows], alpha, y[rows], f"quarter c2 M={M} alpha={alpha}")
    y2, k2 = run(lay, x, alpha, "skinny")
    assert k2 == "skinny"
    assert float(np.abs(y - y2).max()) <= 2e-3 * float(np.abs(y2).max())


@pytest.mark.parametrize("N,group,M,density", [(4096, 128, 32, 0.02), (11008, 128, 32, 0.02), (1000, 128, 19, 0.01),
                                               (4096, None, 32, 0.01), (40, 128, 32, 0.01), (3000, 128, 25, 0.0)])
def test_quarter_shapes(oracle_mod, N, group, M, density):
    lay = W.make_layer(4096, N, group, density, 91 + N + M)
    x = W.make_x(M, 4096, 92 + M)
    y, k = run(lay, x, 1.0, "quarter")
    assert k == "quarter"
    check(oracle_mod, lay, x, 1.0, y, f"quarter N={N} G={group} M={M}")


def test_quarter_skewed_records_and_bias(oracle_mod):
    """c4's Zipf rows overflow some record cells (read from the CSR); the
    bias is added by the reduction with the bits of the unfused add."""
    lay = W.config_layer("c4")
    x = W.make_x(32, lay.K, 4700)
    y, k = run(lay, x, 1.0, "quarter")
    assert k == "quarter"
    rows = np.array([0, 5, 16, 31])
    check(oracle_mod, lay, x[rows], 1.0, y[rows], "quarter c4")
    b = (torch.randn(lay.N, generator=torch.Generator(device="cpu").manual_seed(3)) * 0.5).half().cuda()
    yb, _ = run(lay, x, 1.0, "quarter", bias=b)
    want = (torch.from_numpy(y).half().float() + b.float().cpu()).half().float().numpy()
    assert np.array_equal(yb, want)
