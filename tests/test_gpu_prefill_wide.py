"""The wide-row prefill kernel (orth_prefill.hip, prefill_wide_kernel: one
256-token x 352-row tile per workgroup, or 128 rows in 64-column steps for
layers with too few rows) against the FP64 oracle and against
the 256 x 128 prefill kernel on the same inputs: the metric's 4096->11008
shape at 2048 tokens (every token tile, alpha in {0, 0.5, 1}, planned and
unplanned), ragged token and row counts, a row range that ends inside a
plan block, K = 11,008, group-256 and per-row scales, plan steps with more
entries than the prefetched ones, duplicate columns (the per-row fold),
BF16 activations and the fused bias."""
import numpy as np
import pytest
import torch

from libortho_amd import _C_ops, _lib
from libortho_amd import workloads as W

pytestmark = pytest.mark.gpu

# max|err| / ||y||_inf against the FP64 oracle: the weight operand is
# fp16(fp16(q*s) + alpha*v), as in the 256 x 128 prefill kernel (measured
# 3.5e-4 .. 4.2e-4 there)
TOL = 1e-3


@pytest.fixture(scope="module", autouse=True)
def _dev(gpu):
    torch.cuda.set_device(0)
    yield
    _lib.set_kernel_policy("auto")


def run(layer, x, alpha, policy="prefill_wide", plan=True, dtype=torch.float16, bias=None):
    d = W.to_device(layer)
    xt = torch.from_numpy(np.asarray(x, dtype=np.float32)).to(dtype).cuda()
    y = torch.full((xt.shape[0], layer.N), float("nan"), dtype=dtype, device="cuda")
    p = _C_ops.build_plan(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], layer.K) if plan else None
    _lib.set_kernel_policy(policy)
    try:
        _C_ops.forward_planned(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], xt, y, alpha, p, bias)
        kernel = _C_ops.last_kernel()
    finally:
        _lib.set_kernel_policy("auto")
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), kernel


def x_of(M, K, seed, dtype=torch.float16):
    """Activations as the device sees them (rounded to dtype), as float32."""
    return torch.from_numpy(W.make_x(M, K, seed).astype(np.float32)).to(dtype).float().numpy()


def rows_of(M, tile=256):
    """Two token rows in every 256-token tile, moving across the tiles, plus
    the first and the last row."""
    rows = {0, M - 1}
    for bm in range((M + tile - 1) // tile):
        lo, hi = bm * tile, min(M, (bm + 1) * tile)
        rows.add(lo + (37 * bm + 5) % (hi - lo))
        rows.add(hi - 1 - (53 * bm + 11) % (hi - lo))
    return np.array(sorted(rows))


def check(oracle_mod, layer, x, alpha, y, rows, what, tol=TOL):
    ref = oracle_mod.forward_f64(layer.q, layer.scales, layer.row_ptr, layer.col, layer.vals, x[rows], alpha)
    got = y[rows]
    assert np.isfinite(got).all(), what
    err = float(np.abs(got - ref).max())
    yinf = float(np.abs(ref).max())
    assert err <= tol * yinf, f"{what}: max|err| {err:.3e} > {tol} * ||y||_inf {yinf:.3e}"
    return err / yinf


def agree(y, y2, what, rel=2e-3):
    """Two kernels with the same weight operand, FP32 sums in different orders."""
    assert float(np.abs(y - y2).max()) <= rel * float(np.abs(y2).max()), what


@pytest.mark.parametrize("alpha", [0.0, 0.5, 1.0])
@pytest.mark.parametrize("plan", [True, False])
def test_wide_metric_shape(oracle_mod, alpha, plan):
    """4096 -> 11008 at 2048 tokens: the dispatcher's own pick, every token
    tile, every output column, and the 256 x 128 kernel on the same input."""
    lay = W.config_layer("c2")
    x = x_of(2048, lay.K, 9000)
    y, k = run(lay, x, alpha, policy="auto", plan=plan)
    assert k == "prefill_wide"
    rel = check(oracle_mod, lay, x, alpha, y, rows_of(2048), f"alpha={alpha} plan={plan}")
    print(f"wide 4096->11008 alpha={alpha} plan={plan}: max|err|/||y||_inf = {rel:.3e}")
    y2, k2 = run(lay, x, alpha, policy="prefill", plan=plan)
    assert k2 == "prefill"
    agree(y, y2, f"alpha={alpha} against the 256 x 128 prefill kernel")


@pytest.mark.parametrize("alpha", [0.0, 0.5, 1.0])
@pytest.mark.parametrize("plan", [True, False])
def test_wide_c3_128_row_tile(oracle_mod, alpha, plan):
    """c3 (4096 -> 4096 at 2048 tokens): too few rows for 352-row tiles, so
    the wide kernel takes 128-row tiles in 64-column steps (256 workgroups);
    every token tile and output column, against the oracle and the 256 x
    128 kernel."""
    lay = W.config_layer("c3")
    x = x_of(2048, lay.K, 9050)
    y, k = run(lay, x, alpha, plan=plan)
    assert k == "prefill_wide"
    rel = check(oracle_mod, lay, x, alpha, y, rows_of(2048), f"c3 alpha={alpha} plan={plan}")
    print(f"wide 128-row c3 alpha={alpha} plan={plan}: max|err|/||y||_inf = {rel:.3e}")
    y2, k2 = run(lay, x, alpha, policy="prefill", plan=plan)
    assert k2 == "prefill"
    agree(y, y2, f"c3 alpha={alpha} against the 256 x 128 prefill kernel")


@pytest.mark.parametrize("K,N,group,M,alpha,density", [
    (4096, 1000, 128, 600, 1.0, 0.01),    # one partial row range, a partial token tile
    (1024, 5000, 128, 300, 0.5, 0.02),    # ranges ending inside plan blocks, ragged N
    (2048, 704, 256, 513, 1.0, 0.01),     # group-256 scales, exactly two ranges, 513 tokens
    (3072, 1030, None, 256, 1.0, 0.01),   # per-row scales, N % 4 != 0
    (11008, 4096, 128, 512, 1.0, 0.02),   # c5's down projection (344 steps of 32 columns)
    (4096, 2048, 128, 40, 0.0, 0.0),      # no ortho term, fewer tokens than a tile
])
def test_wide_shapes(oracle_mod, K, N, group, M, alpha, density):
    lay = W.make_layer(K, N, group, density, 9100 + K + N)
    x = x_of(M, K, 9101 + M)
    y, k = run(lay, x, alpha)
    assert k == "prefill_wide"
    check(oracle_mod, lay, x, alpha, y, rows_of(M), f"K={K} N={N} G={group} M={M} alpha={alpha}")
    y2, _ = run(lay, x, alpha, policy="prefill")
    agree(y, y2, f"K={K} N={N} against the 256 x 128 prefill kernel")


def test_wide_skewed_plan_steps(oracle_mod):
    """c4's outlier columns put over a thousand entries in some (block,
    64-column step) cells: past the one prefetched entry per thread the fold
    reads the rest itself."""
    lay = W.config_layer("c4")
    x = x_of(300, lay.K, 9200)
    y, k = run(lay, x, 1.0)
    assert k == "prefill_wide"
    check(oracle_mod, lay, x, 1.0, y, rows_of(300), "c4 skewed")


def test_wide_duplicate_columns_are_deterministic(oracle_mod):
    """Rows that repeat columns (a non-canonical plan): one thread per row
    adds that row's entries in plan order, so repeated calls give the same
    bits, and they match the oracle."""
    rng = np.random.default_rng(12)
    K, N = 1024, 800
    base = W.make_layer(K, N, 128, 0.0, seed=9300)
    counts = rng.integers(0, 30, size=N)
    rp = np.zeros(N + 1, np.int32)
    rp[1:] = np.cumsum(counts)
    col = rng.integers(0, 40, size=rp[-1]).astype(np.int32)
    vals = rng.normal(0, 0.05, rp[-1]).astype(np.float16)
    lay = W.Layer(K, N, base.q, base.scales, rp, col, vals)
    x = x_of(300, K, 9301)
    ys = [run(lay, x, 1.0) for _ in range(3)]
    assert all(k == "prefill_wide" for _, k in ys)
    for y, _ in ys[1:]:
        assert np.array_equal(y.view(np.uint32), ys[0][0].view(np.uint32))
    check(oracle_mod, lay, x, 1.0, ys[0][0], rows_of(300), "duplicate columns")


def test_wide_bf16(oracle_mod):
    lay = W.config_layer("c2")
    x = x_of(1024, lay.K, 9400, torch.bfloat16)
    y, k = run(lay, x, 1.0, dtype=torch.bfloat16)
    assert k == "prefill_wide"
    check(oracle_mod, lay, x, 1.0, y, rows_of(1024), "bf16", tol=1e-2)
    y2, _ = run(lay, x, 1.0, policy="prefill", dtype=torch.bfloat16)
    agree(y, y2, "bf16 against the 256 x 128 prefill kernel", rel=1e-2)


def test_wide_bias_matches_the_unfused_add():
    lay = W.make_layer(4096, 1500, 128, 0.01, seed=9500)
    x = x_of(300, lay.K, 9501)
    y0, _ = run(lay, x, 1.0)
    g = torch.Generator(device="cpu").manual_seed(5)
    for dt in (torch.float16, torch.float32):
        b = (torch.randn(lay.N, generator=g) * 0.5).to(dt).cuda()
        y, k = run(lay, x, 1.0, bias=b)
        assert k == "prefill_wide"
        want = (torch.from_numpy(y0).half().float() + b.float().cpu()).half().float().numpy()
        assert np.array_equal(y, want)


def test_wide_repeated_calls_are_bit_identical():
    lay = W.config_layer("c2")
    x = x_of(1024, lay.K, 9600)
    ys = [run(lay, x, 1.0)[0] for _ in range(3)]
    for y in ys[1:]:
        assert np.array_equal(y.view(np.uint32), ys[0].view(np.uint32))
