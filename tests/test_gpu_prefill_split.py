"""The 256 x 128 prefill kernel with K split over the grid (orth_prefill.hip,
prefill_kernel over slices of K, FP32 partials added in slice order by
split_reduce_kernel): taken where the tile grid alone leaves CUs idle (c3 at
512 or 1024 tokens, any prefill call of one 256-token tile), with a plan or
without an ortho term.  Checked against the FP64 oracle and against the
unsplit wide kernel on the same inputs: slices that start inside a scale
group, K = 11,008, group-256 and per-row scales, N % 4 != 0 (the scalar
reduction), plan steps with more entries than one per thread, duplicate
columns, BF16, the fused bias, no ortho term, and a captured graph replayed
between eager calls."""
import numpy as np
import pytest
import torch

from libortho_amd import _C_ops, _lib
from libortho_amd import workloads as W

pytestmark = pytest.mark.gpu

# max|err| / ||y||_inf against the FP64 oracle: the weight operand is
# fp16(fp16(q*s) + alpha*v) as without the split; only the order of the FP32
# sums changes
TOL = 1e-3


@pytest.fixture(scope="module", autouse=True)
def _dev(gpu):
    torch.cuda.set_device(0)
    yield
    _lib.set_kernel_policy("auto")


def run(layer, x, alpha, policy="auto", plan=True, dtype=torch.float16, bias=None):
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
    return torch.from_numpy(W.make_x(M, K, seed).astype(np.float32)).to(dtype).float().numpy()


def rows_of(M, tile=256):
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
    assert float(np.abs(y - y2).max()) <= rel * float(np.abs(y2).max()), what


@pytest.mark.parametrize("alpha", [0.0, 0.5, 1.0])
def test_split_c3_512_tokens(oracle_mod, alpha):
    """c3 at 512 tokens: 64 tiles, so K in 4 slices (256 workgroups); every
    token tile and output column against the oracle and the unsplit wide
    kernel."""
    lay = W.config_layer("c3")
    x = x_of(512, lay.K, 9700)
    y, k = run(lay, x, alpha)
    assert k == "prefill"
    rel = check(oracle_mod, lay, x, alpha, y, rows_of(512), f"c3 M=512 alpha={alpha}")
    print(f"split c3 M=512 alpha={alpha}: max|err|/||y||_inf = {rel:.3e}")
    y2, k2 = run(lay, x, alpha, policy="prefill_wide")
    assert k2 == "prefill_wide"
    agree(y, y2, f"c3 M=512 alpha={alpha} against the wide kernel")


@pytest.mark.parametrize("K,N,group,M,alpha,density", [
    (4096, 4096, 128, 1024, 1.0, 0.01),   # c3 at 1024 tokens: 2 slices
    (4096, 4096, 128, 65, 1.0, 0.01),     # the smallest prefill call: 8 slices of 8 steps
    (4096, 11008, 128, 256, 1.0, 0.01),   # c2 at 256 tokens: 2 slices
    (2048, 8960, 256, 256, 0.5, 0.01),    # 3 slices of 11, 11, 10 steps: slices start inside group-256 scales
    (11008, 4096, 128, 512, 1.0, 0.02),   # down projection: 4 slices of 43 steps (odd: inside group-128 scales)
    (3072, 1030, None, 100, 1.0, 0.01),   # per-row scales, N % 4 != 0 (the scalar reduction)
    (512, 1000, 128, 300, 1.0, 0.02),     # K = 512: 2 slices of 4 steps, ragged N
    (4096, 4608, 128, 200, 1.0, 0.01),    # 36 tiles: 7 slices, 6 of 10 steps and a last one of 4
    (4096, 2048, 128, 100, 0.0, 0.0),     # no ortho term
])
def test_split_shapes(oracle_mod, K, N, group, M, alpha, density):
    lay = W.make_layer(K, N, group, density, 9710 + K + N)
    x = x_of(M, K, 9711 + M)
    y, k = run(lay, x, alpha)
    assert k == "prefill"
    check(oracle_mod, lay, x, alpha, y, rows_of(M), f"K={K} N={N} G={group} M={M} alpha={alpha}")
    y2, _ = run(lay, x, alpha, policy="prefill_wide")
    agree(y, y2, f"K={K} N={N} M={M} against the wide kernel")


def test_split_skewed_plan_steps(oracle_mod):
    """c4's outlier columns put over a thousand entries in some plan cells:
    the fold's own loop, within each slice's steps."""
    lay = W.config_layer("c4")
    x = x_of(100, lay.K, 9720)
    y, k = run(lay, x, 1.0)
    assert k == "prefill"
    check(oracle_mod, lay, x, 1.0, y, rows_of(100), "c4 skewed, split")


def test_split_duplicate_columns_are_deterministic(oracle_mod):
    rng = np.random.default_rng(13)
    K, N = 1024, 800
    base = W.make_layer(K, N, 128, 0.0, seed=9730)
    counts = rng.integers(0, 30, size=N)
    rp = np.zeros(N + 1, np.int32)
    rp[1:] = np.cumsum(counts)
    col = rng.integers(0, 40, size=rp[-1]).astype(np.int32)
    vals = rng.normal(0, 0.05, rp[-1]).astype(np.float16)
    lay = W.Layer(K, N, base.q, base.scales, rp, col, vals)
    x = x_of(300, K, 9731)
    ys = [run(lay, x, 1.0) for _ in range(3)]
    assert all(k == "prefill" for _, k in ys)
    for y, _ in ys[1:]:
        assert np.array_equal(y.view(np.uint32), ys[0][0].view(np.uint32))
    check(oracle_mod, lay, x, 1.0, ys[0][0], rows_of(300), "duplicate columns, split")


def test_split_bf16(oracle_mod):
    lay = W.config_layer("c3")
    x = x_of(512, lay.K, 9740, torch.bfloat16)
    y, k = run(lay, x, 1.0, dtype=torch.bfloat16)
    assert k == "prefill"
    check(oracle_mod, lay, x, 1.0, y, rows_of(512), "bf16 split", tol=1e-2)
    y2, _ = run(lay, x, 1.0, policy="prefill_wide", dtype=torch.bfloat16)
    agree(y, y2, "bf16 split against the wide kernel", rel=1e-2)


def test_split_bias_matches_the_unfused_add():
    lay = W.make_layer(4096, 1500, 128, 0.01, seed=9750)
    x = x_of(300, lay.K, 9751)
    y0, k0 = run(lay, x, 1.0)
    assert k0 == "prefill"
    g = torch.Generator(device="cpu").manual_seed(6)
    for dt in (torch.float16, torch.float32):
        b = (torch.randn(lay.N, generator=g) * 0.5).to(dt).cuda()
        y, k = run(lay, x, 1.0, bias=b)
        assert k == "prefill"
        want = (torch.from_numpy(y0).half().float() + b.float().cpu()).half().float().numpy()
        assert np.array_equal(y, want)


def test_split_repeated_calls_are_bit_identical():
    lay = W.config_layer("c3")
    x = x_of(512, lay.K, 9760)
    ys = [run(lay, x, 1.0)[0] for _ in range(3)]
    for y in ys[1:]:
        assert np.array_equal(y.view(np.uint32), ys[0].view(np.uint32))


def test_unplanned_calls_stay_unsplit(oracle_mod):
    """Without a plan (alpha > 0) the call builds a temporary one and keeps
    K whole: the same bits as the planned call without the split are not
    promised, but the oracle holds, and repeated calls agree."""
    lay = W.config_layer("c3")
    x = x_of(512, lay.K, 9770)
    y, k = run(lay, x, 1.0, plan=False)
    assert k == "prefill"
    check(oracle_mod, lay, x, 1.0, y, rows_of(512), "c3 M=512 unplanned")
    y2, _ = run(lay, x, 1.0, plan=False)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))


def test_split_forward_captured_on_a_fresh_stream():
    """A split prefill forward captured in a HIP graph on a stream that never
    ran it eagerly (its partials in the GPU's scratch array, 32 MB at c3 with
    512 tokens), replayed several times with eager split forwards of another
    shape between the replays: every replay equals the eager result bit for
    bit."""
    lay = W.config_layer("c3")
    d = W.to_device(lay)
    plan = _C_ops.build_plan(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], lay.K)
    x = torch.from_numpy(W.make_x(512, lay.K, 9780)).cuda()
    y_eager = torch.empty(512, lay.N, dtype=torch.float16, device="cuda")
    _C_ops.forward_planned(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], x, y_eager, 1.0, plan)
    assert _C_ops.last_kernel() == "prefill"
    torch.cuda.synchronize()
    y = torch.empty_like(y_eager)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=s):
        _C_ops.forward_planned(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], x, y, 1.0, plan)
    x2 = torch.from_numpy(W.make_x(300, lay.K, 9781)).cuda()
    y2 = torch.empty(300, lay.N, dtype=torch.float16, device="cuda")
    for r in range(4):
        y.fill_(float("nan"))
        g.replay()
        _C_ops.forward_planned(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], x2, y2, 1.0, plan)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y_eager.view(torch.int16)), f"replay {r}"


@pytest.mark.parametrize("M,dtype", [(33, torch.float16), (64, torch.float16), (40, torch.bfloat16)])
def test_split_takes_33_to_64_tokens_at_wide_k(oracle_mod, M, dtype):
    """c5's down projection (K = 11,008) at 33..64 tokens: the split prefill
    kernel (8 slices), against the oracle and the split-K mid-batch kernel
    that took these calls before."""
    lay = {l.name: l for l in W.llama_block()}["down_proj"]
    x = x_of(M, lay.K, 9790 + M, dtype)
    y, k = run(lay, x, 1.0, dtype=dtype)
    assert k == "prefill"
    tol = TOL if dtype == torch.float16 else 1e-2
    check(oracle_mod, lay, x, 1.0, y, rows_of(M), f"down_proj M={M} {dtype}", tol=tol)
    y2, k2 = run(lay, x, 1.0, policy="skinny", dtype=dtype)
    assert k2 == "skinny"
    agree(y, y2, f"down_proj M={M} against the split-K mid-batch kernel", rel=2e-3 if dtype == torch.float16 else 1e-2)
