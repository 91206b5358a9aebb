"""The slice-split kernel (orth_split.hip: 1024-column slices of K over the
grid, up to 32 tokens, partials added in slice order) against the FP64
oracle, forced through the kernel policy: the c2, c5 (q/o and down_proj,
K = 11008 with a narrower last slice) and c4 shapes, one slice (no
reduction launch), ragged N and M, group-128, group-256 and per-row scales,
alpha in {0, 0.5, 1}, BF16 activations, records that overflow and another
layer's plan (the CSR path), the fused bias, repeated calls; and against
the quarter-split and split-K kernels on the same inputs."""
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


def run(layer, x, alpha, policy="split", bias=None, plan=True, dtype=torch.float16, foreign=None):
    d = W.to_device(layer)
    xt = torch.from_numpy(np.asarray(x, dtype=np.float32)).to(dtype).cuda()
    y = torch.full((xt.shape[0], layer.N), float("nan"), dtype=dtype, device="cuda")
    p = None
    if foreign is not None:
        f = W.to_device(foreign)
        p = _C_ops.build_plan(f["q"], f["scales"], f["vals"], f["col"], f["row_ptr"], foreign.K)
    elif plan:
        p = _C_ops.build_plan(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], layer.K)
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


def check(oracle_mod, layer, x, alpha, y, what):
    ref = oracle_mod.forward_f64(layer.q, layer.scales, layer.row_ptr, layer.col, layer.vals, x, alpha)
    assert np.isfinite(y).all(), what
    err = float(np.abs(y - ref).max())
    assert err <= TOL * float(np.abs(ref).max()), f"{what}: max|err| {err} vs ||y|| {np.abs(ref).max()}"
    return err / float(np.abs(ref).max())


def agree(y, y2, what, rel=2e-3):
    """Two kernels that accumulate in FP32 in different orders and round once."""
    assert float(np.abs(y - y2).max()) <= rel * float(np.abs(y2).max()), what


@pytest.mark.parametrize("M", [17, 24, 32])
@pytest.mark.parametrize("alpha", [1.0, 0.0])
def test_split_c2(oracle_mod, M, alpha):
    lay = W.config_layer("c2")
    x = x_of(M, lay.K, 7700 + M)
    y, k = run(lay, x, alpha)
    assert k == "split"
    rel = check(oracle_mod, lay, x, alpha, y, f"c2 M={M} alpha={alpha}")
    assert rel < 2e-3, rel
    y2, k2 = run(lay, x, alpha, "quarter")
    assert k2 == "quarter"
    agree(y, y2, f"c2 M={M} against the quarter kernel")


@pytest.mark.parametrize("name", ["q_proj", "down_proj"])
@pytest.mark.parametrize("M", [17, 32])
def test_split_c5(oracle_mod, name, M):
    """c5 (2 % ortho: 512-word records); down_proj has K = 11008, ten full
    slices and one of 768 columns."""
    lay = {l.name: l for l in W.llama_block(case=2)}[name]
    x = x_of(M, lay.K, 7800 + M)
    y, k = run(lay, x, 1.0)
    assert k == "split"
    check(oracle_mod, lay, x, 1.0, y, f"c5 {name} M={M}")
    y2, k2 = run(lay, x, 1.0, "skinny")
    assert k2 == "skinny"
    agree(y, y2, f"c5 {name} M={M} against the split-K kernel")


@pytest.mark.parametrize("K,N,group,M,alpha,density", [
    (1024, 2000, 128, 20, 1.0, 0.02),   # one slice: y written by the workgroups, no reduction
    (2048, 1000, 128, 17, 0.5, 0.01),   # ragged N (a partial 64-row group and 16-row block)
    (3072, 1030, None, 31, 1.0, 0.01),  # per-row scales, N % 4 != 0 (one-output reduction)
    (4096, 512, 256, 32, 1.0, 0.01),    # group-256 scales, fewer groups than workgroups
    (1408, 40, 128, 1, 1.0, 0.02),      # 11 chunks (a slice of 3), one token, 40 rows
    (11008, 300, 128, 9, 0.0, 0.0),     # no ortho term
])
def test_split_shapes(oracle_mod, K, N, group, M, alpha, density):
    lay = W.make_layer(K, N, group, density, 7900 + K + N)
    x = x_of(M, K, 7901 + M)
    y, k = run(lay, x, alpha)
    assert k == "split"
    check(oracle_mod, lay, x, alpha, y, f"K={K} N={N} G={group} M={M} alpha={alpha}")


def skewed_rows_layer(K, N, heavy, per_heavy, seed):
    """~1 % uniform rows plus `heavy` rows of `per_heavy` entries each, whose
    16-row blocks hold more entries than a slice record."""
    rng = np.random.default_rng(seed)
    L = W.make_layer(K, N, 128, 0.0, seed=seed)
    rows = []
    for r in range(N):
        n = per_heavy if r in heavy else int(rng.binomial(K, 0.01))
        rows.append(np.sort(rng.choice(K, size=n, replace=False)).astype(np.int32))
    rp = np.zeros(N + 1, np.int32)
    rp[1:] = np.cumsum([len(c) for c in rows])
    col = np.concatenate(rows).astype(np.int32)
    vals = rng.normal(0, 0.05, len(col)).astype(np.float16)
    return W.Layer(K, N, L.q, L.scales, rp, col, vals)


def test_split_overflowing_records_read_the_csr(oracle_mod):
    lay = skewed_rows_layer(4096, 700, {3, 200, 201, 699}, 1500, 8000)
    x = x_of(24, lay.K, 8001)
    y, k = run(lay, x, 1.0)
    assert k == "split"
    check(oracle_mod, lay, x, 1.0, y, "overflowing records")
    y2, _ = run(lay, x, 1.0, "skinny", plan=False)
    agree(y, y2, "overflowing records against the unplanned split-K kernel")


def test_split_foreign_plan_reads_the_csr(oracle_mod):
    # another layer's plan, large enough to pass the size check, fails every
    # record's tag: the kernel reads the CSR instead
    lay = W.make_layer(2048, 1024, 128, 0.01, seed=8100)
    big = W.make_layer(2048, 2048, 128, 0.02, seed=8101)
    x = x_of(20, lay.K, 8102)
    y, k = run(lay, x, 1.0, foreign=big)
    assert k == "split"
    check(oracle_mod, lay, x, 1.0, y, "foreign plan")


@pytest.mark.parametrize("M", [17, 32])
def test_split_bf16(oracle_mod, M):
    lay = {l.name: l for l in W.llama_block(case=2)}["down_proj"]
    x = x_of(M, lay.K, 8200 + M, torch.bfloat16)
    y, k = run(lay, x, 1.0, dtype=torch.bfloat16)
    assert k == "split"
    check(oracle_mod, lay, x, 1.0, y, f"bf16 down_proj M={M}")
    lay = W.config_layer("c2")
    x = x_of(M, lay.K, 8210 + M, torch.bfloat16)
    y, k = run(lay, x, 1.0, dtype=torch.bfloat16)
    assert k == "split"
    check(oracle_mod, lay, x, 1.0, y, f"bf16 c2 M={M}")


@pytest.mark.parametrize("K", [1024, 4096])
def test_split_bias_matches_the_unfused_add(K):
    lay = W.make_layer(K, 1000, 128, 0.01, seed=8300 + K)
    x = x_of(24, K, 8301)
    y0, _ = run(lay, x, 1.0)
    g = torch.Generator(device="cpu").manual_seed(3)
    for dt in (torch.float16, torch.float32):
        b = (torch.randn(lay.N, generator=g) * 0.5).to(dt).cuda()
        y, k = run(lay, x, 1.0, bias=b)
        assert k == "split"
        want = (torch.from_numpy(y0).half().float() + b.float().cpu()).half().float().numpy()
        assert np.array_equal(y, want)


def test_split_repeated_calls_are_bit_identical():
    lay = W.config_layer("c2")
    d = W.to_device(lay)
    p = _C_ops.build_plan(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], lay.K)
    x = torch.from_numpy(W.make_x(32, lay.K, 8400)).cuda()
    outs = []
    _lib.set_kernel_policy("split")
    try:
        for _ in range(4):
            y = torch.full((32, lay.N), float("nan"), dtype=torch.float16, device="cuda")
            _C_ops.forward_planned(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], x, y, 1.0, p)
            assert _C_ops.last_kernel() == "split"
            outs.append(y)
    finally:
        _lib.set_kernel_policy("auto")
    torch.cuda.synchronize()
    for y in outs[1:]:
        assert torch.equal(y.view(torch.int16), outs[0].view(torch.int16))


def test_split_refuses_what_it_cannot_take():
    lay = W.make_layer(4000, 512, None, 0.01, 5)  # K % 128 != 0
    with pytest.raises(RuntimeError, match="slice-split"):
        run(lay, x_of(20, 4000, 1), 1.0)
    lay = W.config_layer("c2")
    with pytest.raises(RuntimeError, match="slice-split"):  # ortho term without a plan
        run(lay, x_of(20, lay.K, 1), 1.0, plan=False)
    with pytest.raises(RuntimeError, match="slice-split"):  # more than 32 tokens
        run(lay, x_of(40, lay.K, 1), 1.0)
