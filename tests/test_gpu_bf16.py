"""BF16 activations and output on the fast paths: the decode kernel (1..4
tokens) and the one-launch mid-batch kernel (5..16 tokens), both at
K = 4096 with v_mfma_f32_16x16x32_bf16 over the exact BF16 integers
q + 136, and the prefill kernel (17+ tokens:
v_mfma_f32_32x32x16_bf16 over bf16(q*s) with the ortho term folded in
BF16).  Each is checked against the FP64 oracle on the same BF16 inputs
(the activations rounded to BF16 before both), and against the general
kernel (FP32 arithmetic) on the identical device inputs."""
import numpy as np
import pytest
import torch

from libortho_amd import _C_ops, _lib
from libortho_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL = 1e-2  # max |err| <= TOL * ||y||_inf (north_star bound; achieved ~4e-3, the BF16 output step)


@pytest.fixture(scope="module", autouse=True)
def _dev(gpu):
    torch.cuda.set_device(0)
    yield
    _lib.set_kernel_policy("auto")


def bf16_x(M, K, seed):
    """Activations rounded to BF16, as float32 (the oracle's input) and as the
    BF16 device tensor."""
    xb = torch.from_numpy(W.make_x(M, K, seed).astype(np.float32)).to(torch.bfloat16)
    return xb.float().numpy(), xb.cuda()


def run(layer, xd, alpha, policy="auto", bias=None, plan=True):
    d = W.to_device(layer)
    y = torch.full((xd.shape[0], layer.N), float("nan"), dtype=torch.bfloat16, device="cuda")
    p = _C_ops.build_plan(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], layer.K) if plan else None
    _lib.set_kernel_policy(policy)
    try:
        _C_ops.forward_planned(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], xd, y, alpha, p, bias)
        kernel = _C_ops.last_kernel()
    finally:
        _lib.set_kernel_policy("auto")
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), kernel


def check(oracle_mod, layer, x_np, alpha, y, what, rows=None):
    ref = oracle_mod.forward_f64(layer.q, layer.scales, layer.row_ptr, layer.col, layer.vals, x_np, alpha)
    if rows is not None:
        ref, y = ref[rows], y[rows]
    assert np.isfinite(y).all(), what
    err = float(np.abs(y - ref).max())
    assert err <= TOL * float(np.abs(ref).max()), f"{what}: max|err| {err} vs ||y|| {np.abs(ref).max()}"


def agree_with_general(layer, xd, alpha, y, what):
    """Both kernels accumulate in FP32 and round once to BF16: at most a few
    BF16 steps apart."""
    yg, kg = run(layer, xd, alpha, policy="general")
    assert kg == "general"
    scale = float(np.abs(yg).max())
    assert float(np.abs(y - yg).max()) <= 2 ** -6 * scale, what


@pytest.mark.parametrize("M", [1, 2, 3, 4, 8, 12, 16])
@pytest.mark.parametrize("alpha", [1.0, 0.0])
def test_bf16_c2(oracle_mod, M, alpha):
    lay = W.config_layer("c2")
    x_np, xd = bf16_x(M, lay.K, 5000 + M)
    y, k = run(lay, xd, alpha)
    assert k == ("decode" if M <= 4 else "mid")
    check(oracle_mod, lay, x_np, alpha, y, f"bf16 {k} c2 M={M} alpha={alpha}")
    agree_with_general(lay, xd, alpha, y, f"bf16 {k} c2 M={M}")
    if M <= 4:
        # the mid-batch kernel takes the same call when forced: same sums in
        # another order
        ym, km = run(lay, xd, alpha, policy="mid")
        assert km == "mid"
        assert float(np.abs(y - ym).max()) <= 2 ** -6 * float(np.abs(ym).max())


@pytest.mark.parametrize("N,group,M,alpha", [(1000, None, 6, 1.0), (40, 128, 16, 0.5), (3000, 128, 2, 1.0),
                                             (1000, None, 1, 1.0), (40, 128, 4, 0.5), (4096, 128, 3, 0.0)])
def test_bf16_shapes(oracle_mod, N, group, M, alpha):
    lay = W.make_layer(4096, N, group, 0.01, 300 + N)
    x_np, xd = bf16_x(M, 4096, 301 + M)
    y, k = run(lay, xd, alpha)
    assert k == ("decode" if M <= 4 else "mid")
    check(oracle_mod, lay, x_np, alpha, y, f"bf16 {k} N={N} G={group} M={M}")


def test_bf16_decode_c5_group(oracle_mod):
    """q/k/v of the c5 block in one BF16 decode launch: the bits of the
    separate calls, and the oracle's values."""
    layers = {l.name: l for l in W.llama_block(case=1)}
    names = ("q_proj", "k_proj", "v_proj")
    x_np, xd = bf16_x(2, 4096, 5300)
    ds, descs, plans, outs, singles = [], [], [], [], []
    for n in names:
        l = layers[n]
        d = W.to_device(l)
        p = _C_ops.build_plan(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], l.K)
        descs.append(_C_ops.make_layer(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], l.K, l.N, 1.0,
                                       torch.device("cuda:0")))
        plans.append(p)
        outs.append(torch.full((2, l.N), float("nan"), dtype=torch.bfloat16, device="cuda"))
        ys = torch.full((2, l.N), float("nan"), dtype=torch.bfloat16, device="cuda")
        _C_ops.forward_planned(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], xd, ys, 1.0, p)
        assert _C_ops.last_kernel() == "decode"
        singles.append(ys)
        ds.append(d)
    _C_ops.forward_group(descs, xd, outs, plans, None)
    assert _C_ops.last_kernel() == "decode_group"
    torch.cuda.synchronize()
    for n, yo, ys in zip(names, outs, singles):
        assert torch.equal(yo.view(torch.int16), ys.view(torch.int16)), n
        check(oracle_mod, layers[n], x_np, 1.0, yo.float().cpu().numpy(), f"bf16 group {n}")


def test_bf16_decode_down_proj(oracle_mod):
    """c5's down projection (K = 11008: 22-chunk quarters, paired group-128
    scales, 2 % ortho in records of more than 1024 words) in the BF16 decode
    kernel at one token; two tokens of K = 11008 exceed the staged
    activation block and take the split-K kernel, as FP16 does."""
    lay = {l.name: l for l in W.llama_block(case=1)}["down_proj"]
    x_np, xd = bf16_x(1, lay.K, 5401)
    for alpha in (1.0, 0.0):
        y, k = run(lay, xd, alpha)
        assert k == "decode"
        check(oracle_mod, lay, x_np, alpha, y, f"bf16 down_proj M=1 alpha={alpha}")
        agree_with_general(lay, xd, alpha, y, "bf16 down_proj M=1")
    _, xd2 = bf16_x(2, lay.K, 5402)
    _, k2 = run(lay, xd2, 1.0)
    assert k2 == "skinny"


def test_bf16_c5_block_takes_no_general_kernel(oracle_mod):
    """Every projection of the c5 block at one BF16 token on a fast kernel."""
    x_np, xd = bf16_x(1, 4096, 5500)
    acts = {}
    for l in W.llama_block(case=1):
        xin_np, xin = (x_np, xd) if l.K == 4096 else bf16_x(1, l.K, 5501)
        y, k = run(l, xin, 1.0)
        assert k == "decode", (l.name, k)
        check(oracle_mod, l, xin_np, 1.0, y, f"bf16 c5 {l.name}")


@pytest.mark.parametrize("M,kernel", [(8, "mid"), (1, "decode"), (3, "decode")])
def test_bf16_bias_matches_the_unfused_add(M, kernel):
    from oracle import pack_oracle as PO
    lay = W.config_layer("c2")
    _, xd = bf16_x(M, lay.K, 5100 + M)
    y0, _ = run(lay, xd, 1.0)
    for dt in (torch.bfloat16, torch.float32):
        b = (torch.randn(lay.N, generator=torch.Generator(device="cpu").manual_seed(4)) * 0.5).to(dt).cuda()
        y, k = run(lay, xd, 1.0, bias=b)
        assert k == kernel
        want = PO.f32_to_bf16_bits(y0.astype(np.float32) + b.float().cpu().numpy()[None, :])
        got = torch.from_numpy(y).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got, want)


def test_bf16_without_a_plan_takes_the_split_k_kernel(oracle_mod):
    lay = W.config_layer("c2")
    for M in (4, 8):
        x_np, xd = bf16_x(M, lay.K, 5200 + M)
        y, k = run(lay, xd, 1.0, plan=False)
        assert k == "skinny"  # the BF16 decode and mid kernels read the ortho term from the plan
        check(oracle_mod, lay, x_np, 1.0, y, f"bf16 unplanned skinny M={M}")
        _, k = run(lay, xd, 0.0, plan=False)
        assert k == ("decode" if M <= 4 else "mid")  # no ortho term: no plan needed


@pytest.mark.parametrize("alpha,plan", [(1.0, True), (0.5, False), (0.0, True)])
def test_prefill_bf16(oracle_mod, alpha, plan):
    lay = W.make_layer(4096, 1000, 128, 0.01, 400)
    x_np, xd = bf16_x(300, 4096, 401)
    y, k = run(lay, xd, alpha, plan=plan)
    assert k == "prefill"
    # rows in every 256-token tile, the first and the last
    rows = np.array([0, 1, 100, 255, 256, 280, 299])
    check(oracle_mod, lay, x_np, alpha, y, f"bf16 prefill alpha={alpha} plan={plan}", rows=rows)
    agree_with_general(lay, xd, alpha, y, f"bf16 prefill alpha={alpha}")


def test_prefill_bf16_per_row_scales_and_bias(oracle_mod):
    from oracle import pack_oracle as PO
    lay = W.make_layer(2048, 520, None, 0.02, 410)
    x_np, xd = bf16_x(80, 2048, 411)  # (up to 64 tokens take the split-K kernel)
    y, k = run(lay, xd, 1.0)
    assert k == "prefill"
    check(oracle_mod, lay, x_np, 1.0, y, "bf16 prefill per-row scales")
    b = (torch.randn(lay.N, generator=torch.Generator(device="cpu").manual_seed(5)) * 0.5).to(torch.bfloat16).cuda()
    yb, _ = run(lay, xd, 1.0, bias=b)
    want = PO.f32_to_bf16_bits(y.astype(np.float32) + b.float().cpu().numpy()[None, :])
    got = torch.from_numpy(yb).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("M", [2, 8, 16, 32])
@pytest.mark.parametrize("alpha", [1.0, 0.0])
def test_bf16_split_k_down_proj(oracle_mod, M, alpha):
    """c5's down projection (K = 11008, group-128, 2 % ortho) with BF16
    activations at 2..32 tokens: the split-K kernel (bf16 MFMA over q + 136,
    FP32 partials, a BF16 reduction)."""
    lay = {l.name: l for l in W.llama_block(case=1)}["down_proj"]
    x_np, xd = bf16_x(M, lay.K, 5600 + M)
    y, k = run(lay, xd, alpha, policy="skinny")  # (17..32 tokens take the slice-split kernel by default)
    assert k == "skinny"
    check(oracle_mod, lay, x_np, alpha, y, f"bf16 skinny down_proj M={M} alpha={alpha}")
    agree_with_general(lay, xd, alpha, y, f"bf16 skinny down_proj M={M}")


@pytest.mark.parametrize("K,N,M", [(11008, 4096, 8), (11008, 1001, 24), (4096, 1040, 40)])
def test_bf16_split_k_bias_matches_the_unfused_add(oracle_mod, K, N, M):
    """The fused bias in the split-K path: the reduction's BF16 store (4
    outputs per thread when N % 4 == 0, one otherwise) has the bits of the
    FP32 add after the unfused call."""
    from oracle import pack_oracle as PO
    lay = W.make_layer(K, N, 128, 0.01, 5700 + N)
    x_np, xd = bf16_x(M, K, 5701 + M)
    y0, k = run(lay, xd, 1.0, policy="skinny")
    assert k == "skinny"
    check(oracle_mod, lay, x_np, 1.0, y0, f"bf16 skinny K={K} N={N} M={M}")
    for dt in (torch.bfloat16, torch.float32):
        b = (torch.randn(N, generator=torch.Generator(device="cpu").manual_seed(6)) * 0.5).to(dt).cuda()
        y, kb = run(lay, xd, 1.0, policy="skinny", bias=b)
        assert kb == "skinny"
        want = PO.f32_to_bf16_bits(y0.astype(np.float32) + b.float().cpu().numpy()[None, :])
        got = torch.from_numpy(y).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("M", [17, 24, 32])
@pytest.mark.parametrize("alpha", [1.0, 0.0])
def test_bf16_quarter_c2(oracle_mod, M, alpha):
    """17..32 BF16 tokens at K = 4096 with 256-word plan records: the
    quarter-split kernel (q + 136 weights, 136 * sum(x) per chunk and token
    formed once at staging, BF16 stores in the reduction)."""
    lay = W.config_layer("c2")
    x_np, xd = bf16_x(M, lay.K, 5800 + M)
    y, k = run(lay, xd, alpha)
    assert k == "quarter"
    check(oracle_mod, lay, x_np, alpha, y, f"bf16 quarter c2 M={M} alpha={alpha}")
    agree_with_general(lay, xd, alpha, y, f"bf16 quarter c2 M={M}")


@pytest.mark.parametrize("N,group,M", [(1040, 128, 24), (1001, 128, 20), (520, None, 17)])
def test_bf16_quarter_shapes_and_bias(oracle_mod, N, group, M):
    """Ragged N (the reduction's one-output path when N % 4 != 0), per-row
    scales, and the fused BF16 / FP32 bias with the bits of the unfused add."""
    from oracle import pack_oracle as PO
    lay = W.make_layer(4096, N, group, 0.01, 5900 + N)
    x_np, xd = bf16_x(M, 4096, 5901 + M)
    y0, k = run(lay, xd, 1.0)
    assert k == "quarter"
    check(oracle_mod, lay, x_np, 1.0, y0, f"bf16 quarter N={N} G={group} M={M}")
    for dt in (torch.bfloat16, torch.float32):
        b = (torch.randn(N, generator=torch.Generator(device="cpu").manual_seed(7)) * 0.5).to(dt).cuda()
        y, kb = run(lay, xd, 1.0, bias=b)
        assert kb == "quarter"
        want = PO.f32_to_bf16_bits(y0.astype(np.float32) + b.float().cpu().numpy()[None, :])
        got = torch.from_numpy(y).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got, want)


def test_bf16_quarter_leaves_larger_records_to_the_slice_split(oracle_mod):
    """c5's q_proj (2 % ortho: 512-word records) at 32 BF16 tokens takes the
    slice-split kernel (the quarter kernel takes BF16 with 256-word records only)."""
    lay = {l.name: l for l in W.llama_block(case=1)}["q_proj"]
    x_np, xd = bf16_x(32, lay.K, 6000)
    y, k = run(lay, xd, 1.0)
    assert k == "split"
    check(oracle_mod, lay, x_np, 1.0, y, "bf16 c5 q_proj M=32")
