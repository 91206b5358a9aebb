"""Grouped forward (orth_layers_forward_hip): the projections of one
Llama-2-7B block that read one activation (q/k/v, gate/up) in one decode
launch, and at 17..32 tokens in one slice-split launch.  Each output must
have the bits of that layer's own forward call with the same kernel (the
same arithmetic per workgroup), and be within the parity bar of the FP64
oracle; groups that cannot share a launch fall back to one call per layer
with the same results."""
import numpy as np
import pytest
import torch

from libortho_amd import _C_ops, _lib
from libortho_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL = 1e-2  # max |err| <= TOL * ||y||_inf, as for single layers


@pytest.fixture(scope="module")
def block(gpu):
    torch.cuda.set_device(0)
    layers = {l.name: l for l in W.llama_block(case=1)}
    dev = {}
    for name, l in layers.items():
        d = W.to_device(l)
        d["plan"] = _C_ops.build_plan(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], l.K)
        dev[name] = d
    yield layers, dev
    _lib.set_kernel_policy("auto")


def desc(l, d, alpha):
    return _C_ops.make_layer(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], l.K, l.N, alpha,
                             torch.device("cuda:0"))


def separate(l, d, x, alpha, plan, bias=None, policy="auto"):
    y = torch.full((x.shape[0], l.N), float("nan"), dtype=x.dtype, device="cuda")
    _lib.set_kernel_policy(policy)
    try:
        _C_ops.forward_planned(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], x, y, alpha,
                               d["plan"] if plan else None, bias)
    finally:
        _lib.set_kernel_policy("auto")
    return y


def grouped(names, layers, dev, x, alphas, plan, biases=None):
    ls = [layers[n] for n in names]
    ds = [dev[n] for n in names]
    outs = [torch.full((x.shape[0], l.N), float("nan"), dtype=x.dtype, device="cuda") for l in ls]
    _C_ops.forward_group([desc(l, d, a) for l, d, a in zip(ls, ds, alphas)], x, outs,
                         [d["plan"] if plan else None for d in ds], biases)
    kernel = _C_ops.last_kernel()
    return outs, kernel


@pytest.mark.parametrize("names", [("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj"),
                                   ("q_proj", "k_proj", "v_proj", "o_proj")])
@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("plan", [True, False])
def test_group_matches_separate_calls(block, oracle_mod, names, M, plan):
    layers, dev = block
    K = layers[names[0]].K
    x_np = W.make_x(M, K, 900 + M)
    x = torch.from_numpy(x_np).cuda()
    outs, kernel = grouped(names, layers, dev, x, [1.0] * len(names), plan)
    assert kernel == "decode_group", kernel
    for n, y in zip(names, outs):
        ref_y = separate(layers[n], dev[n], x, 1.0, plan)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref_y.view(torch.int16)), f"{n}: group differs from its own call"
        l = layers[n]
        ref = oracle_mod.forward_f64(l.q, l.scales, l.row_ptr, l.col, l.vals, x_np, 1.0)
        err = float(np.abs(y.float().cpu().numpy() - ref).max())
        assert err <= TOL * float(np.abs(ref).max()), f"{n} M={M}: {err}"


def test_group_with_biases_and_mixed_alpha(block):
    """Biases fused per layer; a layer with alpha = 0 beside two with alpha =
    1 (a different ortho mode) runs as separate calls with the same bits."""
    layers, dev = block
    names = ("q_proj", "k_proj", "v_proj")
    x = torch.from_numpy(W.make_x(2, 4096, 77)).cuda()
    g = torch.Generator(device="cpu").manual_seed(5)
    biases = [(torch.randn(4096, generator=g) * 0.1).to(dt).cuda()
              for dt in (torch.float16, torch.bfloat16, torch.float32)]
    outs, kernel = grouped(names, layers, dev, x, [1.0] * 3, True, biases)
    assert kernel == "decode_group"
    for n, y, b in zip(names, outs, biases):
        assert torch.equal(y.view(torch.int16), separate(layers[n], dev[n], x, 1.0, True, b).view(torch.int16))
    outs, kernel = grouped(names, layers, dev, x, [1.0, 0.0, 1.0], True, biases)
    assert kernel != "decode_group"
    for n, y, a, b in zip(names, outs, (1.0, 0.0, 1.0), biases):
        assert torch.equal(y.view(torch.int16), separate(layers[n], dev[n], x, a, True, b).view(torch.int16))


@pytest.mark.parametrize("M", [8, 300])
def test_group_above_decode_falls_back(block, oracle_mod, M):
    layers, dev = block
    names = ("gate_proj", "up_proj")
    x_np = W.make_x(M, 4096, 300 + M)
    x = torch.from_numpy(x_np).cuda()
    outs, kernel = grouped(names, layers, dev, x, [1.0, 1.0], True)
    for n, y in zip(names, outs):
        assert torch.equal(y.view(torch.int16), separate(layers[n], dev[n], x, 1.0, True).view(torch.int16))
    rows = np.arange(M) if M <= 32 else np.array([0, 1, M // 2, M - 1])
    l = layers["up_proj"]
    ref = oracle_mod.forward_f64(l.q, l.scales, l.row_ptr, l.col, l.vals, x_np[rows], 1.0)
    err = float(np.abs(outs[1].float().cpu().numpy()[rows] - ref).max())
    assert err <= TOL * float(np.abs(ref).max())


@pytest.mark.parametrize("names", [("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj"),
                                   ("q_proj", "k_proj", "v_proj", "o_proj")])
@pytest.mark.parametrize("M", [17, 32])
@pytest.mark.parametrize("alpha", [1.0, 0.0])
def test_group_17_to_32_tokens_in_one_slice_split_launch(block, oracle_mod, names, M, alpha):
    """17..32 tokens: one slice-split launch and one reduction for the
    group; each output has the bits of that layer's own slice-split call
    (policy "split"; the default single call at K = 4096 takes the quarter
    kernel, equal up to FP32 summation order)."""
    layers, dev = block
    x_np = W.make_x(M, 4096, 950 + M)
    x = torch.from_numpy(x_np).cuda()
    outs, kernel = grouped(names, layers, dev, x, [alpha] * len(names), alpha > 0)
    assert kernel == "split_group", kernel
    for n, y in zip(names, outs):
        ys = separate(layers[n], dev[n], x, alpha, alpha > 0, policy="split")
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ys.view(torch.int16)), f"{n}: group differs from its own call"
        yq = separate(layers[n], dev[n], x, alpha, alpha > 0).float().cpu().numpy()
        yv = y.float().cpu().numpy()
        assert float(np.abs(yv - yq).max()) <= 2e-3 * float(np.abs(yq).max()), n
        l = layers[n]
        rows = np.array([0, 5, 16, M - 1])
        ref = oracle_mod.forward_f64(l.q, l.scales, l.row_ptr, l.col, l.vals, x_np[rows], alpha)
        err = float(np.abs(yv[rows] - ref).max())
        assert err <= TOL * float(np.abs(ref).max()), f"{n} M={M}: {err}"


def test_group_17_to_32_tokens_bf16_bias_and_fallbacks(block):
    """BF16 activations and per-layer biases in the grouped launch; a mixed
    alpha (another ortho class) and a forced kernel policy run one call per
    layer with the same bits as separate calls."""
    layers, dev = block
    names = ("q_proj", "k_proj", "v_proj")
    x = torch.from_numpy(W.make_x(24, 4096, 977)).to(torch.bfloat16).cuda()
    g = torch.Generator(device="cpu").manual_seed(8)
    biases = [(torch.randn(4096, generator=g) * 0.1).to(dt).cuda()
              for dt in (torch.bfloat16, torch.float32, torch.bfloat16)]
    outs, kernel = grouped(names, layers, dev, x, [1.0] * 3, True, biases)
    assert kernel == "split_group"
    for n, y, b in zip(names, outs, biases):
        ys = separate(layers[n], dev[n], x, 1.0, True, b, policy="split")
        assert torch.equal(y.view(torch.int16), ys.view(torch.int16)), n
    outs, kernel = grouped(names, layers, dev, x, [1.0, 0.0, 1.0], True, biases)
    assert kernel != "split_group"
    for n, y, a, b in zip(names, outs, (1.0, 0.0, 1.0), biases):
        assert torch.equal(y.view(torch.int16), separate(layers[n], dev[n], x, a, True, b).view(torch.int16))
    _lib.set_kernel_policy("skinny")
    try:
        outs, kernel = grouped(names, layers, dev, x, [1.0] * 3, True, biases)
    finally:
        _lib.set_kernel_policy("auto")
    assert kernel == "skinny"
    for n, y, b in zip(names, outs, biases):
        ys = separate(layers[n], dev[n], x, 1.0, True, b, policy="skinny")
        assert torch.equal(y.view(torch.int16), ys.view(torch.int16)), n


def test_group_argument_checks(block):
    layers, dev = block
    x = torch.from_numpy(W.make_x(1, 4096, 1)).cuda()
    q = layers["q_proj"]
    dq = desc(q, dev["q_proj"], 1.0)
    y = torch.empty(1, 4096, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="overlap"):
        _C_ops.forward_group([dq, dq], x, [y, y])
    with pytest.raises(RuntimeError, match="1..4"):
        _C_ops.forward_group([dq] * 5, x, [torch.empty_like(y) for _ in range(5)])
    dd = desc(layers["down_proj"], dev["down_proj"], 1.0)
    with pytest.raises(RuntimeError, match="in_features"):
        _C_ops.forward_group([dq, dd], x, [y, torch.empty(1, 4096, dtype=torch.float16, device="cuda")])


def test_ortholinear_forward_group(gpu):
    from libortho_amd.torch_bind import OrthoLinear
    g = torch.Generator(device="cpu").manual_seed(12)
    mods = []
    for n_out in (1024, 1024, 512):
        m = OrthoLinear(1024, n_out, bias=True).cuda()
        w = (torch.randn(n_out, 1024, generator=g) * 0.02).cuda()
        wo = torch.where(torch.rand(n_out, 1024, generator=g).cuda() < 0.01, w, torch.zeros_like(w))
        m.load_from_weights(w - wo, wo)
        with torch.no_grad():
            m.bias.copy_(torch.randn(n_out, generator=g))
        mods.append(m)
    for shape in ((1, 1024), (2, 1, 1024), (40, 1024)):
        x = torch.randn(*shape, generator=g).half().cuda()
        with torch.no_grad():
            got = OrthoLinear.forward_group(mods, x)
            if shape[0] * (shape[1] if len(shape) == 3 else 1) <= 4:
                assert _C_ops.last_kernel() == "decode_group"
            for m, y in zip(mods, got):
                ref = m(x)
                assert y.shape == ref.shape
                assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
