"""The bias fused into every kernel's store (orth_layer_forward_hip_ex):
y = fp16(float(fp16(acc)) + bias[n]), the arithmetic of the reference's
`output += bias` after the kernel (/root/reference/torch_bind/
ortho_linear.py:165-166), checked bit for bit against that sum taken on the
CPU (numpy, FP32 add, round to nearest even) from the unfused output, and
against torch's own `+=` on the GPU, which can differ by one FP16 step where
the FP32 sum is exactly halfway between two FP16 values.  OrthoLinear fuses
the bias only where autograd does not need the add."""
import numpy as np
import pytest
import torch

from libortho_amd import OrthoLinear, _C_ops, _lib
from libortho_amd import workloads as W

pytestmark = pytest.mark.gpu

CASES = [
    # K, N, group, M, policy, expected kernel (unplanned, planned)
    (4096, 1040, 128, 1, "auto", ("decode", "decode")), (4096, 1040, 128, 3, "auto", ("decode", "decode")),
    (4096, 1040, 128, 8, "auto", ("decode", "mid")), (4096, 1040, 128, 8, "skinny", ("skinny", "skinny")),
    (4096, 1040, 128, 40, "auto", ("skinny", "skinny")), (4096, 1040, 128, 300, "auto", ("prefill", "prefill")),
    (200, 96, 40, 5, "auto", ("general", "general")), (4096, 1040, None, 1, "auto", ("decode", "decode")),
]


@pytest.mark.parametrize("K,N,group,M,policy,kernel", CASES)
@pytest.mark.parametrize("bdt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("planned", [False, True])
def test_fused_bias_has_the_bits_of_the_fp32_add(K, N, group, M, policy, kernel, bdt, planned):
    print(f"bias K={K} N={N} G={group} M={M} {bdt} planned={planned}", flush=True)
    lay = W.make_layer(K, N, group, 0.02, seed=K + N + M)
    d = W.to_device(lay)
    plan = _C_ops.build_plan(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], K) if planned else None
    x = torch.from_numpy(W.make_x(M, K, 5 + M)).cuda()
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(M)) * 0.3).to(bdt).cuda()
    _lib.set_kernel_policy(policy)
    try:
        y0 = torch.empty(M, N, dtype=torch.float16, device="cuda")
        _C_ops.forward_planned(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], x, y0, 1.0, plan)
        plain = y0.cpu().numpy()
        y0 += bias
        y1 = torch.empty(M, N, dtype=torch.float16, device="cuda")
        _C_ops.forward_planned(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], x, y1, 1.0, plan,
                               bias=bias)
        assert _C_ops.last_kernel() == kernel[int(planned)]
        torch.cuda.synchronize()
    finally:
        _lib.set_kernel_policy("auto")
    want = (plain.astype(np.float32) + bias.float().cpu().numpy()[None, :]).astype(np.float16)
    got = y1.cpu().numpy()
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    # torch's += : the same bits except at FP32 sums halfway between two FP16 values
    diff = y0.cpu().numpy().view(np.uint16) != got.view(np.uint16)
    assert diff.mean() < 1e-3
    if diff.any():
        s32 = plain.astype(np.float32) + bias.float().cpu().numpy()[None, :]
        lo = s32[diff].astype(np.float16).astype(np.float32)
        step = np.spacing(np.abs(lo).astype(np.float16)).astype(np.float32)
        assert np.all(np.isclose(np.abs(s32[diff] - lo), step / 2, rtol=0, atol=0)), "differs off a tie"


@pytest.mark.parametrize("io", [torch.bfloat16, torch.float32])
def test_fused_bias_in_the_general_kernel_for_other_io_dtypes(io):
    from oracle import pack_oracle as PO
    lay = W.make_layer(520, 96, 40, 0.02, seed=31)  # K % 128 != 0: no fast kernel for any dtype
    d = W.to_device(lay)
    x = torch.from_numpy(W.make_x(4, 520, 32)).cuda().to(io)
    bias = torch.randn(96, generator=torch.Generator().manual_seed(3)).cuda()
    y0 = torch.empty(4, 96, dtype=io, device="cuda")
    _C_ops.forward(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], x, y0, 1.0)
    y1 = torch.empty(4, 96, dtype=io, device="cuda")
    _C_ops.forward_planned(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], x, y1, 1.0, None,
                           bias=bias)
    assert _C_ops.last_kernel() == "general"
    s32 = y0.float().cpu().numpy() + bias.cpu().numpy()[None, :]
    if io == torch.float32:
        assert np.array_equal(y1.cpu().numpy().view(np.uint32), s32.view(np.uint32))
    else:
        got = y1.view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got, PO.f32_to_bf16_bits(s32))


def test_ortholinear_fuses_only_without_autograd():
    K, N = 1024, 256
    rng = np.random.default_rng(8)
    m = OrthoLinear(K, N, bias=True, group_size=128).cuda()
    m.load_from_weights(torch.from_numpy((rng.standard_normal((N, K)) * 0.02).astype(np.float32)).cuda(),
                        torch.from_numpy(np.where(rng.random((N, K)) < 0.02, rng.standard_normal((N, K)), 0.0)
                                         .astype(np.float32)).cuda())
    with torch.no_grad():
        m.bias.copy_(torch.randn(N, generator=torch.Generator(device="cpu").manual_seed(8)) * 0.1)
    x = torch.from_numpy(W.make_x(2, K, 9)).cuda()
    with torch.no_grad():
        y_fused = m(x)
        b, m.bias = m.bias, None
        y0 = m(x)
        m.bias = b
    y_graph = m(x)  # bias requires grad: the add stays outside the kernel
    assert y_graph.requires_grad and not y_fused.requires_grad
    want = (y0.float().cpu().numpy() + m.bias.detach().cpu().numpy()[None, :]).astype(np.float16)
    assert np.array_equal(y_fused.cpu().numpy().view(np.uint16), want.view(np.uint16))
    # torch's `+=` on the GPU: the same bits except one FP16 step at FP32 ties
    steps = np.abs(y_graph.detach().cpu().numpy().view(np.int16).astype(np.int32) - want.view(np.int16))
    assert steps.max() <= 1
    y_graph.float().sum().backward()
    assert torch.allclose(m.bias.grad, torch.full_like(m.bias.grad, 2.0))
