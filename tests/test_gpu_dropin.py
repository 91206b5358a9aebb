"""The reference's own call paths on the GPU, imported exactly as the
reference's README and example import them
(/root/reference/README.md:64,79, /root/reference/examples/basic_usage.py:15-16):
sieve -> OrthoLinear.load_from_weights -> forward, and the 8-argument
libortho._C_ops.forward, each checked against the FP64 oracle."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def oracle_forward(oracle_mod, m, x, alpha):
    scales = m.base_scales.cpu().numpy()
    return oracle_mod.forward_f64(m.base_weight.cpu().numpy(), scales, m.ortho_row_ptr.cpu().numpy(),
                                  m.ortho_col_indices.cpu().numpy(), m.ortho_values.cpu().numpy(),
                                  x.cpu().numpy(), alpha)


@pytest.mark.parametrize("M", [1, 8, 300])
def test_example_flow_through_reference_imports(gpu, oracle_mod, M):
    from tools.sieve import compute_hessian_diag_approx, hessian_sieve
    from torch_bind.ortho_linear import OrthoLinear
    g = torch.Generator(device="cpu").manual_seed(11)
    K, N = 1024, 768
    w = (torch.randn(N, K, generator=g) * 0.02).cuda()
    calib = torch.randn(512, K, generator=g).cuda()
    H = compute_hessian_diag_approx(calib)
    w_base, w_ortho = hessian_sieve(w, H, sparsity_target=0.01)
    layer = OrthoLinear(K, N).cuda()
    layer.load_from_weights(w_base, w_ortho)
    assert int(layer.ortho_values.numel()) == int(0.01 * N * K) - 1
    x = torch.randn(M, K, generator=g).half().cuda()
    with torch.no_grad():
        for alpha in (1.0, 0.0):
            layer.set_alpha(alpha)
            y = layer(x)
            torch.cuda.synchronize()
            ref = oracle_forward(oracle_mod, layer, x, alpha)
            err = float(np.abs(y.float().cpu().numpy() - ref).max())
            assert err <= 1e-2 * float(np.abs(ref).max()), f"M={M} alpha={alpha}: {err}"


def test_libortho_c_ops_forward(gpu, oracle_mod):
    import libortho._C_ops as _C
    from libortho.torch_bind import OrthoLinear
    from libortho_amd import workloads as W
    L = W.config_layer("c1")
    d = W.to_device(L)
    x = torch.from_numpy(W.make_x(3, L.K, 21)).cuda()
    y = torch.empty(3, L.N, dtype=torch.float16, device="cuda")
    assert _C.forward(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], x, y, 1.0) is None
    torch.cuda.synchronize()
    ref = oracle_mod.forward_f64(L.q, L.scales, L.row_ptr, L.col, L.vals, W.make_x(3, L.K, 21), 1.0)
    assert float(np.abs(y.float().cpu().numpy() - ref).max()) <= 1e-2 * float(np.abs(ref).max())
    assert OrthoLinear.__module__.startswith("libortho_amd")
