"""The offline sieve's kernels (orth_sieve.hip) against the reference's
torch ops run on the same GPU tensors (/root/reference/tools/sieve.py:13-95)
and against the numpy oracle: quantize_int4 and hessian_sieve bit for bit,
the Hessian diagonal within FP32 summation-order error."""
import numpy as np
import pytest
import torch

from oracle import sieve_oracle as SO

pytestmark = pytest.mark.gpu

TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    a, b = a.float().cpu(), b.float().cpu()
    na, nb = torch.isnan(a), torch.isnan(b)
    if not torch.equal(na, nb):
        return False
    return torch.equal(a[~na].view(torch.int32), b[~nb].view(torch.int32))


def make_w(dt, N, K, seed, device):
    g = torch.Generator(device="cpu").manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.05
    w[3] = 0.0
    w[5, 7] = float("inf")
    w[6, :] = 1e-9
    w[8, 11] = float("nan")
    return w.to(TD[dt]).to(device)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", [(64, 4096), (37, 1000), (16, 11008)])
def test_quantize_int4_matches_torch_ops(gpu, dt, shape):
    from libortho_amd import _C_ops
    from libortho_amd.tools.sieve import quantize_int4, quantize_int4_torch
    w = make_w(dt, *shape, seed=1, device=gpu)
    got = quantize_int4(w)
    torch.cuda.synchronize()
    assert got.dtype == w.dtype and got.shape == w.shape
    assert bits_equal(got, quantize_int4_torch(w))
    assert bits_equal(got, _C_ops.sieve_quantize(w))
    ref = SO.quantize_int4(w.float().cpu().numpy(), dt)
    assert bits_equal(got, torch.from_numpy(ref))


@pytest.mark.parametrize("dt,hdt", [("f32", "f32"), ("f16", "f32"), ("bf16", "f32"), ("f16", "f16"),
                                    ("bf16", "bf16")])
@pytest.mark.parametrize("target", [None, 0.01, 0.0, 1e-7])
def test_hessian_sieve_matches_torch_ops(gpu, dt, hdt, target):
    from libortho_amd.tools.sieve import hessian_sieve, hessian_sieve_torch
    w = make_w(dt, 96, 2048, seed=2, device=gpu)
    g = torch.Generator(device="cpu").manual_seed(3)
    h = (torch.rand(2048, generator=g) * 2 + 0.05).to(TD[hdt]).to(gpu)
    thresh = 2e-6
    wb, wo = hessian_sieve(w, h, curvature_thresh=thresh, sparsity_target=target)
    wb_t, wo_t = hessian_sieve_torch(w, h, curvature_thresh=thresh, sparsity_target=target)
    torch.cuda.synchronize()
    assert bits_equal(wb, wb_t)
    assert bits_equal(wo, wo_t)
    _, wo_o, _ = SO.hessian_sieve(w.float().cpu().numpy(), dt, h.float().cpu().numpy(), hdt,
                                  curvature_thresh=thresh, sparsity_target=target)
    assert bits_equal(wo, torch.from_numpy(wo_o))


def test_hessian_sieve_matrix_h_and_ties(gpu):
    """H_inv given as a matrix (its diagonal is used) and a score with many
    exact ties at the threshold (the k-th largest value is the same whatever
    order topk breaks ties in)."""
    from libortho_amd.tools.sieve import hessian_sieve, hessian_sieve_torch
    K = 512
    q = torch.randint(-7, 8, (64, K), dtype=torch.float32)
    q[:, 0] = 7.0
    w = q * 2.0 ** -5
    w[:, 1::7] += 2.0 ** -7            # identical residuals: thousands of tied scores
    w = w.to(gpu)
    H = torch.rand(K, K) + torch.eye(K)
    H = H.to(gpu)
    for target in (0.01, 0.1, 0.5):
        wb, wo = hessian_sieve(w, H, sparsity_target=target)
        wb_t, wo_t = hessian_sieve_torch(w, H, sparsity_target=target)
        assert bits_equal(wb, wb_t) and bits_equal(wo, wo_t)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", [(1000, 128), (4096, 4096), (3, 11008)])
def test_hessian_diag_matches_torch(gpu, dt, shape):
    from libortho_amd.tools.sieve import compute_hessian_diag_approx, compute_hessian_diag_approx_torch
    g = torch.Generator(device="cpu").manual_seed(4)
    x = torch.randn(*shape, generator=g).to(TD[dt]).to(gpu)
    got = compute_hessian_diag_approx(x)
    torch.cuda.synchronize()
    assert got.dtype == x.dtype and got.shape == (shape[1],)
    ref = SO.compute_hessian_diag_approx(x.float().cpu().numpy(), dt)
    # FP32 partial sums over at most 4096 rows vs an FP64 sum: a few FP32
    # ulps, then the result's own rounding (one step of FP16 / BF16)
    tol = {"f32": 2e-6, "f16": 1e-3, "bf16": 8e-3}[dt]
    np.testing.assert_allclose(got.float().cpu().numpy(), ref, rtol=tol)
    tt = compute_hessian_diag_approx_torch(x).float().cpu().numpy()
    np.testing.assert_allclose(got.float().cpu().numpy(), tt, rtol=max(tol, 2e-5))
