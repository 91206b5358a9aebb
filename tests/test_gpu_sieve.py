"""The offline sieve's kernels (orth_sieve.hip) on the GPU, checked against
the numpy oracle (oracle/sieve_oracle.py) and against the outputs of the
reference's own functions on CPU tensors (tests/golden/sieve_cases.npz):

* GPU tensors: torch divides a GPU tensor by a host scalar as a product with
  the FP32 reciprocal; the oracle's "reciprocal" mode models that, and one
  torch division on the GPU pins the model.  quantize_int4 and hessian_sieve
  bit for bit against that mode; the Hessian diagonal within FP32
  summation-order error.
* CPU tensors: the product copies them to the GPU and runs the kernels with
  IEEE division; the results equal the reference's CPU outputs bit for bit
  (the diagonal to FP32 summation order)."""
import os

import numpy as np
import pytest
import torch

from oracle import sieve_oracle as SO

pytestmark = pytest.mark.gpu

TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
HS_COMBOS = [("f32", "f32"), ("f16", "f32"), ("bf16", "f32"), ("f16", "f16"), ("bf16", "bf16"), ("f32", "f16")]
HS_TARGETS = [("none", None), ("t02", 0.02), ("t0", 0.0), ("t1e4", 1e-4), ("t50", 0.5)]


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


def gold_tensor(gold, key, dt):
    """A fixture array as a CPU tensor of dtype dt (bit patterns restored)."""
    a = gold[key]
    if dt == "f32":
        return torch.from_numpy(a.astype(np.float32))
    return torch.from_numpy(a.view(np.int16).copy()).view(TD[dt])


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(os.path.dirname(__file__), "golden", "sieve_cases.npz"))


def test_gpu_scalar_division_is_the_reciprocal_product(gpu):
    """Pins the oracle's model of torch on a GPU tensor: t / 7.0 and t / n
    round t * fp32(1 / d), which differs from IEEE division for these m."""
    m = torch.arange(1, 4000, dtype=torch.float32) * 0.37
    for d in (7.0, 300.0):
        got = (m.to(gpu) / d).cpu().numpy()
        rec = SO._scalar_div("f32", m.numpy(), d, "reciprocal")
        ieee = SO._scalar_div("f32", m.numpy(), d, "ieee")
        assert np.array_equal(got.view(np.uint32), rec.view(np.uint32))
        assert not np.array_equal(got.view(np.uint32), ieee.view(np.uint32))


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", [(64, 4096), (37, 1000), (16, 11008)])
def test_quantize_int4_matches_oracle(gpu, dt, shape):
    from libortho_amd import _C_ops
    from libortho_amd.tools.sieve import quantize_int4
    w = make_w(dt, *shape, seed=1, device=gpu)
    got = quantize_int4(w)
    torch.cuda.synchronize()
    assert got.dtype == w.dtype and got.shape == w.shape and got.is_cuda
    ref = SO.quantize_int4(w.float().cpu().numpy(), dt)
    assert bits_equal(got, torch.from_numpy(ref))
    assert bits_equal(got, _C_ops.sieve_quantize(w))


@pytest.mark.parametrize("dt,hdt", [("f32", "f32"), ("f16", "f32"), ("bf16", "f32"), ("f16", "f16"),
                                    ("bf16", "bf16")])
@pytest.mark.parametrize("target", [None, 0.01, 0.0, 1e-7])
def test_hessian_sieve_matches_oracle(gpu, dt, hdt, target):
    from libortho_amd.tools.sieve import hessian_sieve
    w = make_w(dt, 96, 2048, seed=2, device=gpu)
    g = torch.Generator(device="cpu").manual_seed(3)
    h = (torch.rand(2048, generator=g) * 2 + 0.05).to(TD[hdt]).to(gpu)
    thresh = 2e-6
    wb, wo = hessian_sieve(w, h, curvature_thresh=thresh, sparsity_target=target)
    torch.cuda.synchronize()
    wb_o, wo_o, _ = SO.hessian_sieve(w.float().cpu().numpy(), dt, h.float().cpu().numpy(), hdt,
                                     curvature_thresh=thresh, sparsity_target=target)
    assert bits_equal(wb, torch.from_numpy(wb_o))
    assert bits_equal(wo, torch.from_numpy(wo_o))


def test_hessian_sieve_matrix_h_and_ties(gpu):
    """H_inv given as a matrix (its diagonal is used) and a score with many
    exact ties at the threshold (the k-th largest value is the same whatever
    order a select breaks ties in)."""
    from libortho_amd.tools.sieve import hessian_sieve
    K = 512
    q = torch.randint(-7, 8, (64, K), dtype=torch.float32)
    q[:, 0] = 7.0
    w = q * 2.0 ** -5
    w[:, 1::7] += 2.0 ** -7            # identical residuals: thousands of tied scores
    H = torch.rand(K, K) + torch.eye(K)
    for target in (0.01, 0.1, 0.5):
        wb, wo = hessian_sieve(w.to(gpu), H.to(gpu), sparsity_target=target)
        wb_o, wo_o, _ = SO.hessian_sieve(w.numpy(), "f32", H.numpy(), "f32", sparsity_target=target)
        assert bits_equal(wb, torch.from_numpy(wb_o)) and bits_equal(wo, torch.from_numpy(wo_o))


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", [(1000, 128), (4096, 4096), (3, 11008)])
def test_hessian_diag_matches_oracle(gpu, dt, shape):
    from libortho_amd.tools.sieve import compute_hessian_diag_approx
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


# ----------------------------------------- CPU tensors: the reference's outputs

@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_cpu_tensor_quantize_equals_reference_outputs(gpu, gold, dt):
    from tools.sieve import quantize_int4
    w = gold_tensor(gold, f"quant_{dt}_w", dt)
    got = quantize_int4(w)
    assert got.device.type == "cpu" and got.dtype == w.dtype
    assert bits_equal(got, gold_tensor(gold, f"quant_{dt}_out", dt))


@pytest.mark.parametrize("dt,hdt", HS_COMBOS)
def test_cpu_tensor_hessian_sieve_equals_reference_outputs(gpu, gold, dt, hdt):
    from tools.sieve import hessian_sieve
    w, h = gold_tensor(gold, f"hs_{dt}_{hdt}_w", dt), gold_tensor(gold, f"hs_{dt}_{hdt}_h", hdt)
    cases = [(n, dict(curvature_thresh=2e-6, sparsity_target=t)) for n, t in HS_TARGETS]
    cases.append(("mid", dict(curvature_thresh=2.1e-5)))
    cases.append(("edge", dict(curvature_thresh=float(gold[f"hs_{dt}_{hdt}_edge_t"][0]))))
    for name, kw in cases:
        wb, wo = hessian_sieve(w, h, **kw)
        assert wb.device.type == "cpu" and wo.device.type == "cpu"
        assert bits_equal(wb, gold_tensor(gold, f"hs_{dt}_{hdt}_{name}_wb", dt)), name
        assert bits_equal(wo, gold_tensor(gold, f"hs_{dt}_{hdt}_{name}_wo", dt)), name


def test_cpu_tensor_matrix_h_and_ties_equal_reference_outputs(gpu, gold):
    from tools.sieve import hessian_sieve
    w, H = torch.from_numpy(gold["hsm_w"]), torch.from_numpy(gold["hsm_H"])
    for name, t in (("t01", 0.01), ("t10", 0.1), ("t50", 0.5)):
        wb, wo = hessian_sieve(w, H, sparsity_target=t)
        assert bits_equal(wb, torch.from_numpy(gold[f"hsm_{name}_wb"]))
        assert bits_equal(wo, torch.from_numpy(gold[f"hsm_{name}_wo"]))


def test_cpu_tensor_hessian_diag_equals_reference_outputs(gpu, gold):
    from tools.sieve import compute_hessian_diag_approx
    for key in gold.files:
        if not (key.startswith("hd_") and key.endswith("_x")):
            continue
        dt = key.split("_")[1]
        got = compute_hessian_diag_approx(gold_tensor(gold, key, dt))
        ref = gold_tensor(gold, key[:-2] + "_out", dt)
        assert got.device.type == "cpu" and got.dtype == ref.dtype
        if dt == "f32":
            np.testing.assert_allclose(got.numpy(), ref.numpy(), rtol=2e-6)
        else:
            assert bits_equal(got, ref), key


def test_reference_example_flow_on_cpu_tensors(gpu):
    """examples/basic_usage.py:20-60's separation step through the
    reference's import path, on CPU tensors (split on the GPU)."""
    from tools.sieve import compute_hessian_diag_approx, hessian_sieve, pack_ortho_sparse
    torch.manual_seed(0)
    w = torch.randn(64, 64)
    x = torch.randn(200, 64)
    H = compute_hessian_diag_approx(x)
    wb, wo = hessian_sieve(w, H, sparsity_target=0.05)
    assert wb.shape == w.shape and wo.shape == w.shape and wo.device.type == "cpu"
    k = int(0.05 * w.numel())
    assert int((wo != 0).sum()) == k - 1      # strictly above the k-th largest score
    rp, col, vals = pack_ortho_sparse(wo, "csr")
    assert int(rp[-1]) == k - 1
    wb_o, wo_o, _ = SO.hessian_sieve(w.numpy(), "f32", H.numpy(), "f32", sparsity_target=0.05,
                                     scalar_div="ieee")
    assert bits_equal(wo, torch.from_numpy(wo_o))
