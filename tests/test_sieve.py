"""The offline sieve (/root/reference/tools/sieve.py:13-95) on the CPU: the
numpy oracle pinned against closed forms and against the reference's torch
ops on CPU tensors, and the reference's import paths (README.md:64,79,
examples/basic_usage.py:15-16, setup.py:189-195) resolving to this build."""
import numpy as np
import pytest
import torch

from oracle import sieve_oracle as SO
from oracle.pack_oracle import f32_to_bf16_bits

TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def to_torch(a, dt):
    if dt == "bf16":
        return torch.from_numpy(f32_to_bf16_bits(a).view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(np.asarray(a, np.float32)).to(TORCH_DT[dt])


def from_torch(t):
    return t.float().numpy()


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return np.array_equal(a.view(np.uint32), b.view(np.uint32)) or \
        (np.array_equal(np.isnan(a), np.isnan(b)) and
         np.array_equal(a[~np.isnan(a)].view(np.uint32), b[~np.isnan(b)].view(np.uint32)))


def weights(dt, N=24, K=96, seed=0):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    w[3] = 0.0                       # all-zero row: the 1e-8 floor
    w[5, 7] = np.inf                 # an infinite weight: NaN scale, row -> 0
    w[6, :] = np.float32(1e-9)       # below the floor in FP32 and BF16
    w[8, ::5] = -w[8, ::5]
    return np.asarray(SO.round_to(dt, w), np.float32)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_quantize_oracle_equals_reference_torch_ops(dt):
    from libortho_amd.tools.sieve import quantize_int4_torch
    w = weights(dt)
    ref = from_torch(quantize_int4_torch(to_torch(w, dt)))
    got = SO.quantize_int4(w, dt, scalar_div="ieee")
    assert same_bits(got, ref)


def test_quantize_recovers_planted_grid():
    # w = q * s with s a power of two and |q| reaching 7 in every row: s is
    # recovered exactly (max|w| / 7 = s) and so is every weight
    rng = np.random.default_rng(1)
    q = rng.integers(-8, 8, size=(16, 64)).astype(np.float32)
    q[:, 0] = 7.0
    q = np.clip(q, -7, 7)
    s = (2.0 ** rng.integers(-12, -2, size=(16, 1))).astype(np.float32)
    w = q * s
    for dt in ("f32", "f16", "bf16"):
        for div in ("ieee", "reciprocal"):
            got = SO.quantize_int4(SO.round_to(dt, w), dt, scalar_div=div)
            np.testing.assert_array_equal(got, w)


def test_quantize_rounds_half_to_even_and_clamps():
    # s = 1 (max 7): w / s = 2.5 -> 2, 3.5 -> 4, -0.5 -> -0, -8.6 clamps to -8
    w = np.array([[7.0, 2.5, 3.5, -0.5, 0.49, -6.5]], np.float32)
    np.testing.assert_array_equal(SO.quantize_int4(w, "f32"), [[7.0, 2.0, 4.0, -0.0, 0.0, -6.0]])
    w = np.array([[-7.0, 1.0]], np.float32)  # max 7 -> s 1
    np.testing.assert_array_equal(SO.quantize_int4(w, "f32"), [[-7.0, 1.0]])


@pytest.mark.parametrize("dt,hdt", [("f32", "f32"), ("f16", "f32"), ("bf16", "f32"), ("f16", "f16")])
@pytest.mark.parametrize("target", [None, 0.02, 0.0])
def test_hessian_sieve_oracle_equals_reference_torch_ops(dt, hdt, target):
    from libortho_amd.tools.sieve import hessian_sieve_torch
    w = weights(dt, seed=2)
    rng = np.random.default_rng(3)
    h = SO.round_to(hdt, (rng.random(w.shape[1]) * 2 + 0.1).astype(np.float32))
    wb_t, wo_t = hessian_sieve_torch(to_torch(w, dt), to_torch(h, hdt), curvature_thresh=1e-6,
                                     sparsity_target=target)
    wb, wo, _ = SO.hessian_sieve(w, dt, h, hdt, curvature_thresh=1e-6, sparsity_target=target,
                                 scalar_div="ieee")
    assert same_bits(wb, from_torch(wb_t))
    assert same_bits(wo, from_torch(wo_t))


def test_hessian_sieve_matrix_h_takes_the_diagonal():
    from libortho_amd.tools.sieve import hessian_sieve_torch
    w = weights("f32", seed=4)
    rng = np.random.default_rng(5)
    H = rng.random((w.shape[1], w.shape[1])).astype(np.float32) + 0.5
    wb_t, wo_t = hessian_sieve_torch(to_torch(w, "f32"), to_torch(H, "f32"), sparsity_target=0.05)
    wb, wo, _ = SO.hessian_sieve(w, "f32", H, "f32", sparsity_target=0.05, scalar_div="ieee")
    assert same_bits(wo, from_torch(wo_t))


def test_hessian_sieve_selects_planted_outliers():
    # a grid weight plus 6 planted off-grid outliers: with unit curvature their
    # squared residuals are the only nonzero scores.  A target of exactly 6
    # entries puts the threshold at the smallest outlier's score, and the
    # reference keeps score > threshold (strictly, sieve.py:72): the 5 larger
    # outliers survive, the smallest and the grid do not; w_base is the grid
    rng = np.random.default_rng(6)
    q = np.clip(rng.integers(-8, 8, size=(8, 32)), -7, 7).astype(np.float32)
    q[:, 1] = 7.0
    s = np.float32(2.0 ** -6)
    w = q * s
    pos = [(0, 3), (1, 9), (2, 30), (4, 4), (6, 17), (7, 2)]
    for r, c in pos:
        q[r, c] = np.clip(q[r, c], -5, 5)             # the outlier stays below the row's max
    w = q * s
    for i, (r, c) in enumerate(pos):
        w[r, c] += s * np.float32(0.25 + 0.01 * i)   # below half a step: q unchanged
    h = np.ones(32, np.float32)
    wb, wo, score = SO.hessian_sieve(w, "f32", h, "f32", sparsity_target=len(pos) / w.size)
    np.testing.assert_array_equal(wb, q * s)
    expect = np.zeros_like(w)
    for r, c in pos[1:]:
        expect[r, c] = w[r, c] - q[r, c] * s
    np.testing.assert_array_equal(wo, expect)


def test_kth_largest_nan_is_largest():
    sc = np.array([[1.0, np.nan, 3.0, 2.0]], np.float32)
    assert np.isnan(SO._kth_largest(sc, 1))
    assert SO._kth_largest(sc, 2) == 3.0
    assert SO._kth_largest(sc, 4) == 1.0


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_hessian_diag_oracle(dt):
    from libortho_amd.tools.sieve import compute_hessian_diag_approx_torch
    rng = np.random.default_rng(7)
    x = SO.round_to(dt, rng.standard_normal((300, 40)).astype(np.float32))
    got = SO.compute_hessian_diag_approx(x, dt, scalar_div="ieee")
    closed = (x.astype(np.float64) ** 2).sum(0) / 300 + 1e-6
    tol = {"f32": 1e-6, "f16": 2e-3, "bf16": 1.6e-2}[dt]
    np.testing.assert_allclose(got, closed, rtol=tol)
    ref = from_torch(compute_hessian_diag_approx_torch(to_torch(x, dt)))
    np.testing.assert_allclose(got, ref, rtol=tol)


def test_reference_import_paths():
    import libortho._C_ops as _C
    import libortho.torch_bind as lt
    import torch_bind
    from libortho.tools import compute_hessian_diag_approx as c1, hessian_sieve as h1
    from libortho.tools.sieve import pack_ortho_sparse as p1, quantize_int4 as q1
    from libortho_amd.tools import sieve
    from libortho_amd.torch_bind.ortho_linear import OrthoLinear as Native
    from tools.sieve import compute_hessian_diag_approx, hessian_sieve, pack_ortho_sparse, quantize_int4
    from torch_bind.ortho_linear import OrthoLinear
    assert hasattr(_C, "forward")
    assert OrthoLinear is Native and torch_bind.OrthoLinear is Native and lt.OrthoLinear is Native
    assert hessian_sieve is sieve.hessian_sieve is h1
    assert compute_hessian_diag_approx is sieve.compute_hessian_diag_approx is c1
    assert quantize_int4 is sieve.quantize_int4 is q1
    assert pack_ortho_sparse is sieve.pack_ortho_sparse is p1
    import tools
    assert tools.sieve is sieve


def test_reference_example_flow_on_cpu_tensors():
    """examples/basic_usage.py:20-60's separation step through the
    reference's import path, on CPU tensors (the torch-op form)."""
    from tools.sieve import compute_hessian_diag_approx, hessian_sieve, pack_ortho_sparse
    torch.manual_seed(0)
    w = torch.randn(64, 64)
    x = torch.randn(200, 64)
    H = compute_hessian_diag_approx(x)
    wb, wo = hessian_sieve(w, H, sparsity_target=0.05)
    assert wb.shape == w.shape and wo.shape == w.shape
    k = int(0.05 * w.numel())
    assert int((wo != 0).sum()) == k - 1      # strictly above the k-th largest score
    rp, col, vals = pack_ortho_sparse(wo, "csr")
    assert int(rp[-1]) == k - 1
