"""The offline sieve (/root/reference/tools/sieve.py:13-95) on the CPU: the
numpy oracle pinned against closed forms and against the outputs the
reference's own functions gave on CPU tensors (tests/golden/sieve_cases.npz,
written by tests/golden/make_sieve_golden.py in the build container), and
the reference's import paths (README.md:64,79, examples/basic_usage.py:15-16,
setup.py:189-195) resolving to this build."""
import os

import numpy as np
import pytest
import torch

from oracle import sieve_oracle as SO
from oracle.pack_oracle import bf16_bits_to_f32


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return np.array_equal(a.view(np.uint32), b.view(np.uint32)) or \
        (np.array_equal(np.isnan(a), np.isnan(b)) and
         np.array_equal(a[~np.isnan(a)].view(np.uint32), b[~np.isnan(b)].view(np.uint32)))


GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "sieve_cases.npz"))
HS_COMBOS = [("f32", "f32"), ("f16", "f32"), ("bf16", "f32"), ("f16", "f16"), ("bf16", "bf16"), ("f32", "f16")]
HS_TARGETS = [("none", None), ("t02", 0.02), ("t0", 0.0), ("t1e4", 1e-4), ("t50", 0.5)]


def gold(key, dt):
    """A fixture array as FP32 values (FP16 / BF16 stored as bit patterns)."""
    a = GOLD[key]
    if dt == "f16":
        return a.view(np.float16).astype(np.float32)
    if dt == "bf16":
        return bf16_bits_to_f32(a)
    return a.astype(np.float32)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_quantize_oracle_equals_reference_outputs(dt):
    """The reference's quantize_int4 on CPU tensors (tests/golden/
    make_sieve_golden.py): zero, infinite, NaN and sub-floor rows, exact
    half steps, FP16/BF16 intermediate rounding."""
    w = gold(f"quant_{dt}_w", dt)
    assert same_bits(SO.quantize_int4(w, dt, scalar_div="ieee"), gold(f"quant_{dt}_out", dt))


def test_quantize_fixtures_reject_planted_mistakes():
    # the FP32 fixture tells IEEE division from the reciprocal product, the
    # FP16 / BF16 ones tell rounding each step to the dtype from FP32 math
    w = gold("quant_f32_w", "f32")
    assert not same_bits(SO.quantize_int4(w, "f32", scalar_div="reciprocal"), gold("quant_f32_out", "f32"))
    for dt in ("f16", "bf16"):
        w = gold(f"quant_{dt}_w", dt)
        planted = SO.round_to(dt, SO.quantize_int4(w, "f32", scalar_div="ieee"))
        assert not same_bits(planted, gold(f"quant_{dt}_out", dt))


@pytest.mark.parametrize("dt,hdt", HS_COMBOS)
def test_hessian_sieve_oracle_equals_reference_outputs(dt, hdt):
    """hessian_sieve on CPU tensors: both threshold branches (k-th largest
    score with k = 0, small and large; a host threshold below, inside and at
    the edge of the score distribution), dtype promotion of the score."""
    w, h = gold(f"hs_{dt}_{hdt}_w", dt), gold(f"hs_{dt}_{hdt}_h", hdt)
    cases = [(n, dict(curvature_thresh=2e-6, sparsity_target=t)) for n, t in HS_TARGETS]
    cases.append(("mid", dict(curvature_thresh=2.1e-5)))
    cases.append(("edge", dict(curvature_thresh=float(GOLD[f"hs_{dt}_{hdt}_edge_t"][0]))))
    for name, kw in cases:
        wb, wo, _ = SO.hessian_sieve(w, dt, h, hdt, scalar_div="ieee", **kw)
        assert same_bits(wb, gold(f"hs_{dt}_{hdt}_{name}_wb", dt)), name
        assert same_bits(wo, gold(f"hs_{dt}_{hdt}_{name}_wo", dt)), name


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_hessian_sieve_fixture_rejects_unrounded_threshold(dt):
    # the edge threshold sits just below a score value v and rounds to v in
    # the score's dtype: keeping it in FP32 keeps the entries scoring v
    t = float(GOLD[f"hs_{dt}_{dt}_edge_t"][0])
    w, h = gold(f"hs_{dt}_{dt}_w", dt), gold(f"hs_{dt}_{dt}_h", dt)
    wb, _, score = SO.hessian_sieve(w, dt, h, dt, curvature_thresh=t, scalar_div="ieee")
    planted = SO.round_to(dt, SO.round_to(dt, w - wb) * (score > np.float32(t)))
    assert not same_bits(planted, gold(f"hs_{dt}_{dt}_edge_wo", dt))


def test_hessian_sieve_matrix_h_and_tied_scores_equal_reference():
    w, H = GOLD["hsm_w"], GOLD["hsm_H"]
    for name, t in (("t01", 0.01), ("t10", 0.1), ("t50", 0.5)):
        wb, wo, _ = SO.hessian_sieve(w, "f32", H, "f32", sparsity_target=t, scalar_div="ieee")
        assert same_bits(wb, GOLD[f"hsm_{name}_wb"]) and same_bits(wo, GOLD[f"hsm_{name}_wo"]), name


def test_hessian_diag_oracle_equals_reference_outputs():
    # torch forms the full X^T X with its own FP32 summation order: a few
    # FP32 ulps apart from the oracle's FP64 sum, equal after FP16 / BF16 rounding
    for key in GOLD.files:
        if not (key.startswith("hd_") and key.endswith("_x")):
            continue
        dt = key.split("_")[1]
        got = SO.compute_hessian_diag_approx(gold(key, dt), dt, scalar_div="ieee")
        ref = gold(key[:-2] + "_out", dt)
        if dt == "f32":
            np.testing.assert_allclose(got, ref, rtol=2e-6)
        else:
            assert same_bits(got, ref), key


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
def test_hessian_diag_oracle_closed_form(dt):
    rng = np.random.default_rng(7)
    x = SO.round_to(dt, rng.standard_normal((300, 40)).astype(np.float32))
    got = SO.compute_hessian_diag_approx(x, dt, scalar_div="ieee")
    closed = (x.astype(np.float64) ** 2).sum(0) / 300 + 1e-6
    tol = {"f32": 1e-6, "f16": 2e-3, "bf16": 1.6e-2}[dt]
    np.testing.assert_allclose(got, closed, rtol=tol)
    # constant columns: diag = c^2 exactly when c^2 * n is exact
    c = np.full((64, 3), 0.5, np.float32)
    np.testing.assert_array_equal(SO.compute_hessian_diag_approx(c, "f32", scalar_div="ieee"),
                                  np.float32(np.float32(0.25) + np.float32(1e-6)))


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


@pytest.mark.skipif(torch.cuda.is_available(), reason="the CPU-tensor sieve runs on the GPU when one exists")
def test_sieve_on_cpu_tensors_without_a_gpu_raises():
    """The sieve has no CPU implementation in the product: CPU tensors are
    split by the GPU kernels, and without a GPU the call raises."""
    from tools.sieve import compute_hessian_diag_approx, hessian_sieve, quantize_int4
    w = torch.randn(8, 16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        quantize_int4(w)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        hessian_sieve(w, torch.ones(16), sparsity_target=0.1)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        compute_hessian_diag_approx(torch.randn(4, 16))
    with pytest.raises(TypeError):
        quantize_int4(w.double())
