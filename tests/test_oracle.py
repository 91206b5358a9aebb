"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each oracle function is checked against something independent of its own
formula: the reference's golden outputs (tests/golden/ref_coo_cases.npz,
written by the reference's compiled orth_layer_forward), the reference's
compiled code itself when oracle/_ref is built, closed forms, and a numpy
float64 brute force that dequantises the whole matrix and calls matmul.
The last group plants plausible mistakes in the oracle's inputs and shows
that the checks catch them.
"""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_coo_cases.npz")
CASES = ["testcpu_a1", "testcpu_a0", "testcpu_empty", "rand_96x128_m3", "rand_40x200_m5",
         "rand_256x256_m1"]


def golden(name):
    d = np.load(GOLDEN)
    return {k.split("__", 1)[1]: d[k] for k in d.files if k.startswith(name + "__")}


def np_unpack(q: np.ndarray) -> np.ndarray:
    """Independent numpy nibble decode: [N, K/2] uint8 -> [N, K] int."""
    lo = (q & 0xF).astype(np.int16)
    hi = (q >> 4).astype(np.int16)
    w = np.empty((q.shape[0], q.shape[1] * 2), np.int16)
    w[:, 0::2] = lo
    w[:, 1::2] = hi
    return np.where(w >= 8, w - 16, w)


def coo_to_csr(idx, vals, N, K):
    """Keeps duplicates and, within a row, the COO order (stable)."""
    idx = idx.astype(np.int64)
    rows, cols = idx // K, idx % K
    keep = rows < N
    rows, cols, vals = rows[keep], cols[keep], vals[keep]
    order = np.argsort(rows, kind="stable")
    row_ptr = np.zeros(N + 1, np.int32)
    row_ptr[1:] = np.cumsum(np.bincount(rows, minlength=N))
    return row_ptr, cols[order].astype(np.int32), vals[order]


def np_forward_f64(q, scales, row_ptr, col, vals, x, alpha):
    N, K = q.shape[0], q.shape[1] * 2
    s = np.asarray(scales, np.float64).reshape(N, -1)
    W = np_unpack(q).astype(np.float64) * np.repeat(s, K // s.shape[1], axis=1)
    y = np.asarray(x, np.float64) @ W.T
    if alpha > 0 and len(vals):
        S = np.zeros((N, K))
        rows = np.repeat(np.arange(N), np.diff(row_ptr))
        ok = (col >= 0) & (col < K)
        np.add.at(S, (rows[ok], col[ok]), np.asarray(vals, np.float64)[ok])
        y += alpha * (np.asarray(x, np.float64) @ S.T)
    return y


def rand_layer(rng, N, K, groups, density, dup=False):
    q = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    scales = np.abs(rng.normal(0, 0.02, size=(N, groups))).astype(np.float16)
    nnz = max(1, int(density * N * K))
    if dup:
        flat = rng.integers(0, N * K, size=nnz)
    else:
        flat = np.sort(rng.choice(N * K, size=nnz, replace=False))
    rows = flat // K
    order = np.argsort(rows, kind="stable")
    row_ptr = np.zeros(N + 1, np.int32)
    row_ptr[1:] = np.cumsum(np.bincount(rows, minlength=N))
    col = (flat % K)[order].astype(np.int32)
    vals = rng.normal(0, 0.05, size=nnz).astype(np.float16)
    return q, scales, row_ptr, col, vals


# ------------------------------------------------------------ closed forms

def test_unpack_int4_exhaustive(oracle_mod):
    packed = np.arange(256, dtype=np.uint8)
    for b in range(256):
        for half, nib in ((0, b & 0xF), (1, b >> 4)):
            expect = nib - 16 if nib >= 8 else nib
            assert oracle_mod.unpack_int4(packed, 2 * b + half) == expect


def test_dequant_closed_form_bit_exact(oracle_mod):
    rng = np.random.default_rng(1)
    for groups in (1, 4, 32):
        q = rng.integers(0, 256, size=(37, 64), dtype=np.uint8)
        s = np.abs(rng.normal(0, 0.02, size=(37, groups))).astype(np.float16)
        got = oracle_mod.dequant_f32(q, s)
        s32 = np.repeat(s.astype(np.float32), 128 // groups, axis=1)
        expect = np_unpack(q).astype(np.float32) * s32
        assert got.dtype == np.float32
        assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))


def test_f16_converter_matches_ieee(oracle_mod):
    rng = np.random.default_rng(2)
    v = np.concatenate([rng.normal(0, 1, 5000), rng.normal(0, 1e-5, 2000),
                        rng.normal(0, 3e4, 2000),
                        [0.0, -0.0, 65504.0, 65520.0, 65519.99, 1e-8, 5.96e-8, 2.98e-8,
                         np.inf, -np.inf, 6.1e-5, 6.09e-5]]).astype(np.float32)
    got = oracle_mod.f32_to_f16_bits(v)
    with np.errstate(over="ignore"):
        expect = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, expect)


# ------------------------------------------------- reference golden vectors

@pytest.mark.parametrize("case", CASES)
def test_coo_forward_matches_reference_golden(oracle_mod, case):
    g = golden(case)
    y = oracle_mod.forward_ref_coo_f32(g["q"], g["scales"], g["idx"], g["vals"], g["x"],
                                       float(g["alpha"]))
    # the reference's own test tolerance, tests/test_cpu_forward.c:214
    np.testing.assert_allclose(y, g["y"], atol=1e-4, rtol=1e-5)


@pytest.mark.parametrize("case", CASES)
def test_csr_forward_matches_reference_golden(oracle_mod, case):
    g = golden(case)
    N, K = g["q"].shape[0], g["q"].shape[1] * 2
    row_ptr, col, vals = coo_to_csr(g["idx"], g["vals"], N, K)
    alpha = float(g["alpha"])
    y32 = oracle_mod.forward_ref_f32(g["q"], g["scales"], row_ptr, col, vals, g["x"], alpha)
    y64 = oracle_mod.forward_f64(g["q"], g["scales"], row_ptr, col, vals, g["x"], alpha)
    np.testing.assert_allclose(y32, g["y"], atol=1e-4, rtol=1e-5)
    np.testing.assert_allclose(y64, g["y"], atol=1e-4, rtol=1e-5)


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(__file__), "..", "oracle",
                                                    "_ref", "libortho_ref.so")),
                    reason="oracle/_ref (the reference's compiled CPU path) is not built here")
def test_oracle_matches_reference_compiled_code(oracle_mod):
    rng = np.random.default_rng(3)
    for (N, K, M) in ((64, 64, 4), (33, 250, 2), (128, 512, 1), (200, 300, 3)):
        q = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
        s = rng.uniform(0.1, 1.0, size=N).astype(np.float32)
        cnt = max(1, (N * K) // 40)
        idx = rng.integers(0, min(N * K, 65536), size=cnt).astype(np.uint16)
        v = rng.normal(0, 0.05, size=cnt).astype(np.float32)
        x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
        for alpha in (1.0, 0.5, 0.0, -1.0):
            ref = oracle_mod.ref_forward_coo(q, s, idx, v, x, alpha)
            mine = oracle_mod.forward_ref_coo_f32(q, s, idx, v, x, alpha)
            np.testing.assert_allclose(mine, ref, atol=1e-4, rtol=1e-5)


# ------------------------------------------- float64 brute force (numpy)

@pytest.mark.parametrize("groups", [1, 2, 16])
@pytest.mark.parametrize("alpha", [1.0, 0.5])
def test_f64_oracle_equals_numpy_brute_force(oracle_mod, groups, alpha):
    rng = np.random.default_rng(10 + groups)
    N, K, M = 45, 96, 3
    q, s, rp, col, vals = rand_layer(rng, N, K, groups, 0.05, dup=True)
    x = rng.normal(0, 1, size=(M, K)).astype(np.float16)
    y = oracle_mod.forward_f64(q, s, rp, col, vals, x, alpha)
    ref = np_forward_f64(q, s, rp, col, vals, x, alpha)
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)
    y32 = oracle_mod.forward_ref_f32(q, s, rp, col, vals, x, alpha)
    np.testing.assert_allclose(y32, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())


def test_group_scales_with_g_equal_k_is_per_row(oracle_mod):
    rng = np.random.default_rng(4)
    q, s, rp, col, vals = rand_layer(rng, 20, 64, 1, 0.1)
    x = rng.normal(0, 1, size=(2, 64)).astype(np.float16)
    a = oracle_mod.forward_ref_f32(q, s.reshape(20), rp, col, vals, x, 1.0)
    b = oracle_mod.forward_ref_f32(q, s.reshape(20, 1), rp, col, vals, x, 1.0)
    assert np.array_equal(a, b)


def test_alpha_gate_and_empty_ortho(oracle_mod):
    # the reference's gate alpha > 0 && count > 0 (src/ortho.c:343); its test
    # checks alpha = 0 == empty ortho == base only (tests/test_cpu_forward.c:221-319)
    rng = np.random.default_rng(5)
    q, s, rp, col, vals = rand_layer(rng, 30, 64, 4, 0.1)
    x = rng.normal(0, 1, size=(3, 64)).astype(np.float16)
    base = oracle_mod.forward_ref_f32(q, s, None, None, None, x, 1.0)
    for alpha in (0.0, -1.0, -0.0, float("nan")):
        assert np.array_equal(oracle_mod.forward_ref_f32(q, s, rp, col, vals, x, alpha), base)
    full = oracle_mod.forward_ref_f32(q, s, rp, col, vals, x, 1.0)
    assert not np.allclose(full, base)


def test_column_guard_skips_out_of_range(oracle_mod):
    rng = np.random.default_rng(6)
    q, s, rp, col, vals = rand_layer(rng, 10, 32, 1, 0.2)
    x = rng.normal(0, 1, size=(1, 32)).astype(np.float16)
    bad = col.copy()
    bad[::3] = 32 + np.arange(len(bad[::3]))  # out of range: skipped
    keep_vals = vals.copy()
    keep_vals[::3] = 0
    a = oracle_mod.forward_f64(q, s, rp, bad, vals, x, 1.0)
    b = oracle_mod.forward_f64(q, s, rp, col, keep_vals, x, 1.0)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)


def test_cpu_baseline_restatement_agrees(oracle_mod):
    rng = np.random.default_rng(7)
    q, s, rp, col, vals = rand_layer(rng, 64, 256, 2, 0.02)
    x = rng.normal(0, 1, size=(2, 256)).astype(np.float16)
    t, yb = oracle_mod.baseline_time(q, s, rp, col, vals, x, 1.0, 1, 2)
    ref = oracle_mod.forward_f64(q, s, rp, col, vals, x, 1.0)
    assert t > 0
    np.testing.assert_allclose(yb, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())


# ---------------------------------------------------- the checks have teeth

def _fails(y, expect):
    return not np.allclose(y, expect, atol=1e-4, rtol=1e-5)


def test_planted_mistakes_are_caught(oracle_mod):
    g = golden("testcpu_a1")
    q, s, idx, v, x = g["q"], g["scales"], g["idx"], g["vals"], g["x"]
    # 1. nibble order swapped (high nibble taken as the even element)
    q_sw = ((q & 0xF) << 4) | (q >> 4)
    assert _fails(oracle_mod.forward_ref_coo_f32(q_sw, s, idx, v, x, 1.0), g["y"])
    x64 = x.astype(np.float64)
    S = np.zeros((64, 64))
    np.add.at(S, (idx.astype(np.int64) // 64, idx.astype(np.int64) % 64), v)
    sparse = x64 @ S.T
    W = np_unpack(q).astype(np.float64)
    # the brute force itself reproduces the golden output ...
    assert not _fails(x64 @ (W * s[:, None]).T + sparse, g["y"])
    # 2. ... but not with the sign extension dropped (nibbles read as 0..15)
    W_uns = np.where(W < 0, W + 16, W) * s[:, None]
    assert _fails(x64 @ W_uns.T + sparse, g["y"])
    # 3. ... nor with the weight operand transposed (square case)
    assert _fails(x64 @ (W * s[:, None]) + sparse, g["y"])
    # 4. ortho term dropped
    assert _fails(oracle_mod.forward_ref_coo_f32(q, s, idx, v, x, 0.0), g["y"])
    # 5. sparse row/col swapped
    flat = idx.astype(np.int64)
    idx_sw = ((flat % 64) * 64 + flat // 64).astype(np.uint16)
    assert _fails(oracle_mod.forward_ref_coo_f32(q, s, idx_sw, v, x, 1.0), g["y"])
    # 6. sign of the ortho term flipped
    assert _fails(oracle_mod.forward_ref_coo_f32(q, s, idx, -v, x, 1.0), g["y"])
