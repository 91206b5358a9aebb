"""The packing oracle (oracle/pack_oracle.py) pinned on the CPU: closed
forms, a library routine for the CSR (scipy.sparse), and the outputs the
reference's own load_from_weights and pack_ortho_sparse gave on CPU tensors
(tests/golden/pack_cases.npz, written by tests/golden/make_sieve_golden.py
from /root/reference/torch_bind/ortho_linear.py:79-128 and
/root/reference/tools/sieve.py:119-152): FP16 / BF16 weights whose W / s
rounds across a half step in the dtype, given FP16 and FP32 scales, the
1e-6 floor.  The product's CPU packers (pack_base_torch,
pack_ortho_sparse_torch) are checked against the oracle."""
import os

import numpy as np
import pytest
import scipy.sparse as sp
import torch

from libortho_amd.tools.sieve import pack_ortho_sparse_torch
from libortho_amd.torch_bind.ortho_linear import pack_base_torch
from oracle import pack_oracle as PO


def unpack(packed: np.ndarray) -> np.ndarray:
    b = packed.reshape(packed.shape[0], -1).astype(np.int16)
    lo, hi = b & 15, b >> 4
    q = np.stack([lo, hi], axis=-1).reshape(packed.shape[0], -1)
    return np.where(q >= 8, q - 16, q).astype(np.int8)


def to_torch(w: np.ndarray, dtype: str) -> torch.Tensor:
    if dtype == "bf16":
        return torch.from_numpy(w.astype(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(w)


def from_torch(t: torch.Tensor, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return t.view(torch.int16).numpy().astype(np.uint16)
    return t.numpy()


def random_dense(rng, N, K, dtype, scale=1.0):
    w = (rng.standard_normal((N, K)) * scale).astype(np.float32)
    if dtype == "f16":
        return w.astype(np.float16)
    if dtype == "bf16":
        return PO.f32_to_bf16_bits(w)
    return w


GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "pack_cases.npz"))


def gold_dense(key, dtype):
    """A fixture weight in the oracle's input form (BF16 as bit patterns)."""
    a = GOLD[key]
    return a.view(np.float16) if dtype == "f16" else a


@pytest.mark.parametrize("dtype", PO.DTYPES)
def test_pack_base_oracle_equals_reference_load_from_weights(dtype):
    w = gold_dense(f"lw_{dtype}_w", dtype)
    q, s = PO.pack_base(w, dtype, scale_div="ieee")
    assert np.array_equal(q, GOLD[f"lw_{dtype}_q"])
    assert np.array_equal(s.view(np.uint16), GOLD[f"lw_{dtype}_s"])
    for sdt in ("f16", "f32"):
        s_in = GOLD[f"lws_{dtype}_{sdt}_s_in"]
        q, s = PO.pack_base(w, dtype, scales=s_in.view(np.float16) if sdt == "f16" else s_in,
                            scales_dtype=sdt, scale_div="ieee")
        assert np.array_equal(q, GOLD[f"lws_{dtype}_{sdt}_q"]), sdt
        assert np.array_equal(s.view(np.uint16), GOLD[f"lws_{dtype}_{sdt}_s"]), sdt


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_pack_base_fixture_rejects_fp32_math(dtype):
    # the same weights packed with W / s in FP32 (no rounding to the
    # weight's dtype before round()) give other nibbles
    w = PO.as_f32(gold_dense(f"lw_{dtype}_w", dtype), dtype)
    q, _ = PO.pack_base(w, "f32", scale_div="ieee")
    assert not np.array_equal(q, GOLD[f"lw_{dtype}_q"])


@pytest.mark.parametrize("dtype", PO.DTYPES)
def test_csr_oracle_equals_reference_pack_ortho_sparse(dtype):
    w = gold_dense(f"csr_{dtype}_w", dtype)
    rp, col, vals = PO.pack_csr(w, dtype)
    vb = np.uint16 if dtype != "f32" else np.uint32
    assert np.array_equal(rp, GOLD[f"csr_{dtype}_row_ptr"]) and np.array_equal(col, GOLD[f"csr_{dtype}_col"])
    assert np.array_equal(np.asarray(vals).view(vb), GOLD[f"csr_{dtype}_vals"].view(vb))


def test_bf16_rounding_is_nearest_even():
    # 1 + 2^-8 is halfway between bf16 1.0 and 1 + 2^-7: ties to the even 1.0;
    # 1 + 3 * 2^-8 ties up to 1 + 2^-6 (even mantissa)
    v = np.array([1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, -(1 + 2.0 ** -8), np.nan], np.float32)
    got = PO.bf16_bits_to_f32(PO.f32_to_bf16_bits(v))
    assert got[0] == 1.0 and got[1] == 1 + 2.0 ** -6 and got[2] == -1.0 and np.isnan(got[3])


@pytest.mark.parametrize("dtype", PO.DTYPES)
@pytest.mark.parametrize("group", [None, 128])
def test_planted_q_with_power_of_two_scales(dtype, group):
    # every cell holds a 7 * 2^e, so the scale is exactly 2^e (7 * fp32(1/7)
    # rounds to 1) in both division modes, and W / s recovers the planted q
    rng = np.random.default_rng(5)
    N, K = 6, 512
    G = group or K
    q = rng.integers(-7, 8, size=(N, K)).astype(np.int8)
    q.reshape(N, K // G, G)[:, :, 0] = 7
    e = rng.integers(-12, 4, size=(N, K // G))
    s = np.ldexp(1.0, e).astype(np.float32)
    w32 = (q.reshape(N, K // G, G) * s[:, :, None]).reshape(N, K).astype(np.float32)
    w = w32.astype(np.float16) if dtype == "f16" else (PO.f32_to_bf16_bits(w32) if dtype == "bf16" else w32)
    assert np.array_equal(PO.as_f32(w, dtype), w32)  # exact in every dtype
    for mode in ("reciprocal", "ieee"):
        packed, s16 = PO.pack_base(w, dtype, group, scale_div=mode)
        assert np.array_equal(unpack(packed), q)
        assert np.array_equal(s16.reshape(N, -1).astype(np.float32), s)


def test_round_half_to_even_and_clamp():
    # s = 1 (a 7 in the row); halves round to even; given scales clamp
    w = np.array([[7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 6.5]], np.float32)
    packed, s16 = PO.pack_base(w, "f32")
    assert s16[0] == 1.0
    assert unpack(packed).tolist() == [[7, 0, 2, 2, 0, -2, -2, 6]]
    w2 = np.array([[-9.3, 7.6, 100.0, -0.0]], np.float32)
    packed, s16 = PO.pack_base(w2, "f32", scales=np.array([1.0], np.float32), scales_dtype="f32")
    assert unpack(packed).tolist() == [[-8, 7, 7, 0]]
    # an all-zero row takes the 1e-6 floor (in FP32, then its FP16 copy)
    packed, s16 = PO.pack_base(np.zeros((1, 4), np.float32), "f32")
    assert s16[0] == np.float16(np.float32(1e-6)) and not unpack(packed).any()


def test_the_two_scale_divisions_differ():
    # max|W| values where m * fp32(1/7) and m / 7 round to different FP32
    # numbers: the division mode is observable, and the GPU test pins which
    # one torch uses on a GPU tensor
    m = np.float32(np.arange(1, 4000, dtype=np.float32) * np.float32(0.37))
    rec = m * (np.float32(1) / np.float32(7))
    ieee = m / np.float32(7)
    assert (rec != ieee).any()


@pytest.mark.parametrize("dtype", PO.DTYPES)
@pytest.mark.parametrize("group", [None, 128])
@pytest.mark.parametrize("given", [None, "f16", "f32"])
def test_product_cpu_packer_equals_oracle(dtype, group, given):
    rng = np.random.default_rng(11)
    N, K = 33, 512
    w = random_dense(rng, N, K, dtype, scale=0.05)
    G = group or K
    scales = None
    st = None
    if given:
        s = np.abs(rng.standard_normal((N, K // G))).astype(np.float32) * 0.02 + 1e-3
        scales = s.astype(np.float16) if given == "f16" else s
        st = torch.from_numpy(scales.reshape(N) if G == K else scales)
    q_t, s_t = pack_base_torch(to_torch(w, dtype), group, st)
    q_o, s_o = PO.pack_base(w, dtype, group, scales, given, scale_div="ieee")
    assert np.array_equal(q_t.numpy(), q_o)
    assert np.array_equal(s_t.numpy().view(np.uint16), s_o.view(np.uint16))


@pytest.mark.parametrize("dtype", PO.DTYPES)
def test_csr_oracle_equals_scipy_and_the_product_cpu_packer(dtype):
    rng = np.random.default_rng(12)
    N, K = 40, 300
    w32 = rng.standard_normal((N, K)).astype(np.float32)
    w32[rng.random((N, K)) > 0.03] = 0.0
    w32[3, 5] = -0.0          # dropped: -0 == 0
    w32[7] = 0.0              # an empty row
    w32[9, :] = 1.0           # a full row
    w = w32.astype(np.float16) if dtype == "f16" else (PO.f32_to_bf16_bits(w32) if dtype == "bf16" else w32)
    rp, col, vals = PO.pack_csr(w, dtype)
    rp_t, col_t, vals_t = pack_ortho_sparse_torch(to_torch(w, dtype), "csr")
    assert np.array_equal(rp, rp_t.numpy()) and np.array_equal(col, col_t.numpy())
    assert np.array_equal(np.asarray(vals).view(np.uint16 if dtype != "f32" else np.uint32),
                          from_torch(vals_t, dtype).view(np.uint16 if dtype != "f32" else np.uint32))
    ref = sp.csr_matrix(PO.as_f32(w, dtype))
    assert np.array_equal(rp, ref.indptr) and np.array_equal(col, ref.indices)
    assert np.array_equal(PO.as_f32(vals, dtype), ref.data)


def test_csr_keeps_nan_and_subnormals_and_drops_negative_zero():
    # the subnormal is set through its bits: a library loaded with
    # flush-to-zero host flags would flush a converted 1e-45 to 0
    w = np.array([[0.0, -0.0, np.nan, 0.0], [0.0, 0.0, 0.0, 0.0]], np.float32)
    w.view(np.uint32)[0, 3] = 1
    rp, col, vals = PO.pack_csr(w, "f32")
    assert rp.tolist() == [0, 2, 2] and col.tolist() == [2, 3]
    assert np.isnan(vals[0]) and vals.view(np.uint32)[1] == 1
