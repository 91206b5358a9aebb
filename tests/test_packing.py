"""Host logic on the CPU: the sparse packer, OrthoLinear's buffers and
weight packing, the operator boundary's argument checks, and the workload
generators."""
import numpy as np
import pytest
import torch

from libortho_amd import OrthoLinear, pack_ortho_sparse, _C_ops
from libortho_amd import workloads as W


def np_unpack(packed: np.ndarray) -> np.ndarray:
    lo = (packed & 0xF).astype(np.int16)
    hi = (packed >> 4).astype(np.int16)
    w = np.empty((packed.shape[0], packed.shape[1] * 2), np.int16)
    w[:, 0::2], w[:, 1::2] = lo, hi
    return np.where(w >= 8, w - 16, w)


# ------------------------------------------------------------ CSR packing

@pytest.mark.parametrize("shape,density", [((7, 10), 0.3), ((64, 128), 0.05), ((1, 9), 1.0),
                                           ((5, 6), 0.0)])
def test_pack_csr_invariants_and_torch_equivalence(shape, density):
    g = torch.Generator().manual_seed(0)
    w = torch.randn(shape, generator=g) * (torch.rand(shape, generator=g) < density)
    w[0, 0] = -0.0  # negative zero is a zero (dropped, as w != 0 is False)
    row_ptr, col, val = pack_ortho_sparse(w, "csr")
    N, K = shape
    assert row_ptr.dtype == torch.int32 and col.dtype == torch.int32 and val.dtype == w.dtype
    assert row_ptr.numel() == N + 1 and row_ptr[0] == 0 and row_ptr[-1] == col.numel()
    assert bool((row_ptr[1:] >= row_ptr[:-1]).all())
    for n in range(N):
        c = col[row_ptr[n]:row_ptr[n + 1]]
        assert bool((c[1:] > c[:-1]).all()) and bool(((c >= 0) & (c < K)).all())
    assert bool((val != 0).all())
    ref = w.to_sparse_csr()
    assert torch.equal(row_ptr.long(), ref.crow_indices())
    assert torch.equal(col.long(), ref.col_indices())
    assert torch.equal(val, ref.values())


def test_pack_coo_and_bad_format():
    w = torch.zeros(4, 6)
    w[0, 3], w[2, 1], w[2, 5] = 1, 2, -1
    idx, val, none = pack_ortho_sparse(w, "coo")
    assert none is None and idx.dtype == torch.uint16
    assert idx.to(torch.int32).tolist() == [3, 13, 17] and val.tolist() == [1, 2, -1]
    with pytest.raises(ValueError):
        pack_ortho_sparse(w, "ell")


# ------------------------------------------------------------- OrthoLinear

def test_buffers_match_reference_state_dict():
    m = OrthoLinear(64, 48, bias=True)
    sd = m.state_dict()
    assert list(sd) == ["bias", "base_weight", "base_scales", "ortho_values",
                        "ortho_col_indices", "ortho_row_ptr"] or set(sd) == {
        "bias", "base_weight", "base_scales", "ortho_values", "ortho_col_indices", "ortho_row_ptr"}
    assert sd["base_weight"].dtype == torch.uint8 and tuple(sd["base_weight"].shape) == (48, 32)
    assert sd["base_scales"].dtype == torch.float16 and tuple(sd["base_scales"].shape) == (48,)
    assert sd["ortho_values"].dtype == torch.float16 and sd["ortho_values"].numel() == 0
    assert sd["ortho_col_indices"].dtype == torch.int32
    assert sd["ortho_row_ptr"].dtype == torch.int32 and sd["ortho_row_ptr"].numel() == 0
    assert sd["bias"].dtype == torch.float32
    assert m.alpha == 1.0
    m.set_alpha(0.0)
    assert m.alpha == 0.0
    g = OrthoLinear(256, 8, group_size=128)
    assert tuple(g.base_scales.shape) == (8, 2)
    with pytest.raises(ValueError):
        OrthoLinear(63, 8)


@pytest.mark.parametrize("group", [None, 16])
def test_load_from_weights_packing_closed_form(group):
    g = torch.Generator().manual_seed(1)
    N, K = 24, 64
    Wb = torch.randn(N, K, generator=g)
    Wo = torch.randn(N, K, generator=g) * (torch.rand(N, K, generator=g) < 0.1)
    m = OrthoLinear(K, N, group_size=group)
    m.load_from_weights(Wb, Wo)
    G = K if group is None else group
    s = (Wb.reshape(N, K // G, G).abs().amax(dim=2) / 7.0).clamp(min=1e-6)
    q_expect = (Wb / s.repeat_interleave(G, dim=1)).round().clamp(-8, 7).numpy()
    q_got = np_unpack(m.base_weight.numpy())
    assert np.array_equal(q_got, q_expect)
    s_expect = s.to(torch.float16).reshape(m.base_scales.shape)
    assert torch.equal(m.base_scales, s_expect)
    rp, col, val = pack_ortho_sparse(Wo, "csr")
    assert torch.equal(m.ortho_row_ptr, rp) and torch.equal(m.ortho_col_indices, col)
    assert torch.equal(m.ortho_values, val.to(torch.float16))


def test_load_with_given_scales_uses_them_unrounded():
    N, K = 4, 8
    Wb = torch.arange(N * K, dtype=torch.float32).reshape(N, K) / 10 - 1.5
    s = torch.full((N,), 0.3)
    m = OrthoLinear(K, N)
    m.load_from_weights(Wb, torch.zeros(N, K), base_scales=s)
    q = np_unpack(m.base_weight.numpy())
    assert np.array_equal(q, (Wb / 0.3).round().clamp(-8, 7).numpy())
    assert m.ortho_values.numel() == 0 and m.ortho_row_ptr.tolist() == [0] * (N + 1)


def test_cpu_forward_raises_instead_of_garbage():
    m = OrthoLinear(16, 8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        m(torch.randn(2, 16, dtype=torch.float16))


def test_boundary_rejects_cpu_tensors_before_the_library():
    q = torch.zeros(8, 8, dtype=torch.uint8)
    s = torch.ones(8, dtype=torch.float16)
    e16 = torch.empty(0, dtype=torch.float16)
    e32 = torch.empty(0, dtype=torch.int32)
    x = torch.zeros(1, 16, dtype=torch.float16)
    y = torch.zeros(1, 8, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        _C_ops.forward(q, s, e16, e32, e32, x, y, 1.0)


def test_make_layer_checks_shapes_and_dtypes():
    dev = torch.device("cpu")
    q = torch.zeros(8, 8, dtype=torch.uint8)
    s = torch.ones(8, dtype=torch.float16)
    e16 = torch.empty(0, dtype=torch.float16)
    e32 = torch.empty(0, dtype=torch.int32)
    L = _C_ops.make_layer(q, s, e16, e32, e32, 16, 8, 1.0, dev)
    assert L.base.in_features == 16 and L.base.scale_groups == 1 and L.ortho.count == 0
    L = _C_ops.make_layer(q, torch.ones(8, 4, dtype=torch.float16), e16, e32, e32, 16, 8, 1.0, dev)
    assert L.base.scale_groups == 4
    bad = [
        (q.to(torch.int8), s, "uint8"),
        (torch.zeros(8, 4, dtype=torch.uint8), s, "shape"),
        (q, s.to(torch.bfloat16), "float16 or float32"),
        (q, torch.ones(8, 3, dtype=torch.float16), "does not divide"),
    ]
    for qq, ss, msg in bad:
        with pytest.raises(RuntimeError, match=msg):
            _C_ops.make_layer(qq, ss, e16, e32, e32, 16, 8, 1.0, dev)
    v = torch.ones(3, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="ortho_row_ptr"):
        _C_ops.make_layer(q, s, v, torch.zeros(3, dtype=torch.int32),
                          torch.zeros(5, dtype=torch.int32), 16, 8, 1.0, dev)
    with pytest.raises(RuntimeError, match="int32"):
        _C_ops.make_layer(q, s, v, torch.zeros(3, dtype=torch.int64),
                          torch.zeros(9, dtype=torch.int32), 16, 8, 1.0, dev)


# ---------------------------------------------------------- workloads

def test_uniform_layer_generator():
    L = W.make_layer(256, 96, 128, 0.01, seed=7)
    assert L.q.shape == (96, 128) and L.scales.shape == (96, 2) and L.scales.dtype == np.float16
    assert L.nnz == round(0.01 * 96 * 256)
    flat = np.repeat(np.arange(96), np.diff(L.row_ptr)) * 256 + L.col
    assert len(np.unique(flat)) == L.nnz and np.all(np.diff(flat) > 0)
    assert np.all(L.vals != 0)
    L2 = W.make_layer(256, 96, 128, 0.01, seed=7)
    assert np.array_equal(L.q, L2.q) and np.array_equal(L.col, L2.col)


def test_skewed_layer_generator():
    L = W.make_skewed_layer(512, 300, 128, 0.005, 0.02, seed=3)
    counts = np.diff(L.row_ptr)
    n_out = round(0.02 * 512)
    assert counts.sum() == round(0.005 * 300 * 512) and counts.max() <= n_out
    assert len(np.unique(L.col)) <= n_out
    for n in range(300):
        c = L.col[L.row_ptr[n]:L.row_ptr[n + 1]]
        assert np.all(np.diff(c) > 0)


def test_algorithmic_bytes_match_baseline_table():
    # the published per-config byte counts: c1 9.436 / 8.413 MB, c2 M=1..16, c3, c4, c5
    c1 = W.config_layer("c1")
    assert abs(W.algorithmic_bytes(c1, 1, 1.0) / 1e6 - 9.436) < 1e-3
    assert abs(W.algorithmic_bytes(c1, 1, 0.0) / 1e6 - 8.413) < 1e-3
    c2 = W.config_layer("c2")
    assert abs(W.algorithmic_bytes(c2, 1, 1.0) / 1e6 - 26.028) < 1e-3
    assert abs(W.algorithmic_flops(c2, 1, 1.0) / 1e9 - 0.091) < 1e-3
