"""Packing on the GPU (orth_pack.hip) against the CPU oracle
(oracle/pack_oracle.py, GPU division semantics) and against the
reference's own torch ops run on the same GPU tensors: bit for bit."""
import numpy as np
import pytest
import torch

from libortho_amd import OrthoLinear, _C_ops
from libortho_amd.tools.sieve import pack_ortho_sparse, pack_ortho_sparse_torch
from libortho_amd.torch_bind.ortho_linear import pack_base_torch
from oracle import pack_oracle as PO

pytestmark = pytest.mark.gpu


def to_torch(w: np.ndarray, dtype: str) -> torch.Tensor:
    if dtype == "bf16":
        return torch.from_numpy(w.astype(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(w)


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.cpu()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float32:
        return t.numpy().view(np.uint32)
    return t.numpy()


def random_dense(seed, N, K, dtype, scale=0.05):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * scale).astype(np.float32)
    w[1, :] = 0.0  # a row of zeros: the 1e-6 floor
    if dtype == "f16":
        return w.astype(np.float16)
    if dtype == "bf16":
        return PO.f32_to_bf16_bits(w)
    return w


BASE_CASES = [
    # N, K, group, weight dtype, given-scale dtype, kernel
    (64, 4096, 128, "f32", None, 1), (64, 4096, 128, "f16", None, 1), (64, 4096, 128, "bf16", None, 1),
    (40, 4096, 256, "f32", None, 1), (40, 4096, 2048, "f16", None, 1), (48, 1024, None, "f32", None, 1),
    (48, 4096, None, "f32", None, 2), (48, 11008, None, "f32", None, 2), (48, 11008, None, "f16", None, 2),
    (48, 11008, None, "bf16", None, 2), (20, 14336, None, "f32", None, 2),
    (20, 4096, 128, "f32", "f16", 1), (20, 4096, 128, "f16", "f32", 1), (20, 4096, None, "f32", "f32", 2),
    (20, 4096, None, "bf16", "f16", 2),
    (30, 512, 64, "f32", None, 3), (30, 200, 40, "f16", None, 3), (12, 40000, None, "f32", None, 3),
]


@pytest.mark.parametrize("N,K,group,dtype,given,path", BASE_CASES)
def test_pack_base_matches_oracle_and_torch_ops(N, K, group, dtype, given, path):
    print(f"pack_base N={N} K={K} G={group} {dtype} given={given}", flush=True)
    w = random_dense(1000 + K + N, N, K, dtype)
    G = group or K
    scales = None
    st = None
    if given:
        rng = np.random.default_rng(7 + N)
        s = np.abs(rng.standard_normal((N, K // G))).astype(np.float32) * 0.02 + 1e-3
        scales = s.astype(np.float16) if given == "f16" else s
        st = torch.from_numpy(scales.reshape(N) if G == K else scales).cuda()
    wt = to_torch(w, dtype).cuda()
    q, s16 = _C_ops.pack_base(wt, group, st)
    assert _C_ops.pack_base_path(wt, group, q) == path
    q_o, s_o = PO.pack_base(w, dtype, group, scales, given, scale_div="reciprocal")
    assert np.array_equal(bits(q), q_o)
    assert np.array_equal(bits(s16), s_o.view(np.uint16))
    # the reference's torch ops on the same GPU tensors
    q_t, s_t = pack_base_torch(wt, group, st)
    assert np.array_equal(bits(q), bits(q_t))
    assert np.array_equal(bits(s16), bits(s_t))


@pytest.mark.parametrize("group", [128, None])
def test_pack_base_full_c2_layer(group):
    # 4096 -> 11008 FP32 weights: bit-exact against the oracle, and the
    # dequantised weights within half a step of W
    print(f"pack_base c2 G={group}", flush=True)
    N, K = 11008, 4096
    w = random_dense(77, N, K, "f32")
    wt = torch.from_numpy(w).cuda()
    q, s16 = _C_ops.pack_base(wt, group, None)
    q_o, s_o = PO.pack_base(w, "f32", group, scale_div="reciprocal")
    assert np.array_equal(bits(q), q_o) and np.array_equal(bits(s16), s_o.view(np.uint16))
    deq = _C_ops.dequant(q, s16, K).cpu().numpy()
    G = group or K
    step = np.repeat(s_o.reshape(N, -1).astype(np.float32), G, axis=1)
    assert (np.abs(deq - w) <= 0.5 * step * 1.01 + 1e-6).all()


CSR_CASES = [
    # N, K, dtype, density, layout
    (64, 4096, "f32", 0.01, "aligned"), (64, 4096, "f16", 0.05, "aligned"), (64, 4096, "bf16", 0.05, "aligned"),
    (50, 301, "f32", 0.1, "aligned"), (50, 300, "f16", 0.1, "offset"), (50, 4096, "f32", 0.02, "offset"),
    (70, 1000, "f32", 0.0, "aligned"), (9, 64, "f32", 1.0, "aligned"),
    (40000, 64, "f16", 0.05, "aligned"),  # more rows than one scan pass (16,384): the carry
]


@pytest.mark.parametrize("N,K,dtype,density,layout", CSR_CASES)
def test_pack_csr_matches_oracle_and_torch_ops(N, K, dtype, density, layout):
    print(f"pack_csr N={N} K={K} {dtype} density={density} {layout}", flush=True)
    rng = np.random.default_rng(N * 7 + K)
    w32 = rng.standard_normal((N, K)).astype(np.float32)
    w32[rng.random((N, K)) >= density] = 0.0
    if N > 8 and K > 8:
        w32[2, :] = 0.0                # an empty row
        w32[3, 1] = -0.0               # dropped
        w32[4, 3] = np.nan             # kept
        w32.view(np.uint32)[5, 7] = 0x11111  # an FP32 subnormal, set through its bits (kept)
    w = w32.astype(np.float16) if dtype == "f16" else (PO.f32_to_bf16_bits(w32) if dtype == "bf16" else w32)
    wt = to_torch(w, dtype).cuda()
    if layout == "offset":  # a row-major view one element into its buffer
        buf = torch.empty(N * K + 1, dtype=wt.dtype, device="cuda")
        buf[1:] = wt.reshape(-1)
        wt = buf[1:].view(N, K)
    rp, col, vals = _C_ops.pack_csr(wt)
    rp_o, col_o, vals_o = PO.pack_csr(w, dtype)
    assert np.array_equal(bits(rp), rp_o) and np.array_equal(bits(col), col_o)
    vo = np.asarray(vals_o).view(np.uint32 if dtype == "f32" else np.uint16)
    assert np.array_equal(bits(vals), vo)
    rp_t, col_t, vals_t = pack_ortho_sparse_torch(wt, "csr")
    assert np.array_equal(bits(rp), bits(rp_t)) and np.array_equal(bits(col), bits(col_t))
    assert np.array_equal(bits(vals), bits(vals_t))
    # without the nonzero mask (the fill reads all of w): the same arrays
    rp2, col2, vals2 = _C_ops.pack_csr(wt, use_mask=False)
    assert torch.equal(rp2, rp) and torch.equal(col2, col) and np.array_equal(bits(vals2), bits(vals))
    # FP16 values straight from the kernel: rounded to nearest even
    _, _, v16 = _C_ops.pack_csr(wt, torch.float16)
    assert np.array_equal(bits(v16), PO.as_f32(vals_o, dtype).astype(np.float16).view(np.uint16))


def test_pack_csr_full_c2_density():
    print("pack_csr c2", flush=True)
    N, K, nnz = 11008, 4096, 450888
    rng = np.random.default_rng(88)
    flat = rng.choice(N * K, size=nnz, replace=False)
    w = np.zeros(N * K, np.float32)
    w[flat] = rng.standard_normal(nnz).astype(np.float32) + 3.0
    w = w.reshape(N, K)
    rp, col, vals = pack_ortho_sparse(torch.from_numpy(w).cuda(), "csr")
    rp_o, col_o, vals_o = PO.pack_csr(w, "f32")
    assert int(rp[-1]) == nnz
    assert np.array_equal(bits(rp), rp_o) and np.array_equal(bits(col), col_o)
    assert np.array_equal(bits(vals), vals_o.view(np.uint32))


def test_load_from_weights_on_the_gpu_uses_the_kernels():
    # OrthoLinear.load_from_weights with GPU tensors: the same buffers as the
    # reference's torch ops on those tensors
    N, K = 256, 1024
    rng = np.random.default_rng(99)
    wb = torch.from_numpy((rng.standard_normal((N, K)) * 0.02).astype(np.float32)).cuda()
    wo = torch.from_numpy(np.where(rng.random((N, K)) < 0.02, rng.standard_normal((N, K)), 0.0)
                          .astype(np.float32)).cuda()
    for group in (None, 128):
        layer = OrthoLinear(K, N, q_bits=4, group_size=group).cuda()
        layer.load_from_weights(wb, wo)
        q_t, s_t = pack_base_torch(wb, group, None)
        assert np.array_equal(bits(layer.base_weight), bits(q_t))
        assert np.array_equal(bits(layer.base_scales), bits(s_t))
        rp_t, col_t, vals_t = pack_ortho_sparse_torch(wo, "csr")
        assert np.array_equal(bits(layer.ortho_row_ptr), bits(rp_t))
        assert np.array_equal(bits(layer.ortho_col_indices), bits(col_t))
        assert np.array_equal(bits(layer.ortho_values), bits(vals_t.to(torch.float16)))


def test_reference_checkpoint_forward_on_the_gpu(tmp_path, oracle_mod):
    # a reference-layout checkpoint (per-row FP16 scales, CSR, FP32 bias)
    # loaded with load_checkpoint onto the GPU; the forward (bias added after,
    # as the reference) against the FP64 oracle, before and after the
    # per-row scales are expanded to groups of 128
    from libortho_amd import workloads as W
    from libortho_amd.torch_bind import load_checkpoint
    K, N = 1024, 320
    lay = W.make_layer(K, N, None, 0.02, 1234)
    bias = (torch.arange(N, dtype=torch.float32) * 0.001)
    sd = {"base_weight": torch.from_numpy(lay.q.copy()), "base_scales": torch.from_numpy(lay.scales.copy()),
          "ortho_values": torch.from_numpy(lay.vals.copy()),
          "ortho_col_indices": torch.from_numpy(lay.col.copy()),
          "ortho_row_ptr": torch.from_numpy(lay.row_ptr.copy()), "bias": bias}
    path = tmp_path / "ref.pt"
    torch.save(sd, path)
    m = OrthoLinear(K, N, bias=True)
    load_checkpoint(m, path, map_location="cuda")
    m = m.cuda()
    x_np = W.make_x(3, K, 99)
    ref = oracle_mod.forward_f64(lay.q, lay.scales, lay.row_ptr, lay.col, lay.vals, x_np, 1.0) + bias.numpy()
    for expand in (False, True):
        if expand:
            m.expand_scales(128)
        with torch.no_grad():  # (the bias is fused into the store)
            y = m(torch.from_numpy(x_np).cuda()).float().cpu().numpy()
        err = float(np.abs(y - ref).max())
        assert err <= 1e-2 * float(np.abs(ref).max()), f"expand={expand}: {err}"
