"""Checkpoints: reference-layout state_dicts (per-row FP16 scales, CSR of
any length) load into OrthoLinear, round trips keep every buffer, the
per-row -> group scale conversion leaves every dequantised weight
unchanged, and malformed checkpoints are refused."""
import io

import numpy as np
import pytest
import torch

from libortho_amd import OrthoLinear
from libortho_amd import workloads as W
from libortho_amd.torch_bind import load_checkpoint
from oracle import oracle


def reference_state_dict(K, N, density, seed, bias=True):
    """The buffers a reference OrthoLinear holds after load_from_weights
    (/root/reference/torch_bind/ortho_linear.py:59-74,98-128): packed
    uint8 [N, K/2], FP16 per-row scales [N], the CSR (int32 / FP16) and an
    FP32 bias."""
    lay = W.make_layer(K, N, None, density, seed)
    sd = {
        "base_weight": torch.from_numpy(lay.q.copy()),
        "base_scales": torch.from_numpy(lay.scales.copy()),
        "ortho_values": torch.from_numpy(lay.vals.copy()),
        "ortho_col_indices": torch.from_numpy(lay.col.copy()),
        "ortho_row_ptr": torch.from_numpy(lay.row_ptr.copy()),
    }
    if bias:
        sd["bias"] = torch.arange(N, dtype=torch.float32) * 0.01
    return lay, sd


def save_load(sd):
    buf = io.BytesIO()
    torch.save(sd, buf)
    buf.seek(0)
    return torch.load(buf, weights_only=True)


@pytest.mark.parametrize("group", [None, 128])
def test_reference_checkpoint_loads_into_a_fresh_module(group):
    lay, sd = reference_state_dict(512, 96, 0.02, 3)
    m = OrthoLinear(512, 96, bias=True, group_size=group)  # the checkpoint's layout wins
    m.load_state_dict(save_load(sd))
    assert m.group_size is None and tuple(m.base_scales.shape) == (96,)
    for k, v in sd.items():
        got = getattr(m, k)
        assert got.dtype == v.dtype and torch.equal(got.detach(), v), k
    assert m.ortho_values.numel() == len(lay.vals)


def test_round_trip_of_a_grouped_module_through_a_file(tmp_path):
    rng = np.random.default_rng(4)
    wb = torch.from_numpy((rng.standard_normal((64, 256)) * 0.02).astype(np.float32))
    wo = torch.from_numpy(np.where(rng.random((64, 256)) < 0.05, rng.standard_normal((64, 256)), 0.0)
                          .astype(np.float32))
    a = OrthoLinear(256, 64, group_size=128)
    a.load_from_weights(wb, wo)
    path = tmp_path / "layer.pt"
    torch.save(a.state_dict(), path)
    b = OrthoLinear(256, 64)
    load_checkpoint(b, path)
    assert b.group_size == 128
    for k, v in a.state_dict().items():
        assert torch.equal(b.state_dict()[k], v), k


def test_expand_scales_keeps_every_dequantised_weight():
    lay, sd = reference_state_dict(512, 40, 0.01, 5, bias=False)
    m = OrthoLinear(512, 40)
    m.load_state_dict(sd)
    before = oracle.dequant_f32(m.base_weight.numpy(), m.base_scales.numpy())
    m.expand_scales(128)
    assert m.group_size == 128 and tuple(m.base_scales.shape) == (40, 4)
    after = oracle.dequant_f32(m.base_weight.numpy(), m.base_scales.numpy())
    assert np.array_equal(before.view(np.uint32), after.view(np.uint32))
    with pytest.raises(ValueError):
        m.expand_scales(128)  # already grouped


def test_malformed_checkpoints_are_refused():
    _, sd = reference_state_dict(256, 32, 0.05, 6, bias=False)
    bad = dict(sd, ortho_row_ptr=sd["ortho_row_ptr"][:-1])
    with pytest.raises(RuntimeError, match="row_ptr"):
        OrthoLinear(256, 32).load_state_dict(bad)
    bad = dict(sd, ortho_col_indices=sd["ortho_col_indices"][1:])
    with pytest.raises(RuntimeError, match="row_ptr"):
        OrthoLinear(256, 32).load_state_dict(bad)
    bad = dict(sd, base_weight=torch.zeros(32, 64, dtype=torch.uint8))
    with pytest.raises(RuntimeError, match="base_weight"):
        OrthoLinear(256, 32).load_state_dict(bad)
    bad = dict(sd, base_scales=torch.zeros(32, 3, dtype=torch.float16))  # 3 does not divide 256
    with pytest.raises(RuntimeError, match="base_scales"):
        OrthoLinear(256, 32).load_state_dict(bad)
    bad = {k: v for k, v in sd.items() if k != "ortho_values"}
    with pytest.raises(RuntimeError):
        OrthoLinear(256, 32).load_state_dict(bad)


def test_an_empty_csr_checkpoint_loads():
    _, sd = reference_state_dict(256, 32, 0.0, 7, bias=False)
    m = OrthoLinear(256, 32)
    m.load_state_dict(dict(sd, ortho_row_ptr=torch.tensor([], dtype=torch.int32)))
    assert m.ortho_values.numel() == 0 and m.ortho_row_ptr.numel() == 0


def test_a_refused_checkpoint_leaves_the_module_unchanged():
    """Every check runs before any buffer is replaced: a checkpoint whose
    group scales are valid but whose CSR is not leaves group_size, the
    scales and the CSR as they were."""
    lay, sd = reference_state_dict(256, 64, 0.02, seed=9)
    m = OrthoLinear(256, 64, bias=True)
    m.load_state_dict(sd)
    before = {k: v.clone() for k, v in m.state_dict().items()}
    bad = dict(sd)
    bad["base_scales"] = torch.ones(64, 2, dtype=torch.float16)      # valid group-128 layout
    bad["ortho_row_ptr"] = sd["ortho_row_ptr"].clone()
    bad["ortho_row_ptr"][-1] += 1                                    # does not end at nnz
    with pytest.raises(RuntimeError):
        m.load_state_dict(bad)
    assert m.group_size is None
    for k, v in m.state_dict().items():
        assert torch.equal(v, before[k]), k


def test_copies_carry_the_weights_not_the_derived_caches():
    """A module that has run a forward holds a C descriptor (raw pointers),
    an ortho plan and its build event: ``copy.deepcopy`` and pickling drop
    them (the copy rebuilds its own on its first forward) and keep every
    parameter and buffer."""
    import copy
    import pickle

    from libortho_amd import _lib
    m = OrthoLinear(256, 64, bias=True, group_size=128)
    with torch.no_grad():
        m.bias.copy_(torch.arange(64, dtype=torch.float32))
    m._desc, m._desc_key = _lib.OrthHipLayer(), ("key",)
    m._plan, m._plan_key = torch.zeros(8, dtype=torch.uint8), ("key",)
    m._plan_streams = {0}
    for c in (copy.deepcopy(m), pickle.loads(pickle.dumps(m))):
        assert c._plan is None and c._plan_key is None
        assert not hasattr(c, "_desc") and not hasattr(c, "_plan_streams")
        for (k, a), (k2, b) in zip(m.state_dict().items(), c.state_dict().items()):
            assert k == k2 and torch.equal(a, b)
    assert m._desc_key == ("key",)  # the original keeps its caches
