"""Writes tests/golden/sieve_cases.npz and tests/golden/pack_cases.npz: the
outputs of the reference's own Python (run on CPU tensors, in the build
container, the only place the reference exists) on seeded inputs, so that
the numpy oracles can be pinned on what closed forms leave open (FP16/BF16
intermediate rounding, tie rounding, the threshold's dtype, the k-th
largest score among ties).

    python tests/golden/make_sieve_golden.py

Functions run (each loaded from its file under /root/reference, nothing
copied):
  tools/sieve.py            quantize_int4 (:13-23), hessian_sieve (:25-76),
                            compute_hessian_diag_approx (:79-95),
                            pack_ortho_sparse(..., "csr") (:98-152)
  torch_bind/ortho_linear.py OrthoLinear.load_from_weights (:79-128)

Only data is written: inputs and the reference's outputs, FP16 / BF16
values as their 16-bit patterns, FP32 as float32.
"""
import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"

# the reference's own modules must resolve to the reference, not to this
# repository's re-exports of the same names (tools, torch_bind, libortho)
sys.path = [p for p in sys.path if os.path.abspath(p or ".") not in (REPO, HERE)]
sys.path.insert(0, REF)

import torch  # noqa: E402

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def to_np(t: torch.Tensor) -> np.ndarray:
    """Raw storage: uint16 patterns for FP16/BF16, float32 / ints as they are."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def from_f32(a: np.ndarray, dt: str) -> torch.Tensor:
    """FP32 values -> a tensor of dtype dt (round to nearest even)."""
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DT[dt])


def sieve_weights(rng, N, K, scale=0.05):
    w = (rng.standard_normal((N, K)) * scale).astype(np.float32)
    w[3] = 0.0                                  # the 1e-8 floor
    w[5, 7] = np.inf                            # NaN scale: the row becomes 0
    w[6, :] = np.float32(1e-9)                  # below the floor in FP32/BF16, 0 in FP16
    w[8, 11] = np.nan
    w[9, ::5] = -w[9, ::5]
    # exact halves of the step: max 7 * 2^-5, values (j + 1/2) * 2^-5
    w[10, :] = ((np.arange(K) % 15) - 7 + 0.5) * 2.0 ** -5
    w[10, 0] = 7 * 2.0 ** -5
    # a step that is not a power of two: w / s lands near halves after rounding
    w[11, :] = np.linspace(-0.3, 0.3, K, dtype=np.float32)
    w[12, :] = (np.arange(K) % 29 - 14).astype(np.float32) * 0.013
    return w


def make_sieve(ref_sieve, cases):
    rng = np.random.default_rng(20261202)
    N, K = 16, 96
    for dt in ("f32", "f16", "bf16"):
        w = from_f32(sieve_weights(rng, N, K), dt)
        wb = ref_sieve.quantize_int4(w)
        cases[f"quant_{dt}_w"] = to_np(w)
        cases[f"quant_{dt}_out"] = to_np(wb)

    # hessian_sieve: dtype pairs, both threshold branches, vector and matrix H
    combos = [("f32", "f32"), ("f16", "f32"), ("bf16", "f32"), ("f16", "f16"), ("bf16", "bf16"),
              ("f32", "f16")]
    targets = [("none", None), ("t02", 0.02), ("t0", 0.0), ("t1e4", 1e-4), ("t50", 0.5)]
    for i, (dt, hdt) in enumerate(combos):
        w = from_f32(sieve_weights(rng, N, K), dt)
        h = from_f32((rng.random(K) * 2 + 0.05).astype(np.float32), hdt)
        cases[f"hs_{dt}_{hdt}_w"] = to_np(w)
        cases[f"hs_{dt}_{hdt}_h"] = to_np(h)
        for tname, tgt in targets:
            # 2e-6 sits between FP16 neighbours: the host threshold's rounding
            # to the score's dtype decides entries near it
            wb, wo = ref_sieve.hessian_sieve(w, h, curvature_thresh=2e-6, sparsity_target=tgt)
            cases[f"hs_{dt}_{hdt}_{tname}_wb"] = to_np(wb)
            cases[f"hs_{dt}_{hdt}_{tname}_wo"] = to_np(wo)
        # a threshold inside the score distribution (scores ~1e-5..1e-4)
        wb, wo = ref_sieve.hessian_sieve(w, h, curvature_thresh=2.1e-5)
        cases[f"hs_{dt}_{hdt}_mid_wb"] = to_np(wb)
        cases[f"hs_{dt}_{hdt}_mid_wo"] = to_np(wo)
        # a threshold just below a score value v that rounds to v in the
        # score's dtype: entries scoring v are kept only if the threshold
        # stays in FP32 (the score itself is formed here only to pick v)
        sdt = torch.promote_types(w.dtype, h.dtype)
        res = w - ref_sieve.quantize_int4(w)
        score = ((res ** 2) / (h + 1e-6)).to(sdt).float().flatten()
        v = float(score[torch.isfinite(score) & (score > 0)].median())
        t = v * (1.0 - 2.0 ** -12)
        cases[f"hs_{dt}_{hdt}_edge_t"] = np.array([t], np.float64)
        wb, wo = ref_sieve.hessian_sieve(w, h, curvature_thresh=t)
        cases[f"hs_{dt}_{hdt}_edge_wb"] = to_np(wb)
        cases[f"hs_{dt}_{hdt}_edge_wo"] = to_np(wo)

    # a matrix H_inv (its diagonal is used) and thousands of tied scores
    q = rng.integers(-7, 8, size=(32, 128)).astype(np.float32)
    q[:, 0] = 7.0
    w = q * 2.0 ** -5
    w[:, 1::7] += 2.0 ** -7
    H = (rng.random((128, 128)) + np.eye(128)).astype(np.float32)
    cases["hsm_w"] = w.astype(np.float32)
    cases["hsm_H"] = H
    for tname, tgt in (("t01", 0.01), ("t10", 0.1), ("t50", 0.5)):
        wb, wo = ref_sieve.hessian_sieve(torch.from_numpy(w), torch.from_numpy(H), sparsity_target=tgt)
        cases[f"hsm_{tname}_wb"] = to_np(wb)
        cases[f"hsm_{tname}_wo"] = to_np(wo)

    # compute_hessian_diag_approx (torch's full X^T X on the CPU)
    for dt, (n, k) in (("f32", (300, 40)), ("f16", (300, 40)), ("bf16", (300, 40)), ("f32", (7, 129))):
        x = from_f32(rng.standard_normal((n, k)).astype(np.float32), dt)
        d = ref_sieve.compute_hessian_diag_approx(x)
        cases[f"hd_{dt}_{n}x{k}_x"] = to_np(x)
        cases[f"hd_{dt}_{n}x{k}_out"] = to_np(d)


def pack_weights(rng, N, K):
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[0] = 0.0                                   # all-zero row: the 1e-6 floor
    # exact half steps with a power-of-two scale: max 7 * 2^-6
    w[1] = ((np.arange(K) % 15) - 7 + 0.5) * 2.0 ** -6
    w[1, 0] = 7 * 2.0 ** -6
    # a scale that is not a power of two, values near half steps
    w[2] = (np.arange(K) % 17 - 8).astype(np.float32) * 0.0031 + 0.00155
    w[3] = np.linspace(-0.05, 0.05, K, dtype=np.float32)
    w[4, ::3] = -w[4, ::3] * 8.0
    return w


def make_pack(ref_ol, ref_sieve, cases):
    rng = np.random.default_rng(7070)
    N, K = 64, 64
    for dt in ("f32", "f16", "bf16"):
        w = from_f32(pack_weights(rng, N, K), dt)
        ortho = torch.zeros(N, K, dtype=DT[dt])
        layer = ref_ol.OrthoLinear(K, N)
        layer.load_from_weights(w, ortho)
        cases[f"lw_{dt}_w"] = to_np(w)
        cases[f"lw_{dt}_q"] = to_np(layer.base_weight)
        cases[f"lw_{dt}_s"] = to_np(layer.base_scales)
        # given scales (FP16 and FP32): only the division, round and clamp
        for sdt in ("f16", "f32"):
            s = from_f32((np.abs(rng.standard_normal(N)) * 0.004 + 1e-3).astype(np.float32), sdt)
            layer = ref_ol.OrthoLinear(K, N)
            layer.load_from_weights(w, ortho, base_scales=s)
            cases[f"lws_{dt}_{sdt}_s_in"] = to_np(s)
            cases[f"lws_{dt}_{sdt}_q"] = to_np(layer.base_weight)
            cases[f"lws_{dt}_{sdt}_s"] = to_np(layer.base_scales)

    # CSR of a dense ortho with exact zeros, -0, NaN and subnormals
    for dt in ("f32", "f16", "bf16"):
        d = rng.standard_normal((10, 48)).astype(np.float32)
        d[rng.random((10, 48)) < 0.8] = 0.0
        d[2, 5] = -0.0
        d[3, 7] = np.nan
        d[4, 9] = 1e-41 if dt == "f32" else 1e-7
        d[6] = 0.0
        t = from_f32(d, dt)
        rp, col, vals = ref_sieve.pack_ortho_sparse(t, format="csr")
        cases[f"csr_{dt}_w"] = to_np(t)
        cases[f"csr_{dt}_row_ptr"] = to_np(rp.to(torch.int32))
        cases[f"csr_{dt}_col"] = to_np(col.to(torch.int32))
        cases[f"csr_{dt}_vals"] = to_np(vals)


def main():
    ref_sieve = load("ref_tools_sieve", os.path.join(REF, "tools", "sieve.py"))
    ref_ol = load("ref_ortho_linear", os.path.join(REF, "torch_bind", "ortho_linear.py"))
    sieve_cases, pack_cases = {}, {}
    make_sieve(ref_sieve, sieve_cases)
    make_pack(ref_ol, ref_sieve, pack_cases)
    np.savez_compressed(os.path.join(HERE, "sieve_cases.npz"), **sieve_cases)
    np.savez_compressed(os.path.join(HERE, "pack_cases.npz"), **pack_cases)
    print(f"wrote {len(sieve_cases)} sieve arrays and {len(pack_cases)} pack arrays")


if __name__ == "__main__":
    main()
