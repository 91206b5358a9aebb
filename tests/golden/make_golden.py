"""Writes tests/golden/ref_coo_cases.npz from the reference's own compiled
CPU forward (oracle/_ref/libortho_ref.so, built by ``make -C oracle ref``
from /root/reference/src/ortho.c with the reference's flags).

Run in the build container (the only place the reference exists):

    make -C oracle ref && python tests/golden/make_golden.py

Cases:
  testcpu_a1 / testcpu_a0 / testcpu_empty
      The inputs of the reference's own test, /root/reference/tests/
      test_cpu_forward.c:97-145 (64x64, batch 4, 5% COO, srand(42) glibc
      rand() stream, consumed in the same order), at alpha = 1, alpha = 0
      and with the ortho count set to 0 (:172-319).
  rand_<N>x<K>_m<M>
      Seeded numpy inputs at non-square shapes (catches a transposed
      operand), per-row FP32 scales, COO uint16 indices with duplicates.

Each case stores q (uint8 [N, K/2]), scales (float32 [N]), idx (uint16),
vals (float32), x (float32 [M, K]), alpha and y (float32 [M, N]) as the
reference computed it.  The data are vectors, not reference source.
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle  # noqa: E402


def pack_int4_rowmajor(w: np.ndarray) -> np.ndarray:
    """int values in [-8, 7], shape [N, K] -> uint8 [N, K/2] (low = even)."""
    u = (w.astype(np.int16) & 0xF).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def testcpu_inputs():
    """The srand(42) stream of tests/test_cpu_forward.c:104-141."""
    libc = ctypes.CDLL("libc.so.6")
    libc.rand.restype = ctypes.c_int
    libc.srand(42)
    RAND_MAX = np.float32(2147483647)  # (float)RAND_MAX as C converts it
    DIM, B = 64, 4
    x = np.empty(B * DIM, np.float32)
    for i in range(B * DIM):
        x[i] = np.float32(libc.rand()) / RAND_MAX * np.float32(2.0) - np.float32(1.0)
    w = np.empty(DIM * DIM, np.int8)
    for i in range(DIM * DIM):
        w[i] = libc.rand() % 16 - 8
    s = np.empty(DIM, np.float32)
    for i in range(DIM):
        s[i] = np.float32(0.1) + np.float32(libc.rand()) / RAND_MAX * np.float32(0.9)
    count = DIM * DIM // 20
    idx = np.empty(count, np.uint16)
    vals = np.empty(count, np.float32)
    for i in range(count):
        idx[i] = libc.rand() % (DIM * DIM)
        vals[i] = np.float32(libc.rand()) / RAND_MAX * np.float32(0.1) - np.float32(0.05)
    return pack_int4_rowmajor(w.reshape(DIM, DIM)), s, idx, vals, x.reshape(B, DIM)


def main():
    if not oracle.ref_lib_available():
        if not oracle.build_ref():
            raise SystemExit("oracle/_ref/libortho_ref.so is not built and cannot be")
    cases = {}
    q, s, idx, vals, x = testcpu_inputs()
    for name, alpha, cnt in (("testcpu_a1", 1.0, None), ("testcpu_a0", 0.0, None),
                             ("testcpu_empty", 1.0, 0)):
        i2 = idx if cnt is None else idx[:0]
        v2 = vals if cnt is None else vals[:0]
        y = oracle.ref_forward_coo(q, s, i2, v2, x, alpha)
        cases[name] = dict(q=q, scales=s, idx=i2, vals=v2, x=x, alpha=np.float32(alpha), y=y)

    rng = np.random.Generator(np.random.PCG64(20251201))
    for (N, K, M, dens) in ((96, 128, 3, 0.03), (40, 200, 5, 0.10), (256, 256, 1, 0.01)):
        w = rng.integers(-8, 8, size=(N, K))
        q2 = pack_int4_rowmajor(w)
        s2 = np.abs(rng.normal(0, 0.02, size=N)).astype(np.float32)
        cnt = max(1, int(dens * N * K))
        i2 = rng.integers(0, N * K, size=cnt).astype(np.uint16)  # duplicates allowed
        v2 = rng.normal(0, 0.05, size=cnt).astype(np.float32)
        x2 = rng.normal(0, 1, size=(M, K)).astype(np.float32)
        y2 = oracle.ref_forward_coo(q2, s2, i2, v2, x2, 1.0)
        cases[f"rand_{N}x{K}_m{M}"] = dict(q=q2, scales=s2, idx=i2, vals=v2, x=x2,
                                          alpha=np.float32(1.0), y=y2)

    flat = {}
    for name, d in cases.items():
        for k, v in d.items():
            flat[f"{name}__{k}"] = v
    out = os.path.join(HERE, "ref_coo_cases.npz")
    np.savez_compressed(out, **flat)
    print("wrote", out, "cases:", ", ".join(cases))


if __name__ == "__main__":
    main()
