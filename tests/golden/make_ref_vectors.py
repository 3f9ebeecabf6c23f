"""Write tests/golden/ref_vectors.npz: outputs of the reference's own
src/core/fh3_quant.c + src/core/fh3_ops.c (compiled by oracle/Makefile into
oracle/_ref/libfh3_ref.so) on small seeded Q4_K problems.

Run from the repository root after `make -C oracle ref`:
    python tests/golden/make_ref_vectors.py
The fixture holds inputs and outputs only (no reference code).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import helpers as H  # noqa: E402

CASES = [  # (K, N, M, bias, d_kind)
    (256, 5, 1, False, "normal"),
    (256, 64, 3, True, "normal"),
    (512, 67, 7, True, "normal"),
    (1280, 130, 2, False, "normal"),
    (768, 33, 5, True, "special"),
]


def special_blocks(rng, n_rows, K):
    """Random bytes with d/dmin drawn from edge fp16 patterns: zero, -0,
    subnormals, the largest normal, negative values."""
    raw = H.random_q4k(rng, n_rows, K).reshape(-1, 144)
    pats = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0xBC00, 0x3C00, 0x1400, 0xB400],
                    dtype=np.uint16)
    pick_d = pats[rng.integers(0, len(pats), size=raw.shape[0])]
    pick_m = pats[rng.integers(0, len(pats), size=raw.shape[0])]
    raw[:, 0:2] = pick_d.view(np.uint8).reshape(-1, 2)
    raw[:, 2:4] = pick_m.view(np.uint8).reshape(-1, 2)
    return raw.reshape(-1)


def main():
    ref = H.load_ref()
    if ref is None:
        sys.exit("oracle/_ref/libfh3_ref.so missing: run `make -C oracle ref` first")
    rng = np.random.default_rng(20261201)
    out = {}
    for i, (K, N, M, use_bias, kind) in enumerate(CASES):
        raw = H.random_q4k(rng, N, K) if kind == "normal" else special_blocks(rng, N, K)
        x = rng.standard_normal((M, K)).astype(np.float32)
        bias = rng.standard_normal(N).astype(np.float32) if use_bias else None
        y = H.matmul_with(ref, "fh3_matmul", raw, K, N, x, bias)
        deq = H.oracle_dequant(ref, raw, N, K, fn="fh3_dequant")
        out["c%d_shape" % i] = np.array([K, N, M, int(use_bias)], dtype=np.int64)
        out["c%d_w" % i] = raw
        out["c%d_x" % i] = x
        out["c%d_bias" % i] = bias if bias is not None else np.zeros(0, np.float32)
        out["c%d_y" % i] = y
        out["c%d_deq" % i] = deq
    # seeded normals from the reference generator (src/model/fh3_sched.c:110-159)
    rn = np.empty(1001, dtype=np.float32)
    ref.fh3_rng_normal(7, 3, rn.ctypes.data, rn.size)
    out["rng_seed7_stream3"] = rn
    np.savez_compressed(os.path.join(HERE, "ref_vectors.npz"), **out)
    print("wrote", os.path.join(HERE, "ref_vectors.npz"))


if __name__ == "__main__":
    main()
