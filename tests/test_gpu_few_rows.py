"""Weight matrices of 1, 3 and 15 output rows (less than one 16-row block, so
every kernel's first row block is also its last and mostly empty), through
every kernel family and weight type of fh3_hip_matmul_dev, with bias, against
the CPU oracle (fh3's fh3_matmul, src/core/fh3_ops.c:317-404).

Bars: the rel-Frobenius gate of the other product tests (2e-3), the same bits
on a second call, and nothing stored past y: y is followed by 4 KiB of a
sentinel pattern that must be unchanged (a store of an empty row would land
there first).
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3
GUARD = 1024  # floats after y

# name, tokens, in, forced path (None: the automatic choice)
CASES = [
    ("Q4_K", 2, 2048, "GEMV8"),
    ("Q4_K", 6, 2048, "SWEEP"),
    ("Q4_K", 40, 5120, None),      # k_sweep token blocks
    ("Q4_K", 8, 1024, "SKINNY"),
    ("Q4_K", 24, 8192, "MIDM"),
    ("Q4_K", 70, 1024, None),      # k_gemm, K split
    ("Q4_K", 300, 512, None),      # k_gemm on 128-token tiles
    ("Q5_K", 4, 2048, None),       # k_skinny<Q5_K>
    ("Q5_K", 70, 1024, None),      # k_gemm<Q5_K>
    ("Q6_K", 4, 2048, None),       # k_sweep<Q6_K>
    ("Q6_K", 4, 2048, "SKINNY"),   # k_skinny<Q6_K>
    ("Q6_K", 70, 1024, None),      # k_gemm<Q6_K>
    ("F16", 5, 96, None),          # general rows, k_skinny16
    ("F16", 70, 512, None),        # fp16 rows, k_gemm16
    ("Q8_0", 3, 64, None),
]


def _weights(rng, name, N, K):
    if name == "Q4_K":
        return H.random_q4k(rng, N, K)
    return H.random_blocks(rng, name, N, K, scale_lo=-12, scale_hi=-8)


def _run(F, dw, dx, db, K, N, M, qtype):
    dy = F.DeviceBuffer((M * N + GUARD) * 4)
    dy.fill(0x5A)
    F.matmul_dev(dw, K, N, dx, dy, M, db, qtype=qtype)
    F.synchronize()
    out = dy.download(np.float32, (M * N + GUARD,))
    dy.close()
    assert (out[M * N:].view(np.uint8) == 0x5A).all(), "a store landed past y"
    return out[:M * N].reshape(M, N)


@pytest.mark.parametrize("N", [1, 3, 15])
@pytest.mark.parametrize("name,M,K,path", CASES)
def test_few_output_rows(gpu, oracle, name, M, K, path, N):
    F = gpu
    qtype = H.QTYPES[name][0]
    rng = np.random.default_rng(qtype * 101 + M * 7 + K + N)
    raw = _weights(rng, name, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    if path is not None:
        F.set_path(getattr(F, "PATH_" + path))
    try:
        print("few rows %s M=%d K=%d N=%d forced=%s path=%d" % (name, M, K, N, path, F.matmul_path(M, K)),
              flush=True)
        dw, dx, db = (F.DeviceBuffer.from_array(a) for a in (raw, x, bias))
        y = _run(F, dw, dx, db, K, N, M, qtype)
        y2 = _run(F, dw, dx, db, K, N, M, qtype)
        for b in (dw, dx, db):
            b.close()
    finally:
        F.set_path(F.PATH_AUTO)
    assert np.isfinite(y).all()
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    yo = H.matmul_with(oracle, "fh3_oracle_matmul", raw, K, N, x, bias, qtype=qtype)
    err = H.rel_fro(y, yo)
    print("  rel_fro = %.3e" % err, flush=True)
    assert err <= TOL
