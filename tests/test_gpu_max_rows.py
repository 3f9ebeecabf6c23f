"""The longest rows the native kernels take (in = 32768 values, 128
super-blocks; longer rows go through zero-padded fp16 rows, covered by
tests/test_gpu_general_rows.py), through every kernel family of
fh3_hip_matmul_dev, against the CPU oracle (fh3's fh3_matmul,
src/core/fh3_ops.c:317-404).

At this length the sweep runs the most K slices it makes (7 for one token
block, 13 for two, 16 for three or four; 13 for Q6_K), k_skinny's Q5_K / Q6_K
windows and the GEMM's K split are at their widest, and the activation
preparation holds 32 values per thread.  Bars: the rel-Frobenius gate of the
other product tests (2e-3), every output finite, the same bits on a second
call.
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3
K = 32768

# name, tokens, out, forced path (None: the automatic choice), expected kernel path
CASES = [
    ("Q4_K", 1, 96, None, "SWEEP"),       # one token block, 7 slices
    ("Q4_K", 4, 64, None, "SWEEP"),
    ("Q4_K", 16, 130, None, "SWEEP"),
    ("Q4_K", 24, 64, None, "SWEEP"),      # two token blocks, 13 slices
    ("Q4_K", 64, 48, None, "SWEEP"),      # four token blocks, 16 slices
    ("Q4_K", 8, 80, "SKINNY", "SKINNY"),
    ("Q4_K", 40, 64, "MIDM", "MIDM"),
    ("Q4_K", 2, 64, "GEMV8", None),       # past the int8 kernel's window: the choice falls back
    ("Q4_K", 65, 64, None, "GEMM"),       # K split
    ("Q4_K", 300, 40, None, "GEMM"),
    ("Q5_K", 4, 64, None, None),          # k_skinny<Q5_K> in K windows
    ("Q5_K", 100, 40, None, None),        # k_gemm<Q5_K>
    ("Q6_K", 1, 96, None, None),          # k_sweep<Q6_K>, slices of 10
    ("Q6_K", 33, 48, None, None),
    ("Q6_K", 100, 40, None, None),        # k_gemm<Q6_K>
]


def _weights(rng, name, N):
    if name == "Q4_K":
        return H.random_q4k(rng, N, K)
    return H.random_blocks(rng, name, N, K, scale_lo=-12, scale_hi=-8)


def _run(F, dw, dx, db, N, M, qtype):
    dy = F.DeviceBuffer(M * N * 4)
    F.matmul_dev(dw, K, N, dx, dy, M, db, qtype=qtype)
    F.synchronize()
    y = dy.download(np.float32, (M, N))
    dy.close()
    return y


@pytest.mark.parametrize("name,M,N,path,expect", CASES)
def test_longest_native_rows(gpu, oracle, name, M, N, path, expect):
    F = gpu
    qtype = H.QTYPES[name][0]
    rng = np.random.default_rng(qtype * 7 + M * 131 + N)
    raw = _weights(rng, name, N)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    if path is not None:
        F.set_path(getattr(F, "PATH_" + path))
    try:
        chosen = F.matmul_path(M, K)
        print("max rows %s M=%d K=%d N=%d forced=%s path=%d" % (name, M, K, N, path, chosen), flush=True)
        if expect is not None:
            assert chosen == getattr(F, "PATH_" + expect)
        dw, dx, db = (F.DeviceBuffer.from_array(a) for a in (raw, x, bias))
        y = _run(F, dw, dx, db, N, M, qtype)
        y2 = _run(F, dw, dx, db, N, M, qtype)
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
