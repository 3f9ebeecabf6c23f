"""Seeded random shapes through the automatic kernel choice of
fh3_hip_matmul_dev (Q4_K), against the CPU oracle (fh3's fh3_matmul,
src/core/fh3_ops.c:317-404), through the C-ABI.

Each case draws tokens from one of the ranges the dispatcher separates (1-4,
5-16, 17-64, 65-600), a row length of 1-24 super-blocks and any number of
output rows (partial row blocks and tiles), with or without bias, so the
cases land on every kernel family and near the boundaries between them
(k_gemv8, k_sweep, k_skinny, k_gemm with and without a K split).  Bars: the
rel-Frobenius gate of the other product tests, every output finite, and the
same bits on a second call.
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3
RANGES = [(1, 4), (5, 16), (17, 64), (65, 600)]


def _case(i):
    rng = np.random.default_rng(9100 + i)
    lo, hi = RANGES[i % len(RANGES)]
    M = int(rng.integers(lo, hi + 1))
    K = 256 * int(rng.integers(1, 25))
    N = int(rng.integers(16, 700))
    return M, K, N, bool(rng.integers(0, 2)), int(rng.integers(0, 3))


# and the boundaries the draws above can miss: 17-64 tokens on rows of 20 or
# more super-blocks (the sweep in K slices), the GEMM on one super-block and
# with a K split, the first and last token counts of each range, the GEMM's
# tile-width changes
CASES = [_case(i) for i in range(24)] + [
    (17, 5120, 300, True, 0), (33, 5376, 130, False, 1), (64, 8192, 200, True, 2), (65, 6144, 200, False, 0),
    (600, 256, 333, True, 1), (4, 8192, 100, False, 2), (5, 256, 17, True, 0), (16, 6400, 96, False, 1),
    # the GEMM's tile width changes at 257 and 385 tokens
    (257, 2048, 130, True, 0), (384, 5120, 200, False, 1), (385, 1024, 96, True, 2),
]


def _run(F, dw, dx, db, K, N, M):
    dy = F.DeviceBuffer(M * N * 4)
    F.matmul_dev(dw, K, N, dx, dy, M, db)
    F.synchronize()
    y = dy.download(np.float32, (M, N))
    dy.close()
    return y


@pytest.mark.parametrize("M,K,N,use_bias,dist", CASES)
def test_random_shape_vs_oracle(gpu, oracle, M, K, N, use_bias, dist):
    F = gpu
    print("random shape M=%d K=%d N=%d bias=%d path=%d" % (M, K, N, use_bias, F.matmul_path(M, K)), flush=True)
    seed = M * 31 + K + N * 7
    raw = F.synth_q4k_weights(seed, 1, N, K, 0.02, float(dist))
    x = F.synth_x(("normal", "outliers", "silu_gated")[dist], seed, 2, M, K)
    bias = F.rng_normal(seed, 3, N) if use_bias else None
    dw, dx = F.DeviceBuffer.from_array(raw), F.DeviceBuffer.from_array(x)
    db = None if bias is None else F.DeviceBuffer.from_array(bias)
    y = _run(F, dw, dx, db, K, N, M)
    y2 = _run(F, dw, dx, db, K, N, M)
    for b in (dw, dx, db):
        if b is not None:
            b.close()
    assert np.isfinite(y).all()
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    yo = H.oracle_matmul(oracle, raw, K, N, x, bias)
    err = H.rel_fro(y, yo)
    print("  rel_fro = %.3e" % err, flush=True)
    assert err <= TOL
