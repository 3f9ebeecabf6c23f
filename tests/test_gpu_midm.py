"""GPU parity of the middle-M kernel (FH3_HIP_PATH_MIDM: K split into windows
over 128-row workgroups, partial sums, ordered sum with the epilogue) against
the CPU oracle, through the C-ABI.

Bars as for the other product kernels: rel-Frobenius <= 2e-3 against the
oracle (fh3's CPU fh3_matmul), bitwise reproducible run to run.  The window
split covers uneven last windows (K/256 not a multiple of the window), one
window (S = 1), many windows and partial 128-row groups.
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3
EPS = 1e-6


def _say(msg):
    print(msg, flush=True)


def _buf(F, a):
    return F.DeviceBuffer.from_array(np.ascontiguousarray(a, dtype=np.float32))


def _midm(F, raw, K, N, x, bias=None):
    M = x.shape[0]
    F.set_path(F.PATH_MIDM)
    try:
        assert F.matmul_path(M, K) == F.PATH_MIDM
        dw, dx = F.DeviceBuffer.from_array(raw), _buf(F, x)
        dy = F.DeviceBuffer(M * N * 4)
        db = None if bias is None else _buf(F, bias)
        F.matmul_dev(dw, K, N, dx, dy, M, db)
        F.synchronize()
        return dy.download(np.float32, (M, N))
    finally:
        F.set_path(F.PATH_AUTO)


CASES = [
    # M, K, N, x-distribution, weight spread (decades), bias
    (1, 256, 16, "normal", 0.0, False),
    (5, 1280, 4096, "normal", 0.0, True),        # 5 super-blocks: windows of 3 and 2
    (16, 2048, 200, "silu_gated", 2.0, True),
    (17, 1024, 96, "normal", 0.0, False),
    (32, 5120, 640, "outliers", 0.0, False),
    (33, 1536, 130, "outliers", 2.0, True),
    (48, 13824, 640, "silu_gated", 2.0, False),  # 54 super-blocks, many windows
    (64, 4096, 4096, "normal", 0.0, False),      # the single-matmul configuration
    (64, 5120, 17408, "normal", 0.0, True),      # one window per 128 rows pair
]


@pytest.mark.parametrize("M,K,N,dist,spread,use_bias", CASES)
def test_midm_vs_oracle(gpu, oracle, M, K, N, dist, spread, use_bias):
    _say("midm M=%d K=%d N=%d %s spread=%g bias=%d" % (M, K, N, dist, spread, use_bias))
    seed = M * 131 + K * 7 + N
    raw = gpu.synth_q4k_weights(seed, 1, N, K, 0.02, spread)
    x = gpu.synth_x(dist, seed, 2, M, K)
    bias = gpu.rng_normal(seed, 3, N) if use_bias else None
    y = _midm(gpu, raw, K, N, x, bias)
    if N * M > 64 * 4096:  # oracle on a seeded subset of rows (rows are independent)
        rows = np.sort(np.random.default_rng(seed).choice(N, 512, replace=False))
        sub = np.ascontiguousarray(raw.reshape(N, -1)[rows])
        yo = H.oracle_matmul(oracle, sub, K, len(rows), x, None if bias is None else bias[rows])
        y = y[:, rows]
    else:
        yo = H.oracle_matmul(oracle, raw, K, N, x, bias)
    err = H.rel_fro(y, yo)
    _say("  rel_fro = %.3e" % err)
    assert np.isfinite(y).all()
    assert err <= TOL


def test_midm_golden_fixture(gpu, oracle):
    """tests/golden/matmul_ref.bin (K=5376, N=192, M=37, bias)."""
    t, K, N, M, raw, x, bias, yref = H.read_matmul_fixture()
    y = _midm(gpu, raw, K, N, x, bias)
    assert H.rel_fro(y, yref) <= TOL
    assert H.rel_fro(y, H.oracle_matmul(oracle, raw, K, N, x, bias)) <= TOL


def test_midm_deterministic_and_close_to_gemm(gpu, oracle):
    """Bitwise repeatable; the weights are rounded to fp16 as k_gemm rounds
    them, so both stay within the GEMM's own distance from the oracle."""
    rng = np.random.default_rng(21)
    K, N, M = 3072, 384, 40
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    a = _midm(gpu, raw, K, N, x)
    b = _midm(gpu, raw, K, N, x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    yo = H.oracle_matmul(oracle, raw, K, N, x)
    assert H.rel_fro(a, yo) <= 6e-4


def test_midm_extreme_row_magnitudes(gpu, oracle):
    rng = np.random.default_rng(22)
    K, N, M = 1024, 160, 20
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0] *= 1e-30
    x[1] *= 1e4
    x[2] = 0.0
    y = _midm(gpu, raw, K, N, x)
    yo = H.oracle_matmul(oracle, raw, K, N, x)
    for r in range(M):
        if r != 2:
            assert H.rel_fro(y[r], yo[r]) <= TOL
    assert (y[2] == 0).all()


@pytest.mark.parametrize("M", [3, 24, 64])
def test_midm_gate_residual_and_swiglu(gpu, oracle, M):
    F = gpu
    rng = np.random.default_rng(400 + M)
    K, Fd = 2048, 192
    N = 2 * Fd
    raw = F.synth_q4k_weights(M + 13, 1, N, K, 0.05, 0.0)
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    gate = rng.standard_normal((M, N)).astype(np.float32)
    h = rng.standard_normal((M, N)).astype(np.float32)
    y = H.oracle_matmul(oracle, raw, K, N, x, bias)
    F.set_path(F.PATH_MIDM)
    try:
        dwt, dx, db = F.DeviceBuffer.from_array(raw), _buf(F, x), _buf(F, bias)
        # SwiGLU on the [val | gate] rows
        dout = F.DeviceBuffer(M * Fd * 4)
        F.matmul_epi_dev(dwt, K, N, dx, M, F.EPI_SWIGLU, dout, None, db)
        # gate residual, through the two-stage API
        dg, dh = _buf(F, gate), _buf(F, h)
        prep = F.DeviceBuffer(F.prepared_bytes(M, K))
        F.prepare_x_dev(dx, M, K, prep)
        F.matmul_prepared_epi_dev(dwt, K, N, prep, M, F.EPI_GATE_RESIDUAL, dh, dg, db)
        F.synchronize()
        sw = dout.download(np.float32, (M, Fd))
        gr = dh.download(np.float32, (M, N))
    finally:
        F.set_path(F.PATH_AUTO)
    ref = np.zeros((M, Fd), np.float32)
    H.elementwise(oracle, "fh3_oracle_", "swiglu", y.copy(), ref, M, Fd)
    assert H.rel_fro(sw, ref) <= TOL
    href = h.copy()
    H.elementwise(oracle, "fh3_oracle_", "gate_residual", href, gate, y, M, N)
    assert H.rel_fro(gr - h, href - h) <= TOL


def test_midm_graph_replay_matches_eager(gpu):
    """Captured twice-replayed calls equal the eager result (the partial-sum
    workspace is sized by the eager call first)."""
    F = gpu
    rng = np.random.default_rng(23)
    K, N, M = 4096, 512, 64
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    F.set_path(F.PATH_MIDM)
    try:
        dw, dx = F.DeviceBuffer.from_array(raw), _buf(F, x)
        dy = F.DeviceBuffer(M * N * 4)
        F.matmul_dev(dw, K, N, dx, dy, M)
        F.synchronize()
        eager = dy.download(np.float32, (M, N))
        g = F.capture(lambda: F.matmul_dev(dw, K, N, dx, dy, M))
        for _ in range(3):
            dy.upload(np.zeros((M, N), np.float32))
            g.launch()
            F.synchronize()
            assert np.array_equal(dy.download(np.float32, (M, N)).view(np.uint32), eager.view(np.uint32))
        g.close()
    finally:
        F.set_path(F.PATH_AUTO)
