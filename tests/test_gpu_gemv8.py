"""GPU parity of the one- to four-token kernel (FH3_HIP_PATH_GEMV8: int16
activations quantised inside the kernel, integer MFMA on the raw Q4_K
nibbles) against the CPU oracle, through the C-ABI.

Bar: rel-Frobenius <= 2e-3 of the oracle (fh3's CPU fh3_matmul), the
integration target's tolerance; bitwise reproducible run to run.
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _say(msg):
    print(msg, flush=True)


def _dev(F, raw, K, N, x, bias=None, path=None):
    M = x.shape[0]
    if path is not None:
        F.set_path(path)
    try:
        dw = F.DeviceBuffer.from_array(raw)
        dx = F.DeviceBuffer.from_array(np.ascontiguousarray(x, dtype=np.float32))
        dy = F.DeviceBuffer(M * N * 4)
        db = None if bias is None else F.DeviceBuffer.from_array(np.asarray(bias, dtype=np.float32))
        F.matmul_dev(dw, K, N, dx, dy, M, db)
        F.synchronize()
        return dy.download(np.float32, (M, N))
    finally:
        if path is not None:
            F.set_path(F.PATH_AUTO)


def _bits_equal(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return bool(((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))).all())


CASES = [
    # M, K, N, x-distribution, weight spread (decades), bias
    (1, 256, 16, "normal", 0.0, False),
    (1, 512, 37, "outliers", 0.0, True),
    (2, 768, 100, "normal", 2.0, False),
    (1, 2816, 130, "silu_gated", 0.0, True),
    (2, 5120, 640, "outliers", 0.0, True),
    (1, 5120, 5120, "normal", 0.0, False),
    (2, 5120, 1000, "silu_gated", 2.0, False),
    (1, 8192, 256, "normal", 2.0, True),
    (2, 8960, 48, "outliers", 0.0, False),
    (1, 13824, 96, "silu_gated", 0.0, False),
    (1, 17920, 64, "normal", 0.0, True),
    (2, 20480, 80, "outliers", 2.0, True),
    (3, 256, 16, "normal", 0.0, True),
    (3, 5120, 333, "outliers", 2.0, False),
    (4, 768, 100, "silu_gated", 0.0, True),
    (4, 5120, 5120, "normal", 0.0, False),
    (3, 8192, 200, "silu_gated", 2.0, True),
    (4, 12288, 64, "outliers", 0.0, False),
    # blocks left after the full rounds split into parts (N = 4103: one block of
    # 7 rows over 16 workgroups; N = 9000: 51 blocks in quarters)
    (2, 3072, 4103, "normal", 1.0, True),
    (4, 2048, 9000, "outliers", 0.0, True),
    (1, 5120, 17408, "silu_gated", 0.0, False),
]


@pytest.mark.parametrize("M,K,N,dist,spread,use_bias", CASES)
def test_gemv8_vs_oracle(gpu, oracle, M, K, N, dist, spread, use_bias):
    _say("gemv8 M=%d K=%d N=%d %s spread=%g bias=%d" % (M, K, N, dist, spread, use_bias))
    assert gpu.matmul_path(M, K) == gpu.PATH_GEMV8
    seed = M * 977 + K * 3 + N
    raw = gpu.synth_q4k_weights(seed, 1, N, K, 0.02, spread)
    x = gpu.synth_x(dist, seed, 2, M, K)
    bias = gpu.rng_normal(seed, 3, N) if use_bias else None
    y = _dev(gpu, raw, K, N, x, bias)
    yo = H.oracle_matmul(oracle, raw, K, N, x, bias)
    err = H.rel_fro(y, yo)
    _say("  rel_fro = %.3e" % err)
    assert np.isfinite(y).all()
    assert err <= TOL


def test_gemv8_more_accurate_than_fp16_paths(gpu, oracle):
    """The int16 activations of this path carry 14-15 significant bits per
    wavefront window, against 11 for the fp16 paths."""
    K, N = 5120, 512
    raw = gpu.synth_q4k_weights(5, 1, N, K, 0.02, 0.0)
    x = gpu.synth_x("normal", 5, 2, 2, K)
    yo = H.oracle_matmul(oracle, raw, K, N, x)
    e8 = H.rel_fro(_dev(gpu, raw, K, N, x), yo)
    es = H.rel_fro(_dev(gpu, raw, K, N, x, path=gpu.PATH_SKINNY), yo)
    _say("  gemv8 %.2e  skinny %.2e" % (e8, es))
    assert e8 <= 1e-4 and e8 < es


def test_gemv8_deterministic(gpu):
    K, N = 5120, 300
    raw = gpu.synth_q4k_weights(9, 1, N, K, 0.02, 0.0)
    for M in (1, 2, 3, 4):
        x = gpu.synth_x("outliers", 9, 2, M, K)
        a = _dev(gpu, raw, K, N, x)
        b = _dev(gpu, raw, K, N, x)
        assert _bits_equal(a, b)


def test_gemv8_extreme_magnitudes_and_zero_rows(gpu, oracle):
    """Per-window power-of-two scales: rows of 1e-30 and 1e4 keep their
    precision; a zero row gives exactly the bias."""
    rng = np.random.default_rng(12)
    K, N = 1024, 128
    raw = H.random_q4k(rng, N, K)
    bias = rng.standard_normal(N).astype(np.float32)
    x = rng.standard_normal((4, K)).astype(np.float32)
    x[0] *= 1e-30
    x[1] *= 1e4
    x[3] *= 1e-38    # subnormal inputs
    for M in (2, 4):
        y = _dev(gpu, raw, K, N, x[:M])
        yo = H.oracle_matmul(oracle, raw, K, N, x[:M])
        for r in range(M):
            assert H.rel_fro(y[r], yo[r]) <= TOL, (M, r)
    # a single large value among small ones in one window
    x = (rng.standard_normal((1, K)) * 1e-3).astype(np.float32)
    x[0, 77] = 50.0
    assert H.rel_fro(_dev(gpu, raw, K, N, x), H.oracle_matmul(oracle, raw, K, N, x)) <= TOL
    z = np.zeros((1, K), np.float32)
    assert np.array_equal(_dev(gpu, raw, K, N, z, bias)[0], bias)


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_gemv8_non_finite_activations_give_nan(gpu, bad):
    rng = np.random.default_rng(4)
    K, N = 2048, 64
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((4, K)).astype(np.float32)
    x[1, 1500] = bad
    for M in (2, 3, 4):
        y = _dev(gpu, raw, K, N, x[:M])
        assert np.isnan(y[1]).all()
        assert np.isfinite(np.delete(y, 1, axis=0)).all()


def test_gemv8_prepared_two_stage_equals_one_call(gpu):
    F = gpu
    K, N = 4096, 200
    raw = F.synth_q4k_weights(21, 1, N, K, 0.02, 0.0)
    dw = F.DeviceBuffer.from_array(raw)
    for M in (1, 2, 3, 4):
        x = F.synth_x("normal", 21, 2, M, K)
        dx = F.DeviceBuffer.from_array(x)
        prep = F.DeviceBuffer(F.prepared_bytes(M, K))
        F.prepare_x_dev(dx, M, K, prep)
        dy = F.DeviceBuffer(M * N * 4)
        F.matmul_prepared_dev(dw, K, N, prep, dy, M)
        F.synchronize()
        assert _bits_equal(dy.download(np.float32, (M, N)), _dev(F, raw, K, N, x))


def test_gemv8_graph_replay_matches_eager(gpu):
    F = gpu
    K, N = 5120, 512
    raw = F.synth_q4k_weights(31, 1, N, K, 0.02, 0.0)
    dw = F.DeviceBuffer.from_array(raw)
    x = F.synth_x("normal", 31, 2, 2, K)
    dx = F.DeviceBuffer.from_array(x)
    dy = F.DeviceBuffer(2 * N * 4)
    F.matmul_dev(dw, K, N, dx, dy, 2)
    F.synchronize()
    eager = dy.download(np.float32, (2, N))
    g = F.capture(lambda: F.matmul_dev(dw, K, N, dx, dy, 2))
    try:
        for _ in range(4):
            dy.fill(0)
            F.matmul_dev(dw, K, N, dx, dy, 2)   # eager work between replays
            dy.fill(0)
            F.synchronize()
            g.launch()
            F.synchronize()
            assert _bits_equal(dy.download(np.float32, (2, N)), eager)
    finally:
        g.close()
