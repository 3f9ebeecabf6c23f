"""GPU parity of the persistent small-M kernel (FH3_HIP_PATH_SWEEP: up to 64
tokens in one to four token blocks, 512 <= K <= 32768; fp16 activations held in registers, exact fp16
sc*q weights, the offsets dmin*m from the prepared group sums; rows of more
than 20 super-blocks in K slices whose partial sums are added in slice order;
17-64 tokens on rows of at most 16 super-blocks in groups of 32 tokens, each
group swept by its own workgroups)
against the CPU oracle, through the C-ABI.

Bars as for the other product kernels: rel-Frobenius <= 2e-3 against the
oracle (fh3's CPU fh3_matmul, src/core/fh3_ops.c:317-404), bitwise
reproducible run to run.  Cases cover one to sixteen tokens, one and many row
blocks per workgroup, partial row blocks, the window split of K = 5376 (21
super-blocks: the last wavefront's window shares one super-block with its
neighbour), the text-encoder GEMV shapes (sampled rows) and both epilogues.
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _say(msg):
    print(msg, flush=True)


def _buf(F, a):
    return F.DeviceBuffer.from_array(np.ascontiguousarray(a, dtype=np.float32))


def _sweep(F, raw, K, N, x, bias=None, path=None):
    M = x.shape[0]
    F.set_path(F.PATH_SWEEP if path is None else path)
    try:
        if path is None:
            assert F.matmul_path(M, K) == F.PATH_SWEEP
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
    (1, 512, 16, "normal", 0.0, False),
    (5, 1280, 4096, "normal", 0.0, True),
    (8, 2048, 200, "silu_gated", 2.0, True),      # partial last row block
    (9, 5376, 130, "outliers", 0.0, False),       # 21 super-blocks: shared window
    (13, 6144, 640, "normal", 2.0, False),        # 12 wavefronts
    (16, 6400, 96, "outliers", 1.0, True),        # two K slices of 13 and 12 super-blocks
    (12, 8192, 300, "silu_gated", 0.0, False),    # two slices of 16 (the text encoder's o-projection rows)
    (3, 13824, 130, "outliers", 0.0, False),      # three slices (18 each); past the int8 kernel's window
    (1, 25600, 64, "normal", 2.0, True),          # five slices of 20 (the text encoder's down-projection)
    (16, 25600, 520, "normal", 0.0, False),
    (17, 1024, 48, "normal", 0.0, True),          # one group of 32 tokens (two token blocks), the second with one token
    (24, 5120, 300, "outliers", 1.0, False),      # two token blocks, two K slices
    (32, 5120, 17408, "normal", 0.0, True),       # text-encoder MLP shape at 32 tokens (sampled rows)
    (29, 25600, 200, "silu_gated", 2.0, False),   # two token blocks in ten slices of ten super-blocks
    (33, 2048, 96, "normal", 0.0, True),          # two token groups, the second with one token
    (64, 4096, 200, "outliers", 1.0, True),       # two full token groups, eight wavefronts of two super-blocks
    (48, 5120, 640, "outliers", 1.0, True),       # three token blocks in three slices (7, 7, 6)
    (64, 8192, 200, "silu_gated", 0.0, False),    # four token blocks in four slices of eight
    (64, 5120, 17408, "normal", 0.0, False),      # text-encoder MLP shape at 64 tokens (sampled rows)
    (16, 5120, 5120, "normal", 0.0, False),       # text-encoder attention projection
    (16, 5120, 17408, "outliers", 0.0, True),     # text-encoder MLP, several blocks per workgroup
]


@pytest.mark.parametrize("M,K,N,dist,spread,use_bias", CASES)
def test_sweep_vs_oracle(gpu, oracle, M, K, N, dist, spread, use_bias):
    _say("sweep M=%d K=%d N=%d %s spread=%g bias=%d" % (M, K, N, dist, spread, use_bias))
    seed = M * 131 + K * 7 + N
    raw = gpu.synth_q4k_weights(seed, 1, N, K, 0.02, spread)
    x = gpu.synth_x(dist, seed, 2, M, K)
    bias = gpu.rng_normal(seed, 3, N) if use_bias else None
    y = _sweep(gpu, raw, K, N, x, bias)
    if N * M > 16 * 4096:  # oracle on a seeded subset of rows (rows are independent)
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


def test_sweep_golden_fixture(gpu, oracle):
    """The first 16 tokens of tests/golden/matmul_ref.bin (K=5376, N=192, bias)
    against the reference's own outputs."""
    t, K, N, M, raw, x, bias, yref = H.read_matmul_fixture()
    y = _sweep(gpu, raw, K, N, x[:16], bias)
    assert H.rel_fro(y, yref[:16]) <= TOL
    assert H.rel_fro(y, H.oracle_matmul(oracle, raw, K, N, x[:16], bias)) <= TOL


def test_sweep_deterministic_and_close_to_skinny(gpu, oracle):
    """Bitwise repeatable; k_skinny multiplies the same fp16 activations by
    the same exact weights, so the two differ only by fp32 summation order."""
    rng = np.random.default_rng(31)
    K, N, M = 3072, 384, 11
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    a = _sweep(gpu, raw, K, N, x)
    b = _sweep(gpu, raw, K, N, x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    s = _sweep(gpu, raw, K, N, x, path=gpu.PATH_SKINNY)
    assert H.rel_fro(a, s) <= 1e-5
    assert H.rel_fro(a, H.oracle_matmul(oracle, raw, K, N, x)) <= 6e-4


def test_sweep_extreme_row_magnitudes(gpu, oracle):
    rng = np.random.default_rng(32)
    K, N, M = 1024, 160, 12
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0] *= 1e-30
    x[1] *= 1e4
    x[2] = 0.0
    y = _sweep(gpu, raw, K, N, x)
    yo = H.oracle_matmul(oracle, raw, K, N, x)
    for r in range(M):
        if r != 2:
            assert H.rel_fro(y[r], yo[r]) <= TOL
    assert (y[2] == 0).all()


@pytest.mark.parametrize("bad", [np.nan, np.inf])
def test_sweep_non_finite_row_stays_in_its_row(gpu, oracle, bad):
    """A NaN or infinity in one token row makes that row non-finite and
    leaves the other rows exact to tolerance (each A row of the MFMAs and of
    the offset product is one token)."""
    rng = np.random.default_rng(33)
    K, N, M = 2048, 96, 6
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[3, 777] = bad
    y = _sweep(gpu, raw, K, N, x)
    assert not np.isfinite(y[3]).all()
    keep = [r for r in range(M) if r != 3]
    yo = H.oracle_matmul(oracle, raw, K, N, x[keep])
    assert np.isfinite(y[keep]).all()
    assert H.rel_fro(y[keep], yo) <= TOL


@pytest.mark.parametrize("K,M", [(5120, 16), (25600, 16), (5120, 32), (5120, 64)])
def test_sweep_prepared_equals_direct(gpu, K, M):
    """The two-stage API (prepare, then product) gives the one-call result bit
    for bit; the prepared form carries the group sums."""
    F = gpu
    rng = np.random.default_rng(34)
    N = 1024
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    direct = _sweep(F, raw, K, N, x)
    # fragments of 256 rows, their scales, and the group sums
    assert F.prepared_bytes(M, K) >= 256 * K * 2 + 256 * 4 + M * (K // 32) * 4
    dw, dx = F.DeviceBuffer.from_array(raw), _buf(F, x)
    prep = F.DeviceBuffer(F.prepared_bytes(M, K))
    dy = F.DeviceBuffer(M * N * 4)
    F.prepare_x_dev(dx, M, K, prep)
    F.matmul_prepared_dev(dw, K, N, prep, dy, M)
    F.synchronize()
    assert np.array_equal(dy.download(np.float32, (M, N)).view(np.uint32), direct.view(np.uint32))


@pytest.mark.parametrize("M,K", [(5, 2560), (16, 2560), (16, 8192), (32, 2560), (20, 8192), (64, 2560), (40, 1024),
                                 (24, 5120), (48, 5120), (64, 5120)])
def test_sweep_gate_residual_and_swiglu(gpu, oracle, M, K):
    """Both epilogues, in the kernel's store and (K slices) in the ordered sum
    of the slices, for one to four token blocks (K = 5120: the automatic
    choice at 17-64 tokens, in two or three slices)."""
    F = gpu
    rng = np.random.default_rng(410 + M + K)
    Fd = 192
    N = 2 * Fd
    raw = F.synth_q4k_weights(M + 17, 1, N, K, 0.05, 0.0)
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    gate = rng.standard_normal((M, N)).astype(np.float32)
    h = rng.standard_normal((M, N)).astype(np.float32)
    y = H.oracle_matmul(oracle, raw, K, N, x, bias)
    F.set_path(F.PATH_SWEEP)  # the automatic choice takes k_skinny above 16 tokens on rows below 5120
    try:
        assert F.matmul_path(M, K) == F.PATH_SWEEP
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
    finally:
        F.set_path(F.PATH_AUTO)
    sw = dout.download(np.float32, (M, Fd))
    gr = dh.download(np.float32, (M, N))
    ref = np.zeros((M, Fd), np.float32)
    H.elementwise(oracle, "fh3_oracle_", "swiglu", y.copy(), ref, M, Fd)
    assert H.rel_fro(sw, ref) <= TOL
    href = h.copy()
    H.elementwise(oracle, "fh3_oracle_", "gate_residual", href, gate, y, M, N)
    assert H.rel_fro(gr - h, href - h) <= TOL


@pytest.mark.parametrize("K,M", [(4096, 16), (13824, 16), (5120, 32), (5120, 64)])
def test_sweep_graph_replay_matches_eager(gpu, K, M):
    """Captured calls replayed three times equal the eager result (the
    prepared workspace and, for K slices, the partial sums are sized by the
    eager call first)."""
    F = gpu
    rng = np.random.default_rng(35)
    N = 512
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    dw, dx = F.DeviceBuffer.from_array(raw), _buf(F, x)
    dy = F.DeviceBuffer(M * N * 4)
    assert F.matmul_path(M, K) == F.PATH_SWEEP
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
