"""GPU parity of the HIP Q4_K path against the CPU oracle, through the C-ABI.

Bars: dequantisation bit-exact; products within rel-Frobenius 2e-3 of the
oracle (fh3's CPU fh3_matmul), the tolerance the integration target states;
results bitwise reproducible run to run.
"""
import ctypes

import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3  # max rel-Frobenius error vs the CPU path


def _say(msg):
    print(msg, flush=True)


def _dev_matmul(F, raw, K, N, x, bias=None, path=None):
    """Upload, run fh3_hip_matmul_dev, download."""
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


# --------------------------------------------------------------------------
# Dequantisation: bit-exact
# --------------------------------------------------------------------------
def _dev_dequant(F, raw, rows, n):
    src = F.DeviceBuffer.from_array(raw)
    dst = F.DeviceBuffer(rows * n * 4)
    F.dequant_dev(src, dst, rows, n)
    F.synchronize()
    return dst.download(np.float32, (rows, n))


def test_dequant_dev_golden_fixture(gpu):
    _say("dequant_dev: tests/golden/Q4_K.bin 4x512")
    t, rows, cols, raw, ref = H.read_q4k_fixture()
    out = _dev_dequant(gpu, raw, rows, cols)
    assert _bits_equal(out, ref)


def test_dequant_host_wrapper_golden_fixture(gpu):
    t, rows, cols, raw, ref = H.read_q4k_fixture()
    rb = gpu.row_bytes(12, cols)
    out = np.stack([gpu.dequant(12, raw[r * rb:(r + 1) * rb], cols) for r in range(rows)])
    assert _bits_equal(out, ref)


def _special_rows(rng, rows, K):
    raw = H.random_q4k(rng, rows, K).reshape(-1, 144)
    pats = np.array([0x0000, 0x8000, 0x0001, 0x0155, 0x03FF, 0x0400, 0x7BFF, 0xFBFF, 0xBC00, 0x3C00,
                     0x1400, 0xB400, 0x7C00, 0xFC00], dtype=np.uint16)
    raw[:, 0:2] = pats[rng.integers(0, len(pats), raw.shape[0])].view(np.uint8).reshape(-1, 2)
    raw[:, 2:4] = pats[rng.integers(0, len(pats), raw.shape[0])].view(np.uint8).reshape(-1, 2)
    raw[::7, 4:16] = 0xFF      # every scale and min = 63
    raw[::5, 16:] = 0xFF       # every nibble = 15
    raw[::11, 16:] = 0x00
    return raw.reshape(-1)


@pytest.mark.parametrize("kind", ["random", "special", "pattern"])
def test_dequant_dev_vs_oracle(gpu, oracle, kind):
    _say("dequant_dev vs oracle: %s" % kind)
    rng = np.random.default_rng(7)
    if kind == "random":
        rows, K = 37, 5376
        raw = H.random_q4k(rng, rows, K)
    elif kind == "special":
        rows, K = 64, 1024
        raw = _special_rows(rng, rows, K)
    else:
        # the byte pattern (i*37+13) & 0xFF of the reference's tiny.gguf Q4_K
        # tensor (tools/make_gguf_fixture.py:37-47): 2016 blocks, unusual d/dmin
        rows, K = 126, 4096
        raw = ((np.arange(rows * K // 256 * 144) * 37 + 13) & 0xFF).astype(np.uint8)
    out = _dev_dequant(gpu, raw, rows, K)
    want = H.oracle_dequant(oracle, raw, rows, K)
    assert _bits_equal(out, want)


# --------------------------------------------------------------------------
# Matmul vs the reference fixture
# --------------------------------------------------------------------------
@pytest.mark.parametrize("path", ["skinny", "gemm"])
def test_matmul_golden_fixture(gpu, oracle, path):
    """tests/golden/matmul_ref.bin (K=5376, N=192, M=37, bias)."""
    _say("matmul_ref.bin via %s" % path)
    t, K, N, M, raw, x, bias, yref = H.read_matmul_fixture()
    p = gpu.PATH_SKINNY if path == "skinny" else gpu.PATH_GEMM
    y = _dev_matmul(gpu, raw, K, N, x, bias, path=p)
    yo = H.oracle_matmul(oracle, raw, K, N, x, bias)
    assert H.rel_fro(y, yref) <= TOL
    assert H.rel_fro(y, yo) <= TOL


def test_host_fh3_matmul_variants_bitwise(gpu):
    """reference tests/unit/test_matmul.c:107-141: fh3_matmul, _scalar and _avx2
    agree bitwise, with and without bias."""
    t, K, N, M, raw, x, bias, yref = H.read_matmul_fixture()
    for b in (bias, None):
        ys = [gpu.matmul(raw, K, N, x, b, variant=v) for v in ("fh3_matmul", "fh3_matmul_scalar", "fh3_matmul_avx2")]
        assert _bits_equal(ys[0], ys[1]) and _bits_equal(ys[0], ys[2])
    assert H.rel_fro(gpu.matmul(raw, K, N, x, bias), yref) <= TOL


# --------------------------------------------------------------------------
# Seeded shapes, both kernels, the workload distributions
# --------------------------------------------------------------------------
CASES = [
    # M, K, N, path, x-distribution, weight spread (decades), bias
    (1, 256, 16, "skinny", "normal", 0.0, False),
    (1, 5120, 640, "skinny", "normal", 0.0, True),
    (4, 5120, 512, "skinny", "outliers", 0.0, False),
    (16, 2048, 200, "skinny", "silu_gated", 2.0, True),
    (17, 1024, 96, "skinny", "normal", 0.0, False),
    (33, 1536, 130, "skinny", "outliers", 2.0, True),
    (64, 4096, 256, "skinny", "normal", 0.0, False),
    # two to four token blocks: windows of 2-4 super-blocks whose activation
    # fragments are loaded one super-block ahead (the last window moved back
    # inside the row at K = 3328)
    (24, 6144, 160, "skinny", "outliers", 1.0, True),
    (40, 8192, 96, "skinny", "silu_gated", 0.0, False),
    (50, 3328, 200, "skinny", "normal", 2.0, True),
    (64, 5376, 80, "skinny", "normal", 0.0, True),
    (1, 512, 128, "gemm", "normal", 0.0, False),
    (65, 1024, 384, "gemm", "normal", 0.0, True),
    (300, 5120, 256, "gemm", "outliers", 0.0, False),
    (512, 2560, 200, "gemm", "silu_gated", 2.0, True),
    (777, 1280, 640, "gemm", "silu_gated", 0.0, False),
]


@pytest.mark.parametrize("M,K,N,path,dist,spread,use_bias", CASES)
def test_matmul_vs_oracle(gpu, oracle, M, K, N, path, dist, spread, use_bias):
    _say("matmul M=%d K=%d N=%d %s %s spread=%g bias=%d" % (M, K, N, path, dist, spread, use_bias))
    seed = M * 131 + K * 7 + N
    raw = gpu.synth_q4k_weights(seed, 1, N, K, 0.02, spread)
    x = gpu.synth_x(dist, seed, 2, M, K)
    bias = gpu.rng_normal(seed, 3, N) if use_bias else None
    p = gpu.PATH_SKINNY if path == "skinny" else gpu.PATH_GEMM
    y = _dev_matmul(gpu, raw, K, N, x, bias, path=p)
    yo = H.oracle_matmul(oracle, raw, K, N, x, bias)
    err = H.rel_fro(y, yo)
    _say("  rel_fro = %.3e" % err)
    assert np.isfinite(y).all()
    assert err <= TOL


@pytest.mark.parametrize("M,K,N", [(100, 1280, 384), (200, 13824, 640), (300, 5120, 1000)])
def test_gemm_split_k(gpu, oracle, M, K, N):
    """Large-M path with few tiles: K is split into windows (uneven last window
    for K = 1280, 27 windows for K = 13824) whose sums are added in window
    order; within tolerance of the oracle and bitwise repeatable."""
    _say("gemm split-K M=%d K=%d N=%d" % (M, K, N))
    rng = np.random.default_rng(M + K + N)
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    a = _dev_matmul(gpu, raw, K, N, x, bias, path=gpu.PATH_GEMM)
    b = _dev_matmul(gpu, raw, K, N, x, bias, path=gpu.PATH_GEMM)
    assert _bits_equal(a, b)
    err = H.rel_fro(a, H.oracle_matmul(oracle, raw, K, N, x, bias))
    _say("  rel_fro = %.3e" % err)
    assert err <= TOL


def test_matmul_deterministic_and_paths_agree(gpu, oracle):
    rng = np.random.default_rng(11)
    K, N, M = 2048, 256, 48
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    a = _dev_matmul(gpu, raw, K, N, x, path=gpu.PATH_SKINNY)
    b = _dev_matmul(gpu, raw, K, N, x, path=gpu.PATH_SKINNY)
    c = _dev_matmul(gpu, raw, K, N, x, path=gpu.PATH_GEMM)
    d = _dev_matmul(gpu, raw, K, N, x, path=gpu.PATH_GEMM)
    assert _bits_equal(a, b) and _bits_equal(c, d)
    yo = H.oracle_matmul(oracle, raw, K, N, x)
    # the small-M kernel keeps the weights exact (only activations are fp16);
    # the GEMM rounds dequantised weights to fp16 once
    assert H.rel_fro(a, yo) <= 3e-4
    assert H.rel_fro(c, yo) <= 6e-4


@pytest.mark.parametrize("M,K", [(20, 3072), (40, 6144), (64, 8192), (33, 3328), (64, 2304)])
def test_skinny_token_blocks_bitwise_repeatable_and_close_to_sweep(gpu, M, K):
    """k_skinny with two to four token blocks (activations of the next
    super-block loaded during the current one) is bitwise repeatable and
    agrees with the sweep, which multiplies the same fp16 activations by the
    same exact weights, to fp32 summation order: a fragment taken from the
    wrong super-block or token would show as an O(1) difference."""
    rng = np.random.default_rng(M * 7 + K)
    N = 144
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    a = _dev_matmul(gpu, raw, K, N, x, path=gpu.PATH_SKINNY)
    b = _dev_matmul(gpu, raw, K, N, x, path=gpu.PATH_SKINNY)
    assert _bits_equal(a, b)
    s = _dev_matmul(gpu, raw, K, N, x, path=gpu.PATH_SWEEP)
    assert H.rel_fro(a, s) <= 1e-5


def test_matmul_row_scaling_extreme_magnitudes(gpu, oracle):
    """Rows of 1e-30 and 1e4 magnitude: the per-row power-of-two scale keeps
    fp16 activations in range."""
    rng = np.random.default_rng(12)
    K, N, M = 1024, 128, 6
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0] *= 1e-30
    x[1] *= 1e4
    x[2] = 0.0
    for p in (gpu.PATH_SKINNY, gpu.PATH_GEMM):
        y = _dev_matmul(gpu, raw, K, N, x, path=p)
        yo = H.oracle_matmul(oracle, raw, K, N, x)
        for r in (0, 1, 3, 4, 5):
            assert H.rel_fro(y[r], yo[r]) <= TOL
        assert (y[2] == 0).all()


def test_matmul_dev_rejects_bad_arguments(gpu):
    F = gpu
    dw = F.DeviceBuffer(144 * 16)
    dx = F.DeviceBuffer(4 * 256)
    dy = F.DeviceBuffer(4 * 16)
    with pytest.raises(F.Fh3Error) as e:
        F.matmul_dev(dw, 256, 16, dx, dy, 1, qtype=2)   # Q4_0: no decoder in the reference
    assert e.value.code == F.FH3_E_INVALID
    with pytest.raises(F.Fh3Error):
        F.matmul_dev(dw, 200, 16, dx, dy, 1)          # in % 256 != 0
    with pytest.raises(F.Fh3Error):
        F.matmul_dev(dw.ptr + 4, 256, 16, dx, dy, 1)  # misaligned weights
    with pytest.raises(F.Fh3Error):
        F.matmul_dev(dw, 256, 16, dx, dy, 0)


def test_prepared_two_stage_equals_one_call(gpu):
    """fh3_hip_prepare_x_dev + fh3_hip_matmul_prepared_dev == fh3_hip_matmul_dev,
    bitwise, for both kernels, with one prepared buffer feeding two weights."""
    F = gpu
    rng = np.random.default_rng(13)
    K = 1024
    for M in (5, 300):
        x = rng.standard_normal((M, K)).astype(np.float32)
        dx = F.DeviceBuffer.from_array(x)
        prep = F.DeviceBuffer(F.prepared_bytes(M, K))
        F.prepare_x_dev(dx, M, K, prep)
        for N in (96, 256):
            raw = H.random_q4k(rng, N, K)
            dw = F.DeviceBuffer.from_array(raw)
            dy = F.DeviceBuffer(M * N * 4)
            F.matmul_prepared_dev(dw, K, N, prep, dy, M)
            F.synchronize()
            two = dy.download(np.float32, (M, N))
            one = _dev_matmul(F, raw, K, N, x)
            assert _bits_equal(one, two)


def test_graph_replay_matches_eager(gpu):
    """A captured sequence (two products, both kernel families) replayed
    several times, with eager work and synchronisations between replays;
    every replay must equal the eager result bitwise."""
    F = gpu
    rng = np.random.default_rng(21)
    K, N = 1024, 320
    raw = H.random_q4k(rng, N, K)
    dw = F.DeviceBuffer.from_array(raw)
    outs = []
    for M in (4, 260):
        x = rng.standard_normal((M, K)).astype(np.float32)
        dx = F.DeviceBuffer.from_array(x)
        dy = F.DeviceBuffer(M * N * 4)
        F.matmul_dev(dw, K, N, dx, dy, M)   # eager (also sizes the workspace)
        F.synchronize()
        outs.append((M, dx, dy, dy.download(np.float32, (M, N))))

    def seq():
        for M, dx, dy, _ in outs:
            F.matmul_dev(dw, K, N, dx, dy, M)

    g = F.capture(seq)
    try:
        for rep in range(4):
            for M, dx, dy, _ in outs:
                dy.fill(0)
            # unrelated eager work between replays
            F.matmul_dev(dw, K, N, outs[0][1], outs[0][2], outs[0][0])
            for M, dx, dy, _ in outs:
                dy.fill(0)
            F.synchronize()
            g.launch()
            F.synchronize()
            for M, dx, dy, ref in outs:
                assert _bits_equal(dy.download(np.float32, (M, N)), ref), (rep, M)
    finally:
        g.close()


@pytest.mark.parametrize("epi", [0, 1, 2])
def test_gemm_output_any_float_alignment(gpu, epi):
    """y (and the gate) may sit at any float offset: a 4-byte-offset output
    gives bit for bit what an aligned one does, for every epilogue (the GEMM
    stores full blocks 16 bytes at a time only when both are 16-byte aligned).
    K = 512 keeps K whole, so k_gemm's own epilogue writes y (not the ordered
    sum of a split-K product)."""
    F = gpu
    M, K, N = 300, 512, 256
    assert F.matmul_workspace_bytes(K, N, M, epi, prepared=True) == 0
    _say("gemm unaligned output epi=%d" % epi)
    rng = np.random.default_rng(31 + epi)
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    W = N // 2 if epi == 2 else N
    gate = rng.standard_normal((M, N)).astype(np.float32)
    h = rng.standard_normal((M, N)).astype(np.float32)
    dw = F.DeviceBuffer.from_array(raw)
    dx, db = F.DeviceBuffer.from_array(x), F.DeviceBuffer.from_array(bias)
    outs = []
    for off in (0, 4):
        dy = F.DeviceBuffer(M * W * 4 + 16)
        dg = F.DeviceBuffer(M * N * 4 + 16)
        y0 = h[:, :W] if epi == 1 else np.zeros((M, W), np.float32)
        F._check(F.lib().fh3_hip_memcpy_htod(dy.ptr + off, y0.ctypes.data, y0.nbytes), "htod")
        F._check(F.lib().fh3_hip_memcpy_htod(dg.ptr + off, gate.ctypes.data, gate.nbytes), "htod")
        assert F.matmul_path(M, K) == F.PATH_GEMM
        if epi == 0:
            F.matmul_dev(dw, K, N, dx, dy.ptr + off, M, db)
        else:
            F.matmul_epi_dev(dw, K, N, dx, M, epi, dy.ptr + off, dg.ptr + off if epi == 1 else None, db)
        F.synchronize()
        y = np.empty((M, W), np.float32)
        F._check(F.lib().fh3_hip_memcpy_dtoh(y.ctypes.data, dy.ptr + off, y.nbytes), "dtoh")
        outs.append(y)
    assert np.isfinite(outs[0]).all()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
