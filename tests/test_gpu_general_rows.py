"""fh3_matmul over every row length the reference's fh3_matmul takes
(src/core/fh3_ops.c:317-404 -> fh3_dequant, src/core/fh3_quant.c:284-318):
any `in` for F32, F16 and BF16 weights, whole 32-blocks for Q8_0, and rows
longer than 32768 values for every type.  The DiT calls it this way once per
forward: the audio and video patch projections take 32- and 96-value rows
(src/model/fh3_dit.c:352-353, dimensions src/cli/fh3_cli.c:943-945), the
tiny model's text projection 64-value rows.

Such rows are decoded to fp16 rows zero-padded to a multiple of 256, and the
activations are prepared into zero-padded fragments (k_xprep_any), then
k_skinny16 / k_gemm16.  Bar: rel-Frobenius <= 2e-3 of the oracle (the
reference's arithmetic restated), bitwise reproducible, and bitwise equal to
the same product with weights and activations zero-padded by the caller.
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3
F32, F16, BF16, Q8_0 = 0, 1, 30, 8
NAMES = {F32: "F32", F16: "F16", BF16: "BF16", Q8_0: "Q8_0"}


def _say(msg):
    print(msg, flush=True)


def _weights(rng, t, N, K):
    if t == F32:
        return (rng.standard_normal((N, K)) * 0.02).astype(np.float32).view(np.uint8).reshape(-1)
    return H.random_blocks(rng, NAMES.get(t) or t, N, K, scale_lo=-12, scale_hi=-8)


def _dev(F, raw, t, K, N, x, bias=None, path=None):
    M = x.shape[0]
    if path is not None:
        F.set_path(path)
    try:
        dw = F.DeviceBuffer.from_array(raw)
        dx = F.DeviceBuffer.from_array(np.ascontiguousarray(x, dtype=np.float32))
        dy = F.DeviceBuffer(M * N * 4)
        db = None if bias is None else F.DeviceBuffer.from_array(np.asarray(bias, dtype=np.float32))
        F.matmul_dev(dw, K, N, dx, dy, M, db, qtype=t)
        F.synchronize()
        return dy.download(np.float32, (M, N))
    finally:
        if path is not None:
            F.set_path(F.PATH_AUTO)


def _bits_equal(a, b):
    return bool(((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))).all())


CASES = [(t, K) for t in (F32, F16, BF16) for K in (1, 7, 32, 64, 96, 128, 200, 1000)] + \
        [(Q8_0, K) for K in (32, 64, 96, 128, 224)]


@pytest.mark.parametrize("t,K", CASES)
@pytest.mark.parametrize("M", [1, 5, 37, 300])
def test_short_rows_vs_oracle(gpu, oracle, t, K, M):
    _say("case: type %s K=%d M=%d" % (NAMES[t], K, M))
    rng = np.random.default_rng(1000 * t + 7 * K + M)
    N = 96 if M < 300 else 200
    raw = _weights(rng, t, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    y = _dev(gpu, raw, t, K, N, x, bias)
    yo = H.matmul_with(oracle, "fh3_oracle_matmul", raw, K, N, x, bias, qtype=t)
    err = H.rel_fro(y, yo)
    _say("  path %d rel_fro %.3e" % (gpu.matmul_path(M, K), err))
    assert np.isfinite(y).all()
    assert err <= TOL
    assert _bits_equal(y, _dev(gpu, raw, t, K, N, x, bias))


def _pad_cols(a, K, Kp):
    out = np.zeros((a.shape[0], Kp), dtype=a.dtype)
    out[:, :K] = a
    return out


@pytest.mark.parametrize("t", [F32, F16, BF16])
@pytest.mark.parametrize("K,M", [(200, 3), (96, 40), (1000, 300)])
def test_padding_is_exact(gpu, t, K, M):
    """The product of a short row equals, bit for bit, the product the caller
    gets by zero-padding weights and activations to whole super-blocks itself
    (which runs the ordinary path: k_xprep, and F16 rows read in place).  A
    wrong scale rule, a shifted fragment or non-zero padding fails it."""
    _say("case: padding type %s K=%d M=%d" % (NAMES[t], K, M))
    rng = np.random.default_rng(31 * K + M + t)
    N, Kp = 64, (K + 255) // 256 * 256
    if t == F32:
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        wp = _pad_cols(w, K, Kp)
        raw, rawp = w.view(np.uint8).reshape(-1), wp.view(np.uint8).reshape(-1)
    else:
        bits = H.random_blocks(rng, NAMES[t], N, K).view(np.uint16).reshape(N, K)
        raw = bits.view(np.uint8).reshape(-1)
        rawp = _pad_cols(bits, K, Kp).view(np.uint8).reshape(-1)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0, 0] = 300.0                       # the row maximum sits in the short row
    y = _dev(gpu, raw, t, K, N, x)
    yp = _dev(gpu, rawp, t, Kp, N, _pad_cols(x, K, Kp))
    assert _bits_equal(y, yp)


@pytest.mark.parametrize("t,K", [(F16, 40960), (F32, 33000), (BF16, 32769), (12, 33024), (14, 33280)])
@pytest.mark.parametrize("M", [1, 20, 70])
def test_long_rows_vs_oracle(gpu, oracle, t, K, M):
    """Rows longer than 32768 values (any type, in place of a refusal),
    including a Q4_K and a Q6_K weight: oracle on sampled output rows."""
    _say("case: long rows type %d K=%d M=%d" % (t, K, M))
    rng = np.random.default_rng(K + M)
    N = 48
    if t in (12, 14):
        raw = H.random_blocks(rng, "Q4_K" if t == 12 else "Q6_K", N, K, scale_lo=-12, scale_hi=-8)
    else:
        raw = _weights(rng, t, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    y = _dev(gpu, raw, t, K, N, x, bias)
    yo = H.matmul_with(oracle, "fh3_oracle_matmul", raw, K, N, x, bias, qtype=t)
    err = H.rel_fro(y, yo)
    _say("  rel_fro %.3e" % err)
    assert err <= TOL


@pytest.mark.parametrize("name,K", [("Q4_K", 200), ("Q6_K", 300), ("Q2_K", 128), ("Q8_0", 48)])
def test_partial_blocks_refused(gpu, name, K):
    """Rows that end inside a block are undefined in the reference (its
    decoders write whole blocks and leave the rest of the tile as it was):
    refused with FH3_E_INVALID, y untouched."""
    F = gpu
    t = H.QTYPES[name][0]
    dw = F.DeviceBuffer(F.row_bytes(t, K) * 16 + 256)
    dx = F.DeviceBuffer(4 * K * 2)
    dy = F.DeviceBuffer(4 * 16 * 2)
    dy.fill(0x7F)
    with pytest.raises(F.Fh3Error) as e:
        F.matmul_dev(dw, K, 16, dx, dy, 2, qtype=t)
    assert e.value.code == F.FH3_E_INVALID
    F.synchronize()
    assert (dy.download(np.uint8, (4 * 16 * 2,)) == 0x7F).all()


def test_dit_patch_projections(gpu, oracle):
    """The two run-once products of src/model/fh3_dit.c:352-353 at the CLI's
    dimensions (hidden 5376; audio 32-value rows, video 24 channels x 1x2x2
    patches = 96-value rows; F16 weights and F32 biases as in the GGUF), at
    the 640x384 39-frame sequence (6 text, 130 audio, 2880 video tokens),
    written into one residual stream h behind the text rows: each region
    against the oracle on sampled rows, the text rows untouched."""
    F = gpu
    rng = np.random.default_rng(352)
    hidden, T, A, V = 5376, 6, 130, 2880
    h = np.full(((T + A + V), hidden), np.nan, dtype=np.float32)
    h[:T] = rng.standard_normal((T, hidden))
    dh = F.DeviceBuffer.from_array(h)
    regions = []
    for K, n, r0 in ((32, A, T), (96, V, T + A)):
        w = (rng.standard_normal((hidden, K)) * 0.05).astype(np.float16)
        bias = (rng.standard_normal(hidden) * 0.1).astype(np.float32)
        x = rng.standard_normal((n, K)).astype(np.float32)
        dw = F.DeviceBuffer.from_array(w)
        dx = F.DeviceBuffer.from_array(x)
        db = F.DeviceBuffer.from_array(bias)
        F.matmul_dev(dw, K, hidden, dx, dh.ptr + 4 * r0 * hidden, n, db, qtype=F16)
        regions.append((w, bias, x, r0, n, K, dw, dx, db))
    F.synchronize()
    out = dh.download(np.float32, h.shape)
    assert np.array_equal(out[:T].view(np.uint32), h[:T].view(np.uint32))
    for w, bias, x, r0, n, K, *_ in regions:
        rows = np.unique(np.concatenate([np.arange(min(n, 8)), rng.integers(0, n, size=24)]))
        yo = H.matmul_with(oracle, "fh3_oracle_matmul", w.view(np.uint8).reshape(-1), K, hidden,
                           x[rows], bias, qtype=F16)
        err = H.rel_fro(out[r0 + rows], yo)
        _say("  K=%d tokens=%d rel_fro %.3e" % (K, n, err))
        assert err <= TOL
        assert np.isfinite(out[r0:r0 + n]).all()


def test_two_stage_short_rows(gpu):
    """fh3_hip_prepare_x_dev + fh3_hip_matmul_prepared_dev with a 96-value row
    equals fh3_hip_matmul_dev bit for bit, one prepared buffer for two
    weights of different types."""
    F = gpu
    rng = np.random.default_rng(96)
    K = 96
    for M in (3, 100):
        x = rng.standard_normal((M, K)).astype(np.float32)
        dx = F.DeviceBuffer.from_array(x)
        prep = F.DeviceBuffer(F.prepared_bytes(M, K))
        F.prepare_x_dev(dx, M, K, prep)
        for t in (F16, Q8_0):
            raw = _weights(rng, t, 80, K)
            dw = F.DeviceBuffer.from_array(raw)
            dy = F.DeviceBuffer(M * 80 * 4)
            F.matmul_prepared_dev(dw, K, 80, prep, dy, M, qtype=t)
            F.synchronize()
            two = dy.download(np.float32, (M, 80))
            assert _bits_equal(two, _dev(F, raw, t, K, 80, x))


def test_host_wrapper_short_rows(gpu, oracle):
    """The reference-signature host entry fh3_matmul (and its _scalar/_avx2
    twins, bitwise equal) on a 96-value F16 row with bias."""
    F = gpu
    rng = np.random.default_rng(7)
    K, N, M = 96, 5376, 9
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float16)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    raw = w.view(np.uint8).reshape(-1)
    y = F.matmul(raw, K, N, x, bias, qtype=F16)
    for v in ("fh3_matmul_scalar", "fh3_matmul_avx2"):
        assert _bits_equal(y, F.matmul(raw, K, N, x, bias, qtype=F16, variant=v))
    yo = H.matmul_with(oracle, "fh3_oracle_matmul", raw, K, N, x, bias, qtype=F16)
    assert H.rel_fro(y, yo) <= TOL


def test_workspace_bytes_general_rows(gpu):
    """fh3_hip_matmul_workspace_bytes: general rows decode into an fp16 buffer
    of out * round_up(in, 256) * 2 bytes (F16 too), beside the prepared
    activations; Q5_K / Q6_K rows are read in place and need no decode
    buffer: up to 64 tokens the prepared rows and the partial sums of at most
    K/1024 K windows, above 64 tokens the same workspace as Q4_K (prepared rows
    and the GEMM's partial sums)."""
    F = gpu
    N = 1000
    for t, K in ((F16, 96), (F32, 33000), (Q8_0, 224)):
        Kp = (K + 255) // 256 * 256
        for M in (1, 64, 300):
            want = N * Kp * 2 + F.prepared_bytes(M, K)
            assert F.matmul_workspace_bytes(K, N, M, qtype=t) == want
            assert F.matmul_workspace_bytes(K, N, M, prepared=True, qtype=t) == N * Kp * 2
    for t in (13, 14):
        part = F.matmul_workspace_bytes(5120, N, 16, qtype=t) - F.prepared_bytes(16, 5120)
        assert part % (16 * N * 4) == 0 and 0 <= part // (16 * N * 4) <= 5
        assert F.matmul_workspace_bytes(5120, N, 16, prepared=True, qtype=t) == part
        assert F.matmul_workspace_bytes(5120, N, 65, qtype=t) == F.matmul_workspace_bytes(5120, N, 65)
        assert F.matmul_workspace_bytes(5120, N, 65, qtype=t) > F.prepared_bytes(65, 5120)
