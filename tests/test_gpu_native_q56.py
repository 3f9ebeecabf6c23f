"""GPU parity of the Q5_K and Q6_K weights read in place, by the small-M
kernels (k_skinny with QT = Q5_K / Q6_K, and for Q6_K the sweep, k_sweep with
QT = Q6_K, up to 64 tokens) and by the GEMM (k_gemm with QT = Q5_K / Q6_K,
above), through the C-ABI, against the CPU
oracle (fh3's fh3_matmul, src/core/fh3_ops.c:317-404, on the decoders of
src/core/fh3_quant.c:198-282).

Bars: rel-Frobenius <= 2e-3 against the oracle, bitwise reproducible.  The
one-hot cases pin the arithmetic itself: with one non-zero activation per
token the product is one weight.  The small-M kernel forms it as d * (sc * q)
with the integer part exact in fp16 (Q5_K always; Q6_K while
|sc * (q - 32)| <= 2048), so it matches the reference's fp32 value to fp32
rounding, where a product on weights rounded to fp16 would miss it by up to
2^-11 relative (Q6_K weights above that bound: at most that one rounding).
The GEMM stages every weight in fp16: for Q6_K exactly the reference's fp32
value rounded once, for Q5_K within one fp16 rounding of it.
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _say(msg):
    print(msg, flush=True)


def _tid(name):
    return H.QTYPES[name][0]


def _rb(name, K):
    return H.QTYPES[name][2] * (K // 256)


def _dev(F, raw, qtype, K, N, x, bias=None, path=None):
    M = x.shape[0]
    if path is not None:
        F.set_path(path)
    try:
        dw = F.DeviceBuffer.from_array(raw)
        dx = F.DeviceBuffer.from_array(np.ascontiguousarray(x, dtype=np.float32))
        dy = F.DeviceBuffer(M * N * 4)
        db = None if bias is None else F.DeviceBuffer.from_array(np.asarray(bias, dtype=np.float32))
        F.matmul_dev(dw, K, N, dx, dy, M, db, qtype=qtype)
        F.synchronize()
        return dy.download(np.float32, (M, N))
    finally:
        if path is not None:
            F.set_path(F.PATH_AUTO)


def _oracle(oracle, raw, name, K, N, x, bias=None, rows=None):
    t = _tid(name)
    if rows is None:
        return H.matmul_with(oracle, "fh3_oracle_matmul", raw, K, N, x, bias, qtype=t)
    rb = _rb(name, K)
    sub = np.ascontiguousarray(raw.reshape(N, rb)[rows]).reshape(-1)
    return H.matmul_with(oracle, "fh3_oracle_matmul", sub, K, len(rows), x, None if bias is None else bias[rows],
                         qtype=t)


CASES = [
    # M, K, N, bias
    (1, 256, 16, False),     # one super-block: a single wavefront
    (3, 1024, 80, True),
    (16, 5376, 130, False),  # 21 super-blocks: Q6_K rows and super-blocks alternate 4- and 2-byte alignment
    (17, 2048, 200, True),   # two token blocks, partial row block
    (40, 8192, 96, False),
    (64, 5120, 48, True),    # four token blocks
]


@pytest.mark.parametrize("name", ["Q5_K", "Q6_K"])
@pytest.mark.parametrize("M,K,N,use_bias", CASES)
def test_native_vs_oracle(gpu, oracle, name, M, K, N, use_bias):
    _say("native %s M=%d K=%d N=%d bias=%d" % (name, M, K, N, use_bias))
    rng = np.random.default_rng(_tid(name) * 7919 + M * 131 + K + N)
    raw = H.random_blocks(rng, name, N, K, scale_lo=-12, scale_hi=-8)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if use_bias else None
    y = _dev(gpu, raw, _tid(name), K, N, x, bias)
    yo = _oracle(oracle, raw, name, K, N, x, bias)
    err = H.rel_fro(y, yo)
    _say("  rel_fro = %.3e" % err)
    assert np.isfinite(y).all()
    assert err <= TOL
    assert np.array_equal(y.view(np.uint32), _dev(gpu, raw, _tid(name), K, N, x, bias).view(np.uint32))


# plus the sweep's shortest row (two super-blocks), slices with a short last
# one (54 super-blocks in slices of 10), a long row at one token
@pytest.mark.parametrize("M,K,N,use_bias", CASES + [(4, 25600, 96, True), (17, 6144, 64, False), (2, 512, 40, True),
                                                    (16, 13824, 64, False)])
def test_native_q6k_both_small_m_kernels(gpu, oracle, M, K, N, use_bias):
    """Q6_K up to 64 tokens on each of its kernels (forced): the sweep (weights
    in a ring, activations in registers, K slices past 16 super-blocks) and
    k_skinny (K windows when the row blocks are few), against the oracle;
    each bitwise repeatable."""
    F = gpu
    name = "Q6_K"
    rng = np.random.default_rng(4409 + M * 131 + K + N)
    raw = H.random_blocks(rng, name, N, K, scale_lo=-12, scale_hi=-8)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if use_bias else None
    yo = _oracle(oracle, raw, name, K, N, x, bias)
    for path in (F.PATH_SWEEP, F.PATH_SKINNY):
        _say("q6k M=%d K=%d N=%d path=%d" % (M, K, N, path))
        y = _dev(F, raw, _tid(name), K, N, x, bias, path=path)
        err = H.rel_fro(y, yo)
        _say("  rel_fro = %.3e" % err)
        assert np.isfinite(y).all() and err <= TOL
        assert np.array_equal(y.view(np.uint32), _dev(F, raw, _tid(name), K, N, x, bias, path=path).view(np.uint32))


def _onehot_weights(rng, name, N, K):
    """Random blocks with d = 1 + 2^-10 (and dmin 0 for Q5_K) so that d*sc*q is
    rarely an fp16 value."""
    raw = H.random_blocks(rng, name, N, K).reshape(N, K // 256, -1)
    d = np.array([1.0 + 2.0 ** -10], dtype=np.float16).view(np.uint8)
    if name == "Q5_K":
        raw[:, :, 0:2] = d
        raw[:, :, 2:4] = 0
    else:
        raw[:, :, 208:210] = d
    return raw.reshape(-1)


@pytest.mark.parametrize("name", ["Q5_K", "Q6_K"])
def test_native_weights_exact(gpu, oracle, name):
    """One-hot activations read single weights: the native product equals the
    reference's fp32 weight to fp32 rounding (the exact-integer weights)."""
    rng = np.random.default_rng(900 + _tid(name))
    K, N, M = 1024, 64, 24
    raw = _onehot_weights(rng, name, N, K)
    ks = rng.choice(K, M, replace=False)
    x = np.zeros((M, K), np.float32)
    x[np.arange(M), ks] = 1.0
    y = _dev(gpu, raw, _tid(name), K, N, x)
    w = H.oracle_dequant(oracle, raw, N, K, qtype=_tid(name))[:, ks].T  # [token][row]
    if name == "Q6_K":
        # weights with |sc*(q-32)| > 2048 are rounded once to fp16 in the kernel
        sc_q = np.rint(w / np.float32(1.0 + 2.0 ** -10)).astype(np.int64)
        exact = np.abs(sc_q) <= 2048
    else:
        exact = np.ones_like(w, dtype=bool)
    rel = np.abs(y - w) / np.maximum(np.abs(w), 1e-30)
    _say("  max rel (exact weights) = %.3e over %d" % (rel[exact & (w != 0)].max(), int((exact & (w != 0)).sum())))
    assert rel[exact & (w != 0)].max() <= 1e-6
    assert (y[exact & (w == 0)] == 0).all()
    assert rel[~exact].max(initial=0.0) <= 5e-4  # one fp16 rounding of an integer above 2048


GEMM_CASES = [
    # M, K, N, bias: one 128-token tile (one super-block; a partial row block),
    # 129-256 tokens on 128-token tiles, 256-token tiles, K split into windows
    # or not (2048 x 4096: enough tiles), odd super-block counts
    (65, 256, 16, False),
    (100, 1024, 80, True),
    (128, 5376, 130, False),
    (200, 2048, 200, True),
    (300, 8192, 96, False),
    (600, 5120, 300, True),
    (2048, 1024, 4096, False),
]


@pytest.mark.parametrize("name", ["Q5_K", "Q6_K"])
@pytest.mark.parametrize("M,K,N,use_bias", GEMM_CASES)
def test_native_gemm_vs_oracle(gpu, oracle, name, M, K, N, use_bias):
    """Above 64 tokens: the GEMM reads the blocks in place; oracle on up to 160
    seeded output rows (rows are independent)."""
    _say("native gemm %s M=%d K=%d N=%d bias=%d" % (name, M, K, N, use_bias))
    rng = np.random.default_rng(_tid(name) * 7907 + M * 131 + K + N)
    raw = H.random_blocks(rng, name, N, K, scale_lo=-12, scale_hi=-8)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if use_bias else None
    assert gpu.matmul_workspace_bytes(K, N, M, qtype=_tid(name)) == gpu.matmul_workspace_bytes(K, N, M)
    y = _dev(gpu, raw, _tid(name), K, N, x, bias)
    rows = np.arange(N) if N <= 160 else np.sort(rng.choice(N, 160, replace=False))
    yo = _oracle(oracle, raw, name, K, N, x, bias, rows=None if N <= 160 else rows)
    err = H.rel_fro(y[:, rows], yo)
    _say("  rel_fro = %.3e" % err)
    assert np.isfinite(y).all()
    assert err <= TOL
    assert np.array_equal(y.view(np.uint32), _dev(gpu, raw, _tid(name), K, N, x, bias).view(np.uint32))


@pytest.mark.parametrize("name", ["Q5_K", "Q6_K"])
def test_native_gemm_weights(gpu, oracle, name):
    """The identity as activations (512 tokens, K = 512) reads every weight of
    64 rows through the GEMM: Q6_K gives the reference's fp32 weight rounded
    once to fp16, bit for bit; Q5_K stays within one fp16 rounding of it."""
    rng = np.random.default_rng(950 + _tid(name))
    K, N = 512, 64
    raw = H.random_blocks(rng, name, N, K, scale_lo=-12, scale_hi=-8)
    x = np.eye(K, dtype=np.float32)
    y = _dev(gpu, raw, _tid(name), K, N, x)  # y[k][row] = w[row][k]
    w = H.oracle_dequant(oracle, raw, N, K, qtype=_tid(name)).T
    if name == "Q6_K":
        assert np.array_equal(y, w.astype(np.float16).astype(np.float32))
    else:
        err = np.abs(y - w)
        _say("  max |y - w| / max |w| = %.3e, rel_fro %.3e" % (err.max() / np.abs(w).max(), H.rel_fro(y, w)))
        assert err.max() <= 2.0 ** -11 * np.abs(w).max()
        assert H.rel_fro(y, w) <= 5e-4


# the text encoder's Q5_K / Q6_K tensor shapes (K -> N) at prompt lengths
TE_CASES = [("Q5_K", 5120, 1024), ("Q6_K", 5120, 1024), ("Q6_K", 8192, 5120), ("Q6_K", 25600, 5120)]


@pytest.mark.parametrize("name,K,N", TE_CASES)
def test_text_encoder_shapes(gpu, oracle, name, K, N):
    """Oracle on 64 seeded output rows (rows are independent) for M = 1, 4, 16
    and 64 tokens (k_skinny) and 65, 128, 300 and 600 (k_gemm)."""
    rng = np.random.default_rng(_tid(name) + K + N)
    raw = H.random_blocks(rng, name, N, K, scale_lo=-12, scale_hi=-8)
    rows = np.sort(rng.choice(N, 64, replace=False))
    for M in (1, 4, 16, 64, 65, 128, 300, 600):
        _say("te %s K=%d N=%d M=%d" % (name, K, N, M))
        x = rng.standard_normal((M, K)).astype(np.float32)
        y = _dev(gpu, raw, _tid(name), K, N, x)
        err = H.rel_fro(y[:, rows], _oracle(oracle, raw, name, K, N, x, rows=rows))
        _say("  rel_fro = %.3e" % err)
        assert np.isfinite(y).all()
        assert err <= TOL


@pytest.mark.parametrize("name", ["Q5_K", "Q6_K"])
def test_native_skinny_agrees_with_native_gemm(gpu, name):
    """The small-M kernel and the GEMM (forced path), both reading the blocks
    in place, agree to the fp16 rounding of the weights."""
    F = gpu
    rng = np.random.default_rng(77 + _tid(name))
    K, N, M = 3072, 112, 33
    raw = H.random_blocks(rng, name, N, K, scale_lo=-12, scale_hi=-8)
    x = rng.standard_normal((M, K)).astype(np.float32)
    a = _dev(F, raw, _tid(name), K, N, x)
    b = _dev(F, raw, _tid(name), K, N, x, path=F.PATH_GEMM)
    assert H.rel_fro(a, b) <= 1e-3
