"""The DiT block's fused prologue and epilogues on the GPU (fh3_hip.h:
fh3_hip_prepare_x_norm_dev, fh3_hip_rownorm_dev, fh3_hip_matmul_epi_dev,
fh3_hip_matmul_prepared_epi_dev) against the oracle's restatement of the
reference's own sequence (src/model/fh3_dit.c:383-439: rmsnorm, modulate,
fh3_matmul, swiglu, gate_residual), through the C-ABI.

Bar: rel-Frobenius <= 2e-3 for anything that goes through a product (the
product's own tolerance); the fp32 row normalisation within 1e-5 relative.
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


def _oracle_norm(oracle, x, w, shift=None, scale=None):
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    n, d = y.shape
    H.elementwise(oracle, "fh3_oracle_", "rmsnorm", y, w, n, d, EPS)
    if shift is not None:
        H.elementwise(oracle, "fh3_oracle_", "modulate", y, shift, scale, n, d)
    return y


def _inputs(rng, M, K):
    x = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    shift = (0.2 * rng.standard_normal((M, K))).astype(np.float32)
    scale = (0.3 * rng.standard_normal((M, K))).astype(np.float32)
    return x, w, shift, scale


@pytest.mark.parametrize("M", [1, 3, 300])
@pytest.mark.parametrize("modulate", [False, True])
def test_rownorm_dev(gpu, oracle, M, modulate):
    F = gpu
    rng = np.random.default_rng(M + 10 * modulate)
    K = 5120
    x, w, shift, scale = _inputs(rng, M, K)
    dx, dw = _buf(F, x), _buf(F, w)
    ds, dc = (_buf(F, shift), _buf(F, scale)) if modulate else (None, None)
    dy = F.DeviceBuffer(M * K * 4)
    F.rownorm_dev(dx, M, K, dw, EPS, dy, ds, dc)
    F.synchronize()
    y = dy.download(np.float32, (M, K))
    yo = _oracle_norm(oracle, x, w, shift if modulate else None, scale if modulate else None)
    assert np.allclose(y, yo, rtol=1e-5, atol=1e-5 * np.abs(yo).max())
    F.rownorm_dev(dx, M, K, dw, EPS, dx, ds, dc)   # in place
    F.synchronize()
    assert np.array_equal(dx.download(np.float32, (M, K)), y)


@pytest.mark.parametrize("M", [1, 2, 5, 300])
@pytest.mark.parametrize("modulate", [False, True])
def test_prepare_norm_then_product(gpu, oracle, M, modulate):
    """rmsnorm (+ modulate) fused into the activation prep feeds the product
    exactly as the CPU sequence rmsnorm -> modulate -> fh3_matmul."""
    F = gpu
    _say("prepare_x_norm M=%d modulate=%d path=%d" % (M, modulate, F.matmul_path(M, 5120)))
    rng = np.random.default_rng(100 + M + modulate)
    K, N = 5120, 256
    x, w, shift, scale = _inputs(rng, M, K)
    raw = F.synth_q4k_weights(M + 3, 1, N, K, 0.02, 0.0)
    dx, dw, dwt = _buf(F, x), _buf(F, w), F.DeviceBuffer.from_array(raw)
    ds, dc = (_buf(F, shift), _buf(F, scale)) if modulate else (None, None)
    prep = F.DeviceBuffer(F.prepared_bytes(M, K))
    F.prepare_x_norm_dev(dx, M, K, dw, EPS, prep, ds, dc)
    dy = F.DeviceBuffer(M * N * 4)
    F.matmul_prepared_dev(dwt, K, N, prep, dy, M)
    F.synchronize()
    xn = _oracle_norm(oracle, x, w, shift if modulate else None, scale if modulate else None)
    yo = H.oracle_matmul(oracle, raw, K, N, xn)
    err = H.rel_fro(dy.download(np.float32, (M, N)), yo)
    _say("  rel_fro = %.3e" % err)
    assert err <= TOL


@pytest.mark.parametrize("M", [1, 2, 3, 4, 7, 300])
@pytest.mark.parametrize("prepared", [False, True])
def test_gate_residual_epilogue(gpu, oracle, M, prepared):
    F = gpu
    rng = np.random.default_rng(200 + M + prepared)
    K, N = 2048, 384
    raw = F.synth_q4k_weights(M + 7, 1, N, K, 0.02, 0.0)
    x = rng.standard_normal((M, K)).astype(np.float32)
    gate = rng.standard_normal((M, N)).astype(np.float32)
    h = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    dwt, dx, dg, dh, db = F.DeviceBuffer.from_array(raw), _buf(F, x), _buf(F, gate), _buf(F, h), _buf(F, bias)
    if prepared:
        prep = F.DeviceBuffer(F.prepared_bytes(M, K))
        F.prepare_x_dev(dx, M, K, prep)
        F.matmul_prepared_epi_dev(dwt, K, N, prep, M, F.EPI_GATE_RESIDUAL, dh, dg, db)
    else:
        F.matmul_epi_dev(dwt, K, N, dx, M, F.EPI_GATE_RESIDUAL, dh, dg, db)
    F.synchronize()
    out = dh.download(np.float32, (M, N))
    y = H.oracle_matmul(oracle, raw, K, N, x, bias)
    href = h.copy()
    H.elementwise(oracle, "fh3_oracle_", "gate_residual", href, gate, y, M, N)
    assert H.rel_fro(out - h, href - h) <= TOL
    assert H.rel_fro(out, href) <= TOL


@pytest.mark.parametrize("M", [1, 2, 3, 4, 7, 300])
@pytest.mark.parametrize("use_bias", [False, True])
def test_swiglu_epilogue(gpu, oracle, M, use_bias):
    F = gpu
    rng = np.random.default_rng(300 + M + use_bias)
    K, Fd = 1024, 192
    N = 2 * Fd
    raw = F.synth_q4k_weights(M + 11, 1, N, K, 0.05, 0.0)
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if use_bias else None
    dwt, dx = F.DeviceBuffer.from_array(raw), _buf(F, x)
    db = _buf(F, bias) if use_bias else None
    dout = F.DeviceBuffer(M * Fd * 4)
    F.matmul_epi_dev(dwt, K, N, dx, M, F.EPI_SWIGLU, dout, None, db)
    F.synchronize()
    out = dout.download(np.float32, (M, Fd))
    y = H.oracle_matmul(oracle, raw, K, N, x, bias)
    ref = np.zeros((M, Fd), np.float32)
    H.elementwise(oracle, "fh3_oracle_", "swiglu", y, ref, M, Fd)
    err = H.rel_fro(out, ref)
    _say("swiglu M=%d rel_fro = %.3e" % (M, err))
    assert err <= TOL


@pytest.mark.parametrize("M,K,Fd,n_sample", [(300, 512, 192, None), (300, 768, 256, None), (4096, 1024, 1024, 96)])
def test_swiglu_epilogue_direct_store(gpu, oracle, M, K, Fd, n_sample):
    """SwiGLU written by k_gemm's own epilogue (no split of K, so no k_midm_sum):
    full 256-token tiles and a partial last tile, through both the staged
    16-byte stores (aligned output) and the scalar stores (output 4 bytes off)."""
    F = gpu
    N = 2 * Fd
    assert F.matmul_path(M, K) == F.PATH_GEMM
    assert F.matmul_workspace_bytes(K, N, M, F.EPI_SWIGLU, prepared=True) == 0, "the product would split K"
    rng = np.random.default_rng(500 + M + K)
    raw = F.synth_q4k_weights(M + K, 1, N, K, 0.05, 0.0)
    x = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    dwt, dx, db = F.DeviceBuffer.from_array(raw), _buf(F, x), _buf(F, bias)
    outs = []
    for off in (0, 4):
        _say("swiglu direct store M=%d K=%d F=%d out offset %d" % (M, K, Fd, off))
        dout = F.DeviceBuffer(M * Fd * 4 + 16)
        F.matmul_epi_dev(dwt, K, N, dx, M, F.EPI_SWIGLU, dout.ptr + off, None, db)
        F.synchronize()
        o = np.empty((M, Fd), np.float32)
        F._check(F.lib().fh3_hip_memcpy_dtoh(o.ctypes.data, dout.ptr + off, o.nbytes), "dtoh")
        outs.append(o)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    rows = np.arange(M) if n_sample is None else np.unique(np.concatenate(
        [rng.choice(M, n_sample, replace=False), [0, 255, 256, M - 1]]))
    y = H.oracle_matmul(oracle, raw, K, N, x[rows], bias)
    ref = np.zeros((len(rows), Fd), np.float32)
    H.elementwise(oracle, "fh3_oracle_", "swiglu", y, ref, len(rows), Fd)
    err = H.rel_fro(outs[0][rows], ref)
    _say("  rel_fro = %.3e" % err)
    assert err <= TOL


def test_epilogue_argument_errors(gpu):
    F = gpu
    dw = F.DeviceBuffer(144 * 256)
    dx = F.DeviceBuffer(4 * 256)
    dy = F.DeviceBuffer(4 * 256)
    with pytest.raises(F.Fh3Error):      # SwiGLU needs out % 128 == 0
        F.matmul_epi_dev(dw, 256, 64, dx, 1, F.EPI_SWIGLU, dy)
    with pytest.raises(F.Fh3Error):      # gate-residual needs the gate
        F.matmul_epi_dev(dw, 256, 64, dx, 1, F.EPI_GATE_RESIDUAL, dy)
    with pytest.raises(F.Fh3Error):      # unknown epilogue
        F.matmul_epi_dev(dw, 256, 64, dx, 1, 7, dy)
    with pytest.raises(F.Fh3Error):      # fused epilogues take Q4_K weights
        F.matmul_epi_dev(dw, 256, 16, dx, 1, F.EPI_GATE_RESIDUAL, dy, dy, qtype=14)


@pytest.mark.parametrize("M", [2, 96, 300])
def test_dit_block_sequence(gpu, oracle, M):
    """The attention-free part of a DiT block (src/model/fh3_dit.c:383-439 with
    the attention output standing in for its input): norm1+modulate -> out
    projection with gate residual; norm2+modulate -> fc1 with SwiGLU -> fc2
    with gate residual.  Four launches on the GPU against the CPU sequence."""
    F = gpu
    rng = np.random.default_rng(400 + M)
    D, Fd = 1024, 512
    h = rng.standard_normal((M, D)).astype(np.float32)
    n1, s1, c1, n2, s2, c2, g1, g2 = (
        (1 + 0.1 * rng.standard_normal(D)).astype(np.float32), (0.1 * rng.standard_normal((M, D))).astype(np.float32),
        (0.2 * rng.standard_normal((M, D))).astype(np.float32), (1 + 0.1 * rng.standard_normal(D)).astype(np.float32),
        (0.1 * rng.standard_normal((M, D))).astype(np.float32), (0.2 * rng.standard_normal((M, D))).astype(np.float32),
        (0.5 * rng.standard_normal((M, D))).astype(np.float32), (0.5 * rng.standard_normal((M, D))).astype(np.float32))
    w_out = F.synth_q4k_weights(1, 1, D, D, 0.02, 0.0)
    w_fc1 = F.synth_q4k_weights(2, 1, 2 * Fd, D, 0.02, 0.0)
    w_fc2 = F.synth_q4k_weights(3, 1, D, Fd, 0.02, 0.0)
    # GPU
    dh = _buf(F, h)
    d = {k: _buf(F, v) for k, v in dict(n1=n1, s1=s1, c1=c1, n2=n2, s2=s2, c2=c2, g1=g1, g2=g2).items()}
    dwo, dw1, dw2 = (F.DeviceBuffer.from_array(w) for w in (w_out, w_fc1, w_fc2))
    prep = F.DeviceBuffer(F.prepared_bytes(M, max(D, Fd)))
    act = F.DeviceBuffer(M * Fd * 4)
    F.prepare_x_norm_dev(dh, M, D, d["n1"], EPS, prep, d["s1"], d["c1"])
    F.matmul_prepared_epi_dev(dwo, D, D, prep, M, F.EPI_GATE_RESIDUAL, dh, d["g1"])
    F.prepare_x_norm_dev(dh, M, D, d["n2"], EPS, prep, d["s2"], d["c2"])
    F.matmul_prepared_epi_dev(dw1, D, 2 * Fd, prep, M, F.EPI_SWIGLU, act)
    F.matmul_epi_dev(dw2, Fd, D, act, M, F.EPI_GATE_RESIDUAL, dh, d["g2"])
    F.synchronize()
    out = dh.download(np.float32, (M, D))
    # CPU: the reference's sequence through the oracle
    r = h.copy()
    xn = _oracle_norm(oracle, r, n1, s1, c1)
    y = H.oracle_matmul(oracle, w_out, D, D, xn)
    H.elementwise(oracle, "fh3_oracle_", "gate_residual", r, g1, y, M, D)
    xn = _oracle_norm(oracle, r, n2, s2, c2)
    y1 = H.oracle_matmul(oracle, w_fc1, D, 2 * Fd, xn)
    a = np.zeros((M, Fd), np.float32)
    H.elementwise(oracle, "fh3_oracle_", "swiglu", y1, a, M, Fd)
    y2 = H.oracle_matmul(oracle, w_fc2, Fd, D, a)
    H.elementwise(oracle, "fh3_oracle_", "gate_residual", r, g2, y2, M, D)
    err = H.rel_fro(out - h, r - h)
    _say("dit block M=%d: rel_fro of the block's update %.3e" % (M, err))
    assert err <= TOL
