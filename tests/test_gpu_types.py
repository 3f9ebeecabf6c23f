"""fh3_matmul with weights of the other types the reference accepts (every
type its fh3_dequant decodes: src/core/fh3_ops.c:317-404), on the GPU through
the C-ABI, against the CPU oracle.  These weights are decoded per call to fp16
rows (the exact value rounded once) and multiplied by k_skinny16 / k_gemm16,
except Q5_K and Q6_K, which k_skinny (up to 64 tokens) and k_gemm (above)
read in place (tests/test_gpu_native_q56.py covers those kernels on their
own).

Bar: rel-Frobenius <= 2e-3 of the oracle, bitwise reproducible.
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3
TYPES = ["F32", "F16", "BF16", "Q8_0", "Q2_K", "Q3_K", "Q5_K", "Q6_K"]


def _say(msg):
    print(msg, flush=True)


def _weights(rng, name, N, K):
    if name == "F32":
        return (rng.standard_normal((N, K)) * 0.02).astype(np.float32).view(np.uint8).reshape(-1)
    return H.random_blocks(rng, name, N, K, scale_lo=-12, scale_hi=-8)


def _type_id(name):
    return 0 if name == "F32" else H.QTYPES[name][0]


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


def _bits_equal(a, b):
    return bool(((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))).all())


@pytest.mark.parametrize("name", TYPES)
@pytest.mark.parametrize("M,K,N,use_bias", [(1, 1024, 80, True), (7, 2560, 200, False), (40, 512, 130, True),
                                            (300, 1024, 160, False)])
def test_other_types_vs_oracle(gpu, oracle, name, M, K, N, use_bias):
    _say("type %s M=%d K=%d N=%d bias=%d" % (name, M, K, N, use_bias))
    t = _type_id(name)
    rng = np.random.default_rng(t * 1000 + M + K + N)
    raw = _weights(rng, name, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if use_bias else None
    y = _dev(gpu, raw, t, K, N, x, bias)
    yo = H.matmul_with(oracle, "fh3_oracle_matmul", raw, K, N, x, bias, qtype=t)
    err = H.rel_fro(y, yo)
    _say("  rel_fro = %.3e" % err)
    assert np.isfinite(y).all()
    assert err <= TOL
    assert _bits_equal(y, _dev(gpu, raw, t, K, N, x, bias))


@pytest.mark.parametrize("name", ["Q6_K", "Q5_K"])
def test_text_encoder_shape(gpu, oracle, name):
    """The text encoder's Q6_K / Q5_K tensors at K = 5120: one token and a
    prompt-sized block, oracle checked on a subset of output rows."""
    t = _type_id(name)
    rng = np.random.default_rng(t)
    K, N = 5120, 1024
    raw = _weights(rng, name, N, K)
    rb = H.QTYPES[name][2] * (K // 256)
    for M in (1, 77):
        x = rng.standard_normal((M, K)).astype(np.float32)
        y = _dev(gpu, raw, t, K, N, x)
        sub = slice(0, 96)
        yo = H.matmul_with(oracle, "fh3_oracle_matmul", raw[: 96 * rb], K, 96, x, None, qtype=t)
        assert H.rel_fro(y[:, sub], yo) <= TOL


def test_host_wrapper_and_forced_paths(gpu, oracle):
    """fh3_matmul (host pointers) takes a Q6_K weight; both product kernels
    (forced paths) give the oracle's result at the same shape."""
    t = _type_id("Q6_K")
    rng = np.random.default_rng(3)
    K, N, M = 1024, 96, 20
    raw = _weights(rng, "Q6_K", N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    yo = H.matmul_with(oracle, "fh3_oracle_matmul", raw, K, N, x, None, qtype=t)
    assert H.rel_fro(gpu.matmul(raw, K, N, x, qtype=t), yo) <= TOL
    for p in (gpu.PATH_SKINNY, gpu.PATH_GEMM):
        assert H.rel_fro(_dev(gpu, raw, t, K, N, x, path=p), yo) <= TOL


def test_prepared_two_stage_other_type(gpu):
    """Prepared activations feed a Q5_K weight, including the one- and
    two-token shapes whose prepared form is a copy of x."""
    F = gpu
    t = _type_id("Q5_K")
    rng = np.random.default_rng(8)
    K, N = 2048, 64
    raw = _weights(rng, "Q5_K", N, K)
    dw = F.DeviceBuffer.from_array(raw)
    for M in (1, 2, 9, 260):
        x = rng.standard_normal((M, K)).astype(np.float32)
        dx = F.DeviceBuffer.from_array(x)
        prep = F.DeviceBuffer(F.prepared_bytes(M, K))
        F.prepare_x_dev(dx, M, K, prep)
        dy = F.DeviceBuffer(M * N * 4)
        F.matmul_prepared_dev(dw, K, N, prep, dy, M, qtype=t)
        F.synchronize()
        assert _bits_equal(dy.download(np.float32, (M, N)), _dev(F, raw, t, K, N, x))


def test_unsupported_types_rejected(gpu):
    F = gpu
    dw = F.DeviceBuffer(4096)
    dx = F.DeviceBuffer(4 * 256)
    dy = F.DeviceBuffer(4 * 16)
    for qtype in (2, 3, 6, 7, 9, 15):  # Q4_0, Q4_1, Q5_0, Q5_1, Q8_1, Q8_K: no decoder in the reference
        with pytest.raises(F.Fh3Error) as e:
            F.matmul_dev(dw, 256, 16, dx, dy, 1, qtype=qtype)
        assert e.value.code == F.FH3_E_INVALID
