"""Bit-exact prepared activations (fh3_hip_prepare_x_dev) for the large-M
products, from both preparation kernels: one row per workgroup (k_xprep) and,
from 8192 rows, eight rows per workgroup (k_xprep_r8).  The format, stated here
in numpy:

  scale   row t gets 2^e, e = clamp(15 - E, -126, 126) where max|x_t| = f * 2^E
          with f in [0.5, 1); e = 0 for an all-zero row; xs_inv[t] = 2^-e
  values  fp16(x * 2^e), rounded to nearest even
  layout  fragment (t // 32, k // 16) of 64 lanes x 8 fp16; element (t, k) is
          lane (t % 32) + 32 * ((k // 8) % 2), slot k % 8; the fragments of all
          Mpad = round_up(M, 256) rows (rows >= M zero, scale 1), then Mpad fp32
          scales at the next 256-byte boundary.

The normalising form (rmsnorm + modulate, fh3_hip_prepare_x_norm_dev) is
checked by decoding it against the oracle's rmsnorm -> modulate: each value
within one fp16 rounding of the row's scale (the norm's fp32 sum is added in a
different order, so an exact match is not expected).
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _say(msg):
    print(msg, flush=True)


def _buf(F, a):
    return F.DeviceBuffer.from_array(np.ascontiguousarray(a, dtype=np.float32))


def _row_exponents(x):
    mx = np.abs(x).max(axis=1)
    _, E = np.frexp(mx)
    e = np.clip(15 - E, -126, 126).astype(np.int32)
    e[mx == 0] = 0
    return e


def _expected(x, Mpad):
    M, K = x.shape
    e = _row_exponents(x)
    h = np.zeros((Mpad, K), np.float16)
    h[:M] = (x * np.ldexp(np.float32(1), e)[:, None].astype(np.float32)).astype(np.float16)
    frag = h.reshape(Mpad // 32, 32, K // 16, 2, 8).transpose(0, 2, 3, 1, 4).reshape(-1)
    xs = np.ones(Mpad, np.float32)
    xs[:M] = np.ldexp(np.float32(1), -e).astype(np.float32)
    return frag, xs


def _split(raw, Mpad, K):
    off = -(-Mpad * K * 2 // 256) * 256
    frag = raw[:Mpad * K * 2].view(np.float16)
    xs = raw[off:off + 4 * Mpad].view(np.float32)
    return frag, xs


def _inputs(rng, M, K):
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[::7] *= np.float32(1e-36)   # the scale clamps at 2^126 for these rows
    x[1::7] *= np.float32(1e30)   # negative exponents
    x[2::97] = 0.0                # all-zero rows
    x[3::5, ::3] = 0.0            # zeros inside rows
    return x


@pytest.mark.parametrize("M,K", [(300, 5120), (8192, 5120), (8200, 1024), (8300, 13824), (8256, 8192)])
def test_prepared_layout_bit_exact(gpu, M, K):
    F = gpu
    _say("prepare_x M=%d K=%d path=%d" % (M, K, F.matmul_path(M, K)))
    rng = np.random.default_rng(M + K)
    x = _inputs(rng, M, K)
    Mpad = -(-M // 256) * 256
    nbytes = F.prepared_bytes(M, K)
    prep = F.DeviceBuffer(nbytes)
    prep.upload(np.full(nbytes, 0xA5, np.uint8))   # every byte must be written
    F.prepare_x_dev(_buf(F, x), M, K, prep)
    F.synchronize()
    frag, xs = _split(prep.download(np.uint8, (nbytes,)), Mpad, K)
    efrag, exs = _expected(x, Mpad)
    assert np.array_equal(xs.view(np.uint32), exs.view(np.uint32))
    bad = np.flatnonzero(frag.view(np.uint16) != efrag.view(np.uint16))
    assert bad.size == 0, "first mismatching fp16 at %d of %d" % (bad[0], frag.size)


@pytest.mark.parametrize("M,K,modulate", [(300, 5120, True), (8192, 5120, False), (8200, 5120, True),
                                          (8448, 4096, True)])
def test_prepared_norm_decodes_to_oracle(gpu, oracle, M, K, modulate):
    F = gpu
    _say("prepare_x_norm M=%d K=%d modulate=%d" % (M, K, modulate))
    rng = np.random.default_rng(7 * M + K + modulate)
    x = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    x[5] *= np.float32(1e-20)     # rmsnorm lifts tiny rows to unit scale
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    shift = (0.2 * rng.standard_normal((M, K))).astype(np.float32) if modulate else None
    scale = (0.3 * rng.standard_normal((M, K))).astype(np.float32) if modulate else None
    Mpad = -(-M // 256) * 256
    nbytes = F.prepared_bytes(M, K)
    prep = F.DeviceBuffer(nbytes)
    F.prepare_x_norm_dev(_buf(F, x), M, K, _buf(F, w), EPS, prep,
                         None if shift is None else _buf(F, shift), None if scale is None else _buf(F, scale))
    F.synchronize()
    frag, xs = _split(prep.download(np.uint8, (nbytes,)), Mpad, K)
    dec = frag.astype(np.float32).reshape(Mpad // 32, K // 16, 2, 32, 8).transpose(0, 3, 1, 2, 4).reshape(Mpad, K)
    assert (dec[M:] == 0).all() and (xs[M:] == 1).all()
    dec = dec[:M] * xs[:M, None]
    y = x.copy()
    H.elementwise(oracle, "fh3_oracle_", "rmsnorm", y, w, M, K, EPS)
    if modulate:
        H.elementwise(oracle, "fh3_oracle_", "modulate", y, shift, scale, M, K)
    # fp16 keeps 11 bits at the row's top binade [2^14, 2^15): a half ulp there
    # is 2^-11 of the row maximum (plus a margin for the norm's fp32 rounding)
    bound = np.abs(y).max(axis=1, keepdims=True) * 2.0 ** -10
    err = np.abs(dec - y)
    _say("  worst err / bound = %.3f" % (err / bound).max())
    assert (err <= bound).all()
