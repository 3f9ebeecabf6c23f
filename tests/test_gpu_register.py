"""Weight registration at the boundary (fh3_hip_register_weights): a host
range uploaded once and used in place by the host-pointer fh3_matmul /
fh3_dequant, through the C-ABI.  Results must be bitwise those of the
per-call upload path (same kernels, same bytes); the caching semantics are
checked by changing the host bytes behind the registration.
"""
import ctypes

import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu


def test_registered_matmul_bitwise_and_cached(gpu, oracle):
    F = gpu
    K, N, M = 2048, 320, 5
    w = F.synth_q4k_weights(31, 1, N, K, 0.02, 0.0)
    x = np.random.default_rng(3).standard_normal((M, K)).astype(np.float32)
    y0 = F.matmul(w, K, N, x)                      # per-call upload
    assert H.rel_fro(y0, H.oracle_matmul(oracle, w, K, N, x)) <= 2e-3
    d = F.register_weights(w)
    assert d and F.lib().fh3_hip_registered_ptr(w.ctypes.data, w.nbytes) == d
    try:
        y1 = F.matmul(w, K, N, x)
        assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
        # the device copy is used: host changes are not seen until re-registration
        saved = w.copy()
        w[:] = 0
        y2 = F.matmul(w, K, N, x)
        assert np.array_equal(y0.view(np.uint32), y2.view(np.uint32))
        F.register_weights(w)                      # refresh
        assert not F.matmul(w, K, N, x).any()      # all-zero blocks: d = dmin = 0
        w[:] = saved
        F.register_weights(w)
        # the device address works with the _dev entry point too
        dx = F.DeviceBuffer.from_array(x)
        dy = F.DeviceBuffer(M * N * 4)
        F.matmul_dev(d, K, N, dx, dy, M)
        F.synchronize()
        assert np.array_equal(dy.download(np.float32, (M, N)).view(np.uint32), y0.view(np.uint32))
    finally:
        F.unregister_weights(w)
    assert F.lib().fh3_hip_registered_ptr(w.ctypes.data, w.nbytes) is None
    w[:] = 0                                       # unregistered: uploaded per call again
    assert not F.matmul(w, K, N, x).any()


def test_weight_inside_registered_layer(gpu):
    """A packed layer is registered once; each matrix inside it (at a 16-byte
    aligned offset) is found by address."""
    F = gpu
    K = 1024
    a = F.synth_q4k_weights(40, 1, 64, K, 0.02, 0.0)
    b = F.synth_q4k_weights(41, 1, 96, K, 0.02, 0.0)
    layer = np.concatenate([a.ravel(), np.zeros(32, np.uint8), b.ravel()])
    x = np.random.default_rng(5).standard_normal((3, K)).astype(np.float32)
    ya, yb = F.matmul(a, K, 64, x), F.matmul(b, K, 96, x)
    F.register_weights(layer)
    try:
        la = layer[:a.size]
        lb = layer[a.size + 32:]
        assert F.lib().fh3_hip_registered_ptr(lb.ctypes.data, lb.nbytes) is not None
        layer[:] = 0           # the device copy still holds the old bytes
        assert np.array_equal(F.matmul(la, K, 64, x).view(np.uint32), ya.view(np.uint32))
        assert np.array_equal(F.matmul(lb, K, 96, x).view(np.uint32), yb.view(np.uint32))
    finally:
        F.unregister_weights(layer)


def test_registered_dequant(gpu):
    F = gpu
    t, rows, cols, raw, ref = H.read_q4k_fixture()
    raw = np.ascontiguousarray(raw)
    F.register_weights(raw)
    try:
        row_bytes = raw.size // rows
        out = np.zeros(cols, np.float32)
        F.lib().fh3_dequant(12, raw.ctypes.data + row_bytes, out.ctypes.data, cols)
        assert np.array_equal(out.view(np.uint32), ref[1].view(np.uint32))
    finally:
        F.unregister_weights(raw)


def test_registration_errors(gpu):
    F = gpu
    buf = np.zeros(4096, np.uint8)
    F.register_weights(buf)
    try:
        sub = buf[1024:2048]
        with pytest.raises(F.Fh3Error):            # overlapping range
            F.register_weights(sub)
    finally:
        F.unregister_weights(buf)
    with pytest.raises(F.Fh3Error):                # not registered
        F.unregister_weights(buf)
    d = ctypes.c_void_p()
    assert F.lib().fh3_hip_register_weights(None, 16, ctypes.byref(d)) != 0
