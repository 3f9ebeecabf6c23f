"""GPU dequantisation of every block format the reference decodes, through the
C-ABI (fh3_hip_dequant_dev and the reference-signature fh3_dequant), against
the reference's golden fixtures and the CPU oracle.  Bar: bit-exact (NaNs
compared as NaNs).
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

NAMES = sorted(H.QTYPES)


def _say(msg):
    print(msg, flush=True)


def _bits_equal(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return bool(((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))).all())


def _dev_dequant(F, qtype, raw, rows, n):
    src = F.DeviceBuffer.from_array(np.ascontiguousarray(raw, dtype=np.uint8))
    dst = F.DeviceBuffer(rows * n * 4)
    F.dequant_dev(src, dst, rows, n, qtype=qtype)
    F.synchronize()
    return dst.download(np.float32, (rows, n))


@pytest.mark.parametrize("name", NAMES)
def test_fixture_dev_and_host(gpu, name):
    """reference tests/unit/test_quant.c:40-130, on the GPU."""
    _say("dequant fixture %s" % name)
    t, rows, cols, raw, ref = H.read_quant_fixture(name)
    assert _bits_equal(_dev_dequant(gpu, t, raw, rows, cols), ref)
    rb = gpu.row_bytes(t, cols)
    host = np.stack([gpu.dequant(t, raw[r * rb:(r + 1) * rb], cols) for r in range(rows)])
    assert _bits_equal(host, ref)


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("finite", [True, False])
def test_random_blocks_vs_oracle(gpu, oracle, name, finite):
    """Many rows (grid well past one workgroup); with `finite` False the
    scale fields are raw random bytes (Inf / NaN / subnormal fp16 scales)."""
    _say("dequant random %s finite=%s" % (name, finite))
    t = H.QTYPES[name][0]
    rng = np.random.default_rng(1000 + t + 7 * finite)
    rows, cols = 97, 4096
    raw = H.random_blocks(rng, name, rows, cols, finite=finite)
    if not finite and name not in ("F16", "BF16"):
        raw = rng.integers(0, 256, size=raw.size, dtype=np.uint8)
    out = _dev_dequant(gpu, t, raw, rows, cols)
    assert _bits_equal(out, H.oracle_dequant(oracle, raw, rows, cols, qtype=t))


@pytest.mark.parametrize("name", ["F16", "BF16"])
def test_half_every_bit_pattern(gpu, oracle, name):
    """All 65536 patterns, as one row and as 3 rows of an odd length."""
    t = H.QTYPES[name][0]
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.uint8)
    out = _dev_dequant(gpu, t, raw, 1, 65536)
    assert _bits_equal(out, H.oracle_dequant(oracle, raw, 1, 65536, qtype=t))
    sub = raw[: 3 * 2 * 1001]
    out = _dev_dequant(gpu, t, sub, 3, 1001)
    assert _bits_equal(out, H.oracle_dequant(oracle, sub, 3, 1001, qtype=t))


def test_f32_copy(gpu):
    x = np.random.default_rng(3).standard_normal((5, 300)).astype(np.float32)
    out = _dev_dequant(gpu, 0, x.view(np.uint8).reshape(-1), 5, 300)
    assert _bits_equal(out, x)


@pytest.mark.parametrize("name", ["Q8_0", "Q3_K", "Q6_K", "BF16"])
def test_host_wrapper_partial_blocks(gpu, oracle, name):
    """fh3_dequant writes only whole blocks (the reference's decoders do the
    same); the tail of dst keeps its contents."""
    t, bl = H.QTYPES[name][0], H.QTYPES[name][1]
    rng = np.random.default_rng(t)
    n = 1024 - 3
    raw = H.random_blocks(rng, name, 1, 1024)
    out = gpu.dequant(t, raw, n)
    want = np.zeros(n, np.float32)
    oracle.fh3_oracle_dequant(t, raw.ctypes.data, want.ctypes.data, n)
    assert _bits_equal(out, want)
    if bl > 1:
        assert (out[(n // bl) * bl:] == 0).all()


def test_dequant_dev_rejects_bad_arguments(gpu):
    F = gpu
    src = F.DeviceBuffer(4096)
    dst = F.DeviceBuffer(4096 * 4)
    for qtype, n in ((2, 256), (15, 256), (99, 256), (8, 48), (10, 200), (14, 128)):
        with pytest.raises(F.Fh3Error) as e:
            F.dequant_dev(src, dst, 1, n, qtype=qtype)
        assert e.value.code == F.FH3_E_INVALID
    with pytest.raises(F.Fh3Error):
        F.dequant_dev(src.ptr + 2, dst, 1, 256, qtype=14)     # misaligned source
    with pytest.raises(F.Fh3Error):
        F.dequant_dev(src, dst, 0, 256, qtype=14)
