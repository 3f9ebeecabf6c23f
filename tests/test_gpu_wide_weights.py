"""Weight matrices of more than 4 GiB (out * row_bytes >= 2^32): rows whose
bytes lie past the 4 GiB mark, through every kernel that takes up to 64
tokens, against the CPU oracle (fh3's fh3_matmul, src/core/fh3_ops.c:317-404,
on the sampled rows); and above 64 tokens, where the GEMM addresses a matrix
with 32-bit byte offsets, a clean refusal (FH3_E_INVALID, y unwritten) before
any work is enqueued.

The matrix repeats 4099 random rows (a prime period) with the fp16 d of each
row's first super-block set from the row index, so a row read at a wrapped
offset gives another result.  Sampled: the first rows, the rows around the
4 GiB mark and the last rows.
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3
K = 5120
PERIOD = 4099


def _wide(name, seed):
    """Rows of `name` making more than 2^32 bytes, and their count and row bytes."""
    t, bl, bb, offs = H.QTYPES[name]
    rb = bb * (K // bl)
    N = (1 << 32) // rb + 257  # 256 whole rows past the mark and a partial last row block
    rng = np.random.default_rng(seed)
    base = H.random_q4k(rng, PERIOD, K) if name == "Q4_K" else H.random_blocks(rng, name, PERIOD, K, -12, -8)
    raw = np.resize(base.reshape(PERIOD, rb), (N, rb))
    # d values of the generator's magnitude: Q4_K 0.1-0.35, Q6_K about 2^-10
    lo, step = (0.1, 2.5e-4) if name == "Q4_K" else (1e-3, 2.5e-6)
    d = (lo + (np.arange(N) % 1021) * step).astype(np.float16)
    off = offs[0]
    raw[:, off:off + 2] = d.view(np.uint8).reshape(N, 2)
    assert N * rb >= 1 << 32
    return raw, N, rb


@pytest.fixture(scope="module")
def wide(request, gpu):
    F = gpu
    name = request.param
    raw, N, rb = _wide(name, 4242 if name == "Q4_K" else 4343)
    dw = F.DeviceBuffer.from_array(raw)
    yield name, raw, N, rb, dw
    dw.close()


# weight type, tokens, forced path (None: the automatic choice); k_midm takes Q4_K only
CASES = [(t, M, None) for t in ("Q4_K", "Q6_K") for M in (1, 4, 16, 40)] + [
    ("Q4_K", 8, "SKINNY"), ("Q6_K", 8, "SKINNY"), ("Q4_K", 24, "MIDM")]


def _rows(N, rb):
    mark = (1 << 32) // rb
    return np.unique(np.r_[0:16, mark - 16:mark + 16, N - 16:N])


@pytest.mark.parametrize("wide,M,path", CASES, indirect=["wide"])
def test_rows_past_4gib(gpu, oracle, wide, M, path):
    F = gpu
    name, raw, N, rb, dw = wide
    qtype = H.QTYPES[name][0]
    rng = np.random.default_rng(M)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    if path is not None:
        F.set_path(getattr(F, "PATH_" + path))
    try:
        print("wide %s N=%d (%d bytes) M=%d forced=%s path=%d" % (name, N, N * rb, M, path, F.matmul_path(M, K)),
              flush=True)
        dx, db = F.DeviceBuffer.from_array(x), F.DeviceBuffer.from_array(bias)
        dy = F.DeviceBuffer(M * N * 4)
        F.matmul_dev(dw, K, N, dx, dy, M, db, qtype=qtype)
        F.synchronize()
        y = dy.download(np.float32, (M, N))
        for b in (dx, db, dy):
            b.close()
    finally:
        F.set_path(F.PATH_AUTO)
    rows = _rows(N, rb)
    sub = np.ascontiguousarray(raw[rows]).reshape(-1)
    yo = H.matmul_with(oracle, "fh3_oracle_matmul", sub, K, len(rows), x, bias[rows], qtype=qtype)
    got = y[:, rows]
    assert np.isfinite(got).all()
    err = H.rel_fro(got, yo)
    print("  rel_fro = %.3e over %d sampled rows" % (err, len(rows)), flush=True)
    assert err <= TOL


@pytest.mark.parametrize("wide,M", [(t, M) for t in ("Q4_K", "Q6_K") for M in (65, 300)], indirect=["wide"])
def test_gemm_refuses_past_4gib(gpu, wide, M):
    F = gpu
    name, raw, N, rb, dw = wide
    qtype = H.QTYPES[name][0]
    x = np.ones((M, K), dtype=np.float32)
    dx = F.DeviceBuffer.from_array(x)
    dy = F.DeviceBuffer(M * N * 4)
    dy.fill(0x7F)
    with pytest.raises(F.Fh3Error) as e:
        F.matmul_dev(dw, K, N, dx, dy, M, None, qtype=qtype)
    assert e.value.code == F.FH3_E_INVALID
    assert "2^32" in str(e.value)
    F.synchronize()
    # nothing was written
    head = dy.download(np.uint8, (4096,))
    assert (head == 0x7F).all()
    # the host-pointer fh3_matmul refuses it before staging the weights: y
    # stays as it was (the wrapper fills it with NaN) and the reason is kept
    yh = F.matmul(raw, K, N, x, qtype=qtype)
    assert np.isnan(yh).all()
    assert b"2^32" in F.lib().fh3_hip_last_error()
    # and the next call in range still works
    y = F.DeviceBuffer(4 * N)
    F.matmul_dev(dw, K, N, dx, y, 1, None, qtype=qtype)
    F.synchronize()
    for b in (dx, dy, y):
        b.close()
