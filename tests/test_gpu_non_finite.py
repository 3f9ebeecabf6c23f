"""A NaN or an infinity in one token's activations, through every kernel
family and weight type of fh3_hip_matmul_dev, against the CPU oracle (fh3's
fh3_matmul, src/core/fh3_ops.c:317-404, whose fp32 sums carry the NaN or
infinity into every output of that token).

Bars: the oracle's row of that token is non-finite in every column, and so is
the product's; every other token's row is finite and within the rel-Frobenius
gate of the other product tests (2e-3).  Each kernel keeps a token's values in
its own rows of the matrix products, partial sums and group sums, so one
token's non-finite value must not reach another token: a product that mixed
tokens (a shared scale, a sum over the wrong rows) fails the second bar.
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3

# name, tokens, in, out, forced path (None: the automatic choice)
CASES = [
    ("Q4_K", 3, 2048, 96, "GEMV8"),     # k_gemv8
    ("Q4_K", 6, 2048, 96, "SWEEP"),     # k_sweep, one token block
    ("Q4_K", 6, 2048, 96, "SKINNY"),    # k_skinny
    ("Q4_K", 6, 2048, 96, "MIDM"),      # k_midm and its ordered sum
    ("Q4_K", 6, 2048, 96, "GEMM"),      # k_gemm at a few tokens
    ("Q4_K", 40, 13824, 64, None),      # k_sweep token blocks in K slices
    ("Q4_K", 70, 2048, 200, None),      # k_gemm with a K split
    ("Q4_K", 300, 1024, 96, None),      # k_gemm on 128-token tiles
    ("Q5_K", 6, 2048, 96, None),        # k_skinny<Q5_K> in K windows
    ("Q5_K", 70, 2048, 96, None),       # k_gemm<Q5_K>
    ("Q6_K", 6, 2048, 96, None),        # k_sweep<Q6_K>
    ("Q6_K", 6, 2048, 96, "SKINNY"),    # k_skinny<Q6_K>
    ("Q6_K", 70, 2048, 96, None),       # k_gemm<Q6_K>
    ("Q3_K", 6, 512, 64, None),         # fp16 rows, k_skinny16
    ("F16", 6, 96, 200, None),          # a row length off 256: zero-padded fp16 rows
    ("F16", 70, 512, 96, None),         # fp16 rows, k_gemm16
    ("BF16", 3, 32, 64, None),
    ("Q8_0", 5, 96, 130, None),
]


def _weights(rng, name, N, K):
    if name == "Q4_K":
        return H.random_q4k(rng, N, K)
    return H.random_blocks(rng, name, N, K, scale_lo=-12, scale_hi=-8)


@pytest.mark.parametrize("bad", [np.nan, np.inf])
@pytest.mark.parametrize("name,M,K,N,path", CASES)
def test_non_finite_token_stays_in_its_row(gpu, oracle, name, M, K, N, path, bad):
    F = gpu
    qtype = H.QTYPES[name][0]
    r, c = M // 2, K // 3
    print("non-finite %s M=%d K=%d N=%d path=%s x[%d][%d]=%s" % (name, M, K, N, path, r, c, bad), flush=True)
    rng = np.random.default_rng(qtype * 1009 + M * 31 + K + N)
    raw = _weights(rng, name, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[r, c] = bad
    bias = rng.standard_normal(N).astype(np.float32)
    yo = H.matmul_with(oracle, "fh3_oracle_matmul", raw, K, N, x, bias, qtype=qtype)
    assert not np.isfinite(yo[r]).any()
    if path is not None:
        F.set_path(getattr(F, "PATH_" + path))
    try:
        dw, dx, db = (F.DeviceBuffer.from_array(a) for a in (raw, x, bias))
        dy = F.DeviceBuffer(M * N * 4)
        F.matmul_dev(dw, K, N, dx, dy, M, db, qtype=qtype)
        F.synchronize()
        y = dy.download(np.float32, (M, N))
        for b in (dw, dx, db, dy):
            b.close()
    finally:
        F.set_path(F.PATH_AUTO)
    assert not np.isfinite(y[r]).any()
    keep = np.arange(M) != r
    assert np.isfinite(y[keep]).all()
    err = H.rel_fro(y[keep], yo[keep])
    print("  rel_fro = %.3e" % err, flush=True)
    assert err <= TOL
