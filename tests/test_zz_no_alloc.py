"""fh3_hip_matmul_noalloc_dev: the product with its workspace in the library's
fixed scratch array, through the C-ABI, against fh3_hip_matmul_dev (same
kernels, so bit for bit) on every kernel family.

Each case runs two calls in a row, the second with fewer tokens, because the
scratch array keeps the previous call's contents: a kernel that read stale
prepared rows or partial sums would show it there.  Shapes beyond the array
are refused with FH3_E_INVALID.  The call can be captured into a graph the
first time it is made (it allocates nothing).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _pair(F, K, N, M, seed):
    raw = F.synth_q4k_weights(seed, 1, N, K, 0.02, 0.0)
    x = F.synth_x("outliers", seed, 2, M, K)
    bias = F.synth_x("normal", seed, 3, 1, N)[0]
    return F.DeviceBuffer.from_array(raw), F.DeviceBuffer.from_array(x), F.DeviceBuffer.from_array(bias)


# (K, N, first n_tok, second n_tok): k_gemv8; k_sweep then k_gemv8; k_sweep in
# K slices (partial sums in the scratch array); k_skinny; split-K k_gemm;
# k_gemm with K whole
CASES = [(5120, 5120, 2, 1), (5120, 17408, 16, 4), (13824, 5120, 64, 24), (2048, 1024, 40, 20),
         (5120, 5120, 512, 65), (4096, 4096, 4096, 300)]


@pytest.mark.parametrize("K,N,M1,M2", CASES)
def test_noalloc_matches_matmul_dev(gpu, K, N, M1, M2):
    F = gpu
    dw, dx, db = _pair(F, K, N, M1, K + N + M1)
    for M in (M1, M2):
        print("case: noalloc K=%d N=%d M=%d path=%d workspace=%d" % (
            K, N, M, F.matmul_path(M, K), F.matmul_workspace_bytes(K, N, M)), flush=True)
        assert F.matmul_workspace_bytes(K, N, M) <= F.NOALLOC_SCRATCH_BYTES
        want_b = F.DeviceBuffer(M * N * 4)
        got_b = F.DeviceBuffer(M * N * 4)
        got_b.fill(0xFF)
        F.matmul_dev(dw, K, N, dx, want_b, M, db)
        F.matmul_noalloc_dev(dw, K, N, dx, got_b, M, db)
        F.synchronize()
        want = want_b.download(np.float32, (M, N))
        got = got_b.download(np.float32, (M, N))
        assert np.isfinite(want).all()
        assert np.array_equal(_bits(got), _bits(want)), (K, N, M)


def test_noalloc_refuses_what_does_not_fit(gpu):
    F = gpu
    K, N, M = 5120, 5120, 8192      # 84 MB of prepared activations
    assert F.matmul_workspace_bytes(K, N, M) > F.NOALLOC_SCRATCH_BYTES
    dw = F.DeviceBuffer(N * (K // 256) * 144)
    dx = F.DeviceBuffer(M * K * 4)
    dy = F.DeviceBuffer(M * N * 4)
    with pytest.raises(F.Fh3Error) as ei:
        F.matmul_noalloc_dev(dw, K, N, dx, dy, M)
    assert ei.value.code == F.FH3_E_INVALID and "scratch" in str(ei.value)
    # up to 64 tokens, long rows: the K-split partial sums set the need
    K2, N2, M2 = 32768, 12224, 64
    assert F.matmul_workspace_bytes(K2, N2, M2) > F.NOALLOC_SCRATCH_BYTES
    assert F.matmul_workspace_bytes(K2, 12208, M2) <= F.NOALLOC_SCRATCH_BYTES
    dw2 = F.DeviceBuffer(N2 * (K2 // 256) * 144)
    dx2 = F.DeviceBuffer(M2 * K2 * 4)
    dy2 = F.DeviceBuffer(M2 * N2 * 4)
    with pytest.raises(F.Fh3Error) as ei:
        F.matmul_noalloc_dev(dw2, K2, N2, dx2, dy2, M2)
    assert ei.value.code == F.FH3_E_INVALID and "scratch" in str(ei.value)
    with pytest.raises(F.Fh3Error) as ei:          # Q4_K only
        F.matmul_noalloc_dev(dw, 256, 16, dx, dy, 4, qtype=F.FH3_QUANT_Q6_K)
    assert ei.value.code == F.FH3_E_INVALID


def test_noalloc_captures_first_time(gpu):
    """A shape this process never ran: fh3_hip_matmul_dev would refuse its
    first capture (its workspace must grow); the no-allocation call captures
    at once, and every replay equals the eager result."""
    F = gpu
    K, N, M = 7168, 5376, 40
    dw, dx, db = _pair(F, K, N, M, 99)
    dy = F.DeviceBuffer(M * N * 4)
    g = F.capture(lambda: F.matmul_noalloc_dev(dw, K, N, dx, dy, M, db))
    try:
        ref_b = F.DeviceBuffer(M * N * 4)
        F.matmul_noalloc_dev(dw, K, N, dx, ref_b, M, db)
        F.synchronize()
        ref = ref_b.download(np.float32, (M, N))
        for rep in range(3):
            dy.fill(0)
            F.synchronize()
            g.launch()
            F.synchronize()
            assert np.array_equal(_bits(dy.download(np.float32, (M, N))), _bits(ref)), rep
    finally:
        g.close()
