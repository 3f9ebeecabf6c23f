"""The library workspace under HIP graph capture (fh3_hip.h: graph capture and
fh3_hip_matmul_workspace_bytes), through the C-ABI.

A product whose split-K partial sums (or prepared activations) would have to
be allocated cannot be captured the first time: the call returns
FH3_E_INVALID and enqueues nothing.  Run once eagerly, the same call captures,
and its graph keeps replaying correctly after a later eager call has grown the
workspace (the replaced buffer stays allocated while graphs exist).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.fixture
def fresh(gpu):
    """The library with no workspace allocated yet (shutdown frees it)."""
    F = gpu
    F.synchronize()
    F.shutdown()
    F.init(0)
    yield F
    F.synchronize()


def _weights(F, K, N, seed):
    return F.DeviceBuffer.from_array(F.synth_q4k_weights(seed, 1, N, K, 0.02, 0.0))


def test_first_capture_refused_then_replays_across_growth(fresh):
    F = fresh
    K, N = 5120, 5120
    M, M_big = 128, 512
    print("case: prepared split-K GEMM M=%d then M=%d, K=N=%d" % (M, M_big, K), flush=True)
    assert F.matmul_path(M, K) == F.PATH_GEMM
    pb = F.matmul_workspace_bytes(K, N, M, prepared=True)
    pb_big = F.matmul_workspace_bytes(K, N, M_big, prepared=True)
    assert 0 < pb < pb_big, (pb, pb_big)
    dw = _weights(F, K, N, 7)
    x = F.synth_x("normal", 7, 1, M_big, K)
    dx = F.DeviceBuffer.from_array(x)
    prep = F.DeviceBuffer(F.prepared_bytes(M_big, K))
    prep_s = F.DeviceBuffer(F.prepared_bytes(M, K))
    F.prepare_x_dev(dx, M, K, prep_s)
    F.prepare_x_dev(dx, M_big, K, prep)
    dy = F.DeviceBuffer(M * N * 4)
    dy_big = F.DeviceBuffer(M_big * N * 4)
    F.synchronize()

    # 1. first time under capture: refused, nothing enqueued, stream usable
    with pytest.raises(F.Fh3Error) as ei:
        F.capture(lambda: F.matmul_prepared_dev(dw, K, N, prep_s, dy, M))
    assert ei.value.code == F.FH3_E_INVALID
    assert "eagerly" in str(ei.value)

    # 2. eager, then capture succeeds and replays the eager result
    dy.fill(0)
    F.matmul_prepared_dev(dw, K, N, prep_s, dy, M)
    F.synchronize()
    want = dy.download(np.float32, (M, N))
    assert np.isfinite(want).all()
    g = F.capture(lambda: F.matmul_prepared_dev(dw, K, N, prep_s, dy, M))
    try:
        for rep in range(3):
            dy.fill(0)
            if rep == 1:
                # 3. a larger eager call grows the partial-sum workspace while the graph exists
                # (its K windows differ from the 128-token call's, so its rows
                # agree with `want` to rounding, not bit for bit)
                F.matmul_prepared_dev(dw, K, N, prep, dy_big, M_big)
                F.synchronize()
                big = dy_big.download(np.float32, (M_big, N))
                assert np.abs(big[:M] - want).max() <= 1e-4 * np.abs(want).max()
            g.launch()
            F.synchronize()
            assert np.array_equal(_bits(dy.download(np.float32, (M, N))), _bits(want)), rep
    finally:
        g.close()
    # after the last graph is gone the library still works (retired buffers freed)
    dy.fill(0)
    F.matmul_prepared_dev(dw, K, N, prep_s, dy, M)
    F.synchronize()
    assert np.array_equal(_bits(dy.download(np.float32, (M, N))), _bits(want))


def test_first_capture_of_unprepared_product_refused(fresh):
    """fh3_hip_matmul_dev prepares its activations in library workspace: the
    first capture of a small-M call is refused too, and succeeds after an
    eager run."""
    F = fresh
    K, N, M = 4096, 1024, 8
    assert F.matmul_path(M, K) == F.PATH_SWEEP
    assert F.matmul_workspace_bytes(K, N, M) == F.prepared_bytes(M, K)
    assert F.matmul_workspace_bytes(K, N, M, prepared=True) == 0
    assert F.matmul_workspace_bytes(K, N, 1) == 0          # k_gemv8 quantises in the kernel
    dw = _weights(F, K, N, 8)
    dx = F.DeviceBuffer.from_array(F.synth_x("normal", 8, 1, M, K))
    dy = F.DeviceBuffer(M * N * 4)
    with pytest.raises(F.Fh3Error) as ei:
        F.capture(lambda: F.matmul_dev(dw, K, N, dx, dy, M))
    assert ei.value.code == F.FH3_E_INVALID
    F.matmul_dev(dw, K, N, dx, dy, M)
    F.synchronize()
    want = dy.download(np.float32, (M, N))
    g = F.capture(lambda: F.matmul_dev(dw, K, N, dx, dy, M))
    try:
        for rep in range(3):
            dy.fill(0)
            F.synchronize()
            g.launch()
            F.synchronize()
            assert np.array_equal(_bits(dy.download(np.float32, (M, N))), _bits(want)), rep
    finally:
        g.close()


def test_free_inside_capture_is_deferred(gpu):
    """fh3_hip_free on the capturing thread between fh3_hip_graph_begin and
    fh3_hip_graph_end (here an explicit close; in Python also a collected
    DeviceBuffer) is carried out at fh3_hip_graph_end: the capture survives,
    and every replay equals the eager products."""
    F = gpu
    K, N, M = 2048, 640, 24
    print("case: free inside a capture, M=%d K=%d N=%d" % (M, K, N), flush=True)
    dw = _weights(F, K, N, 11)
    dx = F.DeviceBuffer.from_array(F.synth_x("normal", 11, 1, M, K))
    want = F.DeviceBuffer(M * N * 4)
    F.matmul_dev(dw, K, N, dx, want, M)          # eager first: the workspace exists
    F.synchronize()
    ref = want.download(np.float32, (M, N))
    dy, dy2 = F.DeviceBuffer(M * N * 4), F.DeviceBuffer(M * N * 4)
    spare = F.DeviceBuffer(1 << 20)

    def body():
        F.matmul_dev(dw, K, N, dx, dy, M)
        spare.close()
        F.matmul_dev(dw, K, N, dx, dy2, M)

    g = F.capture(body)
    try:
        for rep in range(3):
            dy.fill(0)
            dy2.fill(0)
            F.synchronize()
            g.launch()
            F.synchronize()
            assert np.array_equal(_bits(dy.download(np.float32, (M, N))), _bits(ref)), rep
            assert np.array_equal(_bits(dy2.download(np.float32, (M, N))), _bits(ref)), rep
    finally:
        g.close()
    for b in (dw, dx, want, dy, dy2):
        b.close()
