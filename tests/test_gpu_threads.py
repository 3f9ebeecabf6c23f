"""Calls from several host threads at once.  The host-pointer fh3_matmul
(fh3's signature, src/core/fh3_ops.c:317) runs on the library's compute
stream under the library's lock, and fh3_hip_matmul_dev on that stream
(stream NULL) enqueues its preparation and product in stream order, so
concurrent callers share the library's workspace safely.  Four threads (ctypes
releases the GIL during each call) each run a mix of shapes covering every
kernel family; every result must equal, bit for bit, the same call made alone.
"""
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SHAPES = [(1, 2048, 96), (4, 2048, 130), (16, 5120, 64), (40, 5120, 48), (70, 1024, 200), (300, 512, 64)]


def _inputs(F, i, M, K, N):
    raw = F.synth_q4k_weights(500 + i, 1, N, K, 0.02, 0.0)
    x = F.synth_x("normal", 500 + i, 2, M, K)
    bias = F.rng_normal(500 + i, 3, N)
    return raw, x, bias


def _run_threads(work, n_threads=4):
    errors = []

    def body(t):
        try:
            work(t)
        except BaseException as e:  # surfaced below
            errors.append(e)

    ts = [threading.Thread(target=body, args=(t,)) for t in range(n_threads)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in ts), "a thread did not finish"
    if errors:
        raise errors[0]


def test_host_matmul_from_threads(gpu):
    F = gpu
    print("case: host fh3_matmul from 4 threads, %d shapes" % len(SHAPES), flush=True)
    cases = [_inputs(F, i, *s) for i, s in enumerate(SHAPES)]
    alone = [F.matmul(raw, K, N, x, bias) for (raw, x, bias), (M, K, N) in zip(cases, SHAPES)]
    got = {}

    def work(t):
        for r in range(3):
            for j in range(len(SHAPES)):
                i = (j + t + r) % len(SHAPES)
                (raw, x, bias), (M, K, N) = cases[i], SHAPES[i]
                got.setdefault((t, r, i), F.matmul(raw, K, N, x, bias))

    _run_threads(work)
    assert len(got) == 4 * 3 * len(SHAPES)
    for (t, r, i), y in got.items():
        assert np.array_equal(y.view(np.uint32), alone[i].view(np.uint32)), (t, r, SHAPES[i])


def test_device_matmul_on_library_stream_from_threads(gpu):
    F = gpu
    print("case: fh3_hip_matmul_dev (stream NULL) from 4 threads, %d shapes" % len(SHAPES), flush=True)
    cases = []
    for i, (M, K, N) in enumerate(SHAPES):
        raw, x, bias = _inputs(F, i, M, K, N)
        cases.append((F.DeviceBuffer.from_array(raw), F.DeviceBuffer.from_array(x), F.DeviceBuffer.from_array(bias)))
    alone = []
    for (dw, dx, db), (M, K, N) in zip(cases, SHAPES):
        dy = F.DeviceBuffer(M * N * 4)
        F.matmul_dev(dw, K, N, dx, dy, M, db)
        F.synchronize()
        alone.append(dy.download(np.float32, (M, N)))
        dy.close()
    # one output buffer per (thread, shape): calls of different threads interleave on the stream
    outs = {(t, i): F.DeviceBuffer(M * N * 4) for t in range(4) for i, (M, K, N) in enumerate(SHAPES)}

    def work(t):
        for r in range(3):
            for j in range(len(SHAPES)):
                i = (j + 2 * t + r) % len(SHAPES)
                (dw, dx, db), (M, K, N) = cases[i], SHAPES[i]
                F.matmul_dev(dw, K, N, dx, outs[(t, i)], M, db)

    _run_threads(work)
    F.synchronize()
    for (t, i), dy in outs.items():
        M, K, N = SHAPES[i]
        y = dy.download(np.float32, (M, N))
        assert np.array_equal(y.view(np.uint32), alone[i].view(np.uint32)), (t, SHAPES[i])
        dy.close()
    for bufs in cases:
        for b in bufs:
            b.close()
