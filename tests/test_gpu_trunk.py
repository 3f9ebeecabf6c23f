"""Device side of the layer streamer: the HBM-resident prefix and the two device
slots fed by hipMemcpyAsync from page-locked host memory.

Byte checks follow the reference's trunk tests (tests/unit/test_trunk.c:133-357)
with the device copy read back; the pipeline tests enqueue the matmuls of every
layer without host synchronisation between layers, so the upload/compute
ordering is what keeps each layer's bytes intact, and compare the outputs
bitwise with the same calls on weights held in plain device buffers (the
reference asks streamed and pinned runs to agree bitwise,
tests/unit/test_dit_tiny.c:297-298) and with the oracle.
"""
import ctypes

import numpy as np
import pytest

import helpers

pytestmark = pytest.mark.gpu

MB = 1 << 20


def acquired(fh3, tr, L):
    d = tr.acquire_dev(L)
    assert d is not None, "layer %d: %s" % (L, fh3.lib().fh3_hip_last_error().decode())
    return d


def read_back(fh3, addr, n):
    out = np.empty(n, dtype=np.uint8)
    fh3._check(fh3.lib().fh3_hip_memcpy_dtoh(out.ctypes.data, addr, n), "fh3_hip_memcpy_dtoh")
    return out


def test_dev_stream_pattern_bytes(gpu, tmp_path):
    fh3 = gpu
    path = helpers.write_pattern_pack(str(tmp_path / "p.bin"), [MB] * 10)
    print("case: pattern pack 10 x 1 MB, host budget 8 MB, device budget 5 MB", flush=True)
    with fh3.Trunk(path, 8 * MB) as tr:
        tr.attach_device(5 * MB)
        inf = tr.info()
        assert (inf.npin, inf.dpin, inf.dev_slot_size) == (6, 3, MB)
        for scan in range(3):
            for L in range(10):
                d = acquired(fh3, tr, L)
                if scan < 2:
                    tr.prefetch_dev((L + 1) % 10)
                b = read_back(fh3, d, MB)
                assert np.all(b == 0xA0 + L), (scan, L)
        ds, hs = tr.dev_stats(), tr.stats()
        assert (ds.hits, ds.misses) == (9, 21)
        assert ds.uploads == 21 and ds.bytes_uploaded == 21 * MB
        assert ds.resident_bytes == 3 * MB
        # host reads: layers 6..9 come from disk through the host ring each pass
        assert (hs.misses, hs.bytes_read) == (12, 12 * MB)


def test_dev_slot_pointer_identity(gpu, tmp_path):
    """Two device slots behave as the host ring does: A, prefetch B, A again is
    a hit on the same slot, then B lands in the other one, and A/B alternate
    without uploads."""
    fh3 = gpu
    path = helpers.write_pattern_pack(str(tmp_path / "p.bin"), [MB] * 10)
    with fh3.Trunk(path, 8 * MB) as tr:
        tr.attach_device(2 * MB)
        assert tr.info().dpin == 0
        a1 = acquired(fh3, tr, 7)
        tr.prefetch_dev(8)
        assert tr.acquire_dev(7) == a1
        b1 = acquired(fh3, tr, 8)
        assert b1 != a1
        for L, want in [(7, a1), (8, b1), (7, a1), (8, b1)]:
            assert tr.acquire_dev(L) == want
        ds = tr.dev_stats()
        assert (ds.uploads, ds.misses, ds.hits) == (2, 2, 5)
        assert np.all(read_back(fh3, a1, MB) == 0xA0 + 7) and np.all(read_back(fh3, b1, MB) == 0xA0 + 8)
        with pytest.raises(fh3.Fh3Error):
            tr.attach_device(2 * MB)


def test_dev_short_read_returns_null(gpu, tmp_path):
    fh3 = gpu
    path = helpers.write_pattern_pack(str(tmp_path / "cut.bin"), [MB] * 10, truncate_last=4096)
    with fh3.Trunk(path, 4 * MB) as tr:
        tr.attach_device(2 * MB)
        assert tr.acquire_dev(9) is None
        assert "layer 9" in fh3.lib().fh3_hip_last_error().decode()
        d = acquired(fh3, tr, 8)
        assert np.all(read_back(fh3, d, MB) == 0xA0 + 8)


@pytest.mark.parametrize("what", [1, 2])
def test_dev_upload_failure_returns_null_then_recovers(gpu, tmp_path, what):
    """A HIP error in a slot upload (its copy, or the event that orders it
    behind the compute; injected from the host) makes fh3_trunk_acquire_dev
    return NULL with the error text, as a failed read does in the reference
    (src/io/fh3_trunk.c:453-456,487-490 -> FH3_ERR in src/model/fh3_dit.c:361-368);
    the next acquire of the same layer uploads again and returns its bytes.
    Layers from disk through the host ring and from page-locked host memory."""
    fh3 = gpu
    path = helpers.write_pattern_pack(str(tmp_path / "p.bin"), [MB] * 10)
    with fh3.Trunk(path, 8 * MB) as tr:        # layers 0..5 in host memory, 6..9 from disk
        tr.attach_device(2 * MB)               # every layer streams through the two slots
        for L in (3, 7):
            print("case: injected failure %d at layer %d" % (what, L), flush=True)
            tr.inject_upload_failure(what)
            assert tr.acquire_dev(L) is None
            assert "injected failure" in fh3.lib().fh3_hip_last_error().decode()
            d = acquired(fh3, tr, L)
            assert np.all(read_back(fh3, d, MB) == 0xA0 + L)
        # a failure inside prefetch_dev leaves nothing half done: the acquire uploads again
        tr.inject_upload_failure(1)
        tr.prefetch_dev(4)
        d = acquired(fh3, tr, 4)
        assert np.all(read_back(fh3, d, MB) == 0xA0 + 4)
        for L in range(10):
            d = acquired(fh3, tr, L)
            tr.prefetch_dev((L + 1) % 10)
            assert np.all(read_back(fh3, d, MB) == 0xA0 + L)


# ---------------------------------------------------------------------------
# streamed matmuls
# ---------------------------------------------------------------------------
HIDDEN, QKV, MLP = 512, 768, 1024
N_LAYERS = 6


@pytest.fixture(scope="module")
def dit_pack(tmp_path_factory):
    from fasth3inc_amd import pack as P
    specs = P.dit_block_specs(hidden=HIDDEN, qkv_out=QKV, mlp_hidden=MLP)
    layers = [P.synth_dit_block(specs, seed=11, L=L) for L in range(N_LAYERS)]
    path = str(tmp_path_factory.mktemp("dit") / "dit.bin")
    P.write_pack(path, N_LAYERS, specs, lambda L: layers[L])
    return path, specs, layers


def _tokens(L):
    return 8 if L % 2 == 0 else 300  # small-M and GEMM paths alternate


def _run_layers(fh3, get_w, xs, outs, prefetch=None):
    """Enqueue, per layer: qkv = x1 W_qkv^T, fc2 = x2 W_fc2^T, deq = dequant(W_out);
    no synchronisation until the end."""
    for L in range(N_LAYERS):
        v = get_w(L)
        if prefetch:
            prefetch(L + 1)
        M = _tokens(L)
        x1, x2 = xs[L]
        y1, y2, dq = outs[L]
        fh3.matmul_dev(v.qkv.data, v.qkv.in_, v.qkv.out, x1, y1, M)
        fh3.matmul_dev(v.fc2.data, v.fc2.in_, v.fc2.out, x2, y2, M)
        fh3.dequant_dev(v.out.data, dq, v.out.out, v.out.in_)
    fh3.synchronize()
    return [(y1.download(np.float32, (_tokens(L), QKV)), y2.download(np.float32, (_tokens(L), HIDDEN)),
             dq.download(np.float32, (HIDDEN, HIDDEN))) for L, (y1, y2, dq) in enumerate(outs)]


def _buffers(fh3):
    xs, outs, host_x = [], [], []
    for L in range(N_LAYERS):
        M = _tokens(L)
        a = fh3.synth_x("normal", 5, 2 * L, M, HIDDEN)
        b = fh3.synth_x("silu_gated", 5, 2 * L + 1, M, MLP)
        host_x.append((a, b))
        xs.append((fh3.DeviceBuffer.from_array(a), fh3.DeviceBuffer.from_array(b)))
        outs.append((fh3.DeviceBuffer(M * QKV * 4), fh3.DeviceBuffer(M * HIDDEN * 4),
                     fh3.DeviceBuffer(HIDDEN * HIDDEN * 4)))
    return xs, outs, host_x


@pytest.mark.parametrize("host_budget,dev_budget,name", [
    (1 << 40, 0, "host-resident, all layers through 2 device slots"),
    (0, 0, "disk through the host ring, then 2 device slots"),
    (0, 5 * MB, "device-resident prefix of 2 layers, disk for the rest"),
    (1 << 40, 1 << 40, "everything resident in HBM"),
])
def test_streamed_matmul_matches_resident(gpu, oracle, dit_pack, host_budget, dev_budget, name):
    fh3 = gpu
    path, specs, layers = dit_pack
    print("case:", name, flush=True)
    xs, outs, host_x = _buffers(fh3)

    # weights in plain device buffers
    resident = [[fh3.DeviceBuffer.from_array(a) for a in blk] for blk in layers]
    with fh3.Pack(path) as p:
        views = [p.layer(L, None) for L in range(N_LAYERS)]

    def resident_view(L):
        v = fh3.Fh3LayerView()
        for t, n in enumerate(fh3.LAYER_TENSORS):
            w = getattr(views[L], n)
            setattr(v, n, fh3.Fh3W(w.type, w.in_, w.out, resident[L][t].ptr))
        return v

    want = _run_layers(fh3, resident_view, xs, outs)
    for o in outs:
        for b in o:
            b.fill(0xFF)

    with fh3.Trunk(path, host_budget) as tr:
        tr.attach_device(dev_budget)

        def streamed_view(L):
            return tr.layer(L, acquired(fh3, tr, L))

        got = _run_layers(fh3, streamed_view, xs, outs,
                          prefetch=lambda L: tr.prefetch_dev(L) if L < N_LAYERS else None)
        ds = tr.dev_stats()
        dpin = tr.info().dpin
        assert ds.hits + ds.misses == N_LAYERS
        assert ds.uploads == N_LAYERS - dpin

    for L in range(N_LAYERS):
        for g, w in zip(got[L], want[L]):
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (name, L)
    # and the outputs are right: dequant bit-exact, products within the GPU bound
    for L in range(N_LAYERS):
        blk = layers[L]
        deq = helpers.oracle_dequant(oracle, blk[2], HIDDEN, HIDDEN)
        assert np.array_equal(got[L][2].view(np.uint32), deq.view(np.uint32))
        x1, x2 = host_x[L]
        assert helpers.rel_fro(got[L][0], helpers.oracle_matmul(oracle, blk[0], HIDDEN, QKV, x1)) <= 2e-3
        assert helpers.rel_fro(got[L][1], helpers.oracle_matmul(oracle, blk[4], MLP, HIDDEN, x2)) <= 2e-3
