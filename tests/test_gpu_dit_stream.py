"""DiT blocks of the benchmark's streamed workload at full size, through the
layer streamer's device slots (fh3_trunk_attach_device / prefetch_dev /
acquire_dev), M = 16384 tokens.

Three blocks at the DiT attention/MLP shapes (qkv 5120 -> 15360, out
5120 -> 5120, fc1 = up|gate 5120 -> 27648, fc2 = down 13824 -> 5120; 178.4 MB
of Q4_K per block) are written to an FH3P pack.  Every block's products are
enqueued without host synchronisation between blocks, so the upload of block
L+1 into the idle device slot overlaps block L's kernels and the slot events
alone keep each block's bytes intact.

Checks (the reference asks streamed and pinned runs to agree bit for bit,
tests/unit/test_dit_tiny.c:230-299):
  - every product output of the streamed run equals, bit for bit, the same
    products on the blocks held resident in device buffers, for blocks read
    from disk through the host ring and for blocks held in page-locked host
    memory;
  - 64 seeded token rows of every product against the oracle (rows depend
    only on their own activation row), rel-Frobenius <= 2e-3;
  - the block's fused sequence (norm1+modulate prep -> qkv; out projection
    with the gate residual into h; norm2+modulate prep -> fc1 with SwiGLU ->
    fc2 with the gate residual; the attention output standing in for its
    input, src/model/fh3_dit.c:383-439) streamed over the three blocks: final
    h and every qkv output bit for bit against the resident run, and against
    the oracle's CPU sequence on 64 token rows.
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3
HIDDEN, QKV, MLP = 5120, 15360, 13824
M = 16384
N_BLOCKS = 3
EPS = 1e-6
CHUNK = 256 << 20


@pytest.fixture(scope="module")
def blocks(tmp_path_factory):
    from fasth3inc_amd import pack as P
    specs = P.dit_block_specs(hidden=HIDDEN, qkv_out=QKV, mlp_hidden=MLP)
    path = str(tmp_path_factory.mktemp("dit5") / "dit.fh3p")
    P.write_pack(path, N_BLOCKS, specs, lambda L: P.synth_dit_block(specs, 21, L))
    return path, specs


@pytest.fixture(scope="module")
def acts(fh3):
    """Host and device activations: xa (attention-side input, 1% outliers),
    xm (down-projection input, SiLU-gated), h (residual stream), shift,
    scale and gate rows."""
    F = fh3
    host = {"xa": F.synth_x("outliers", 21, 1, M, HIDDEN), "xm": F.synth_x("silu_gated", 21, 2, M, MLP),
            "h": F.synth_x("normal", 21, 3, M, HIDDEN)}
    for i, k in enumerate(("shift", "scale", "gate")):
        host[k] = (0.1 * F.synth_x("normal", 21, 10 + i, M, HIDDEN)).astype(np.float32)
    return host


def _tokens(seed):
    rng = np.random.default_rng(seed)
    pick = set(int(t) for t in rng.choice(M, 58, replace=False)) | {0, 255, 256, M // 2, M - 256, M - 1}
    return np.array(sorted(pick))


def _equal_on_device(F, a, b, nbytes):
    """Two device buffers hold the same bytes (compared chunk by chunk on the host)."""
    ha = np.empty(min(CHUNK, nbytes), np.uint8)
    hb = np.empty_like(ha)
    for off in range(0, nbytes, CHUNK):
        n = min(CHUNK, nbytes - off)
        F._check(F.lib().fh3_hip_memcpy_dtoh(ha.ctypes.data, a + off, n), "dtoh")
        F._check(F.lib().fh3_hip_memcpy_dtoh(hb.ctypes.data, b + off, n), "dtoh")
        if not np.array_equal(ha[:n], hb[:n]):
            return False
    return True


def _rows(F, buf, N, rows):
    out = np.empty((len(rows), N), np.float32)
    for i, t in enumerate(rows):
        F._check(F.lib().fh3_hip_memcpy_dtoh(out[i].ctypes.data, buf.ptr + int(t) * N * 4, N * 4), "dtoh")
    return out


def _resident_views(F, path, specs):
    from fasth3inc_amd import pack as P
    bufs = [[F.DeviceBuffer.from_array(a) for a in P.synth_dit_block(specs, 21, L)] for L in range(N_BLOCKS)]
    with F.Pack(path) as p:
        views = [p.layer(L, None) for L in range(N_BLOCKS)]
    out = []
    for L in range(N_BLOCKS):
        v = F.Fh3LayerView()
        for t, n in enumerate(F.LAYER_TENSORS):
            w = getattr(views[L], n)
            setattr(v, n, F.Fh3W(w.type, w.in_, w.out, bufs[L][t].ptr))
        out.append(v)
    return out, bufs


def _streamed(F, tr, L):
    d = tr.acquire_dev(L)
    assert d is not None, "block %d: %s" % (L, F.lib().fh3_hip_last_error().decode())
    if L + 1 < N_BLOCKS:
        tr.prefetch_dev(L + 1)
    return tr.layer(L, d)


PRODUCTS = (("qkv", HIDDEN, QKV, "xa"), ("out", HIDDEN, HIDDEN, "xa"), ("fc1", HIDDEN, 2 * MLP, "xa"),
            ("fc2", MLP, HIDDEN, "xm"))


def test_streamed_dit_blocks_m16384_products(gpu, oracle, blocks, acts):
    F = gpu
    path, specs = blocks
    dx = {k: F.DeviceBuffer.from_array(acts[k]) for k in ("xa", "xm")}

    def run(get_view):
        outs = []
        for L in range(N_BLOCKS):
            v = get_view(L)
            ys = []
            for name, K, N, xk in PRODUCTS:
                w = getattr(v, name)
                assert (w.in_, w.out) == (K, N)
                y = F.DeviceBuffer(M * N * 4)
                F.matmul_dev(w.data, K, N, dx[xk], y, M)
                ys.append(y)
            outs.append(ys)
        F.synchronize()
        return outs

    print("case: DiT blocks resident, %d blocks M=%d" % (N_BLOCKS, M), flush=True)
    views, wbufs = _resident_views(F, path, specs)
    want = run(lambda L: views[L])
    for host_budget, label in ((0, "disk -> host ring -> 2 device slots"),
                               (1 << 40, "page-locked host blocks -> 2 device slots")):
        print("case: DiT blocks streamed (%s)" % label, flush=True)
        with F.Trunk(path, host_budget) as tr:
            tr.attach_device(0)
            assert tr.info().dpin == 0
            got = run(lambda L: _streamed(F, tr, L))
            ds = tr.dev_stats()
            assert ds.uploads == N_BLOCKS and ds.misses == N_BLOCKS
        for L in range(N_BLOCKS):
            for (name, K, N, _), g, w in zip(PRODUCTS, got[L], want[L]):
                assert _equal_on_device(F, g.ptr, w.ptr, M * N * 4), (label, L, name)
        for ys in got:
            for b in ys:
                b.close()
    # the products themselves, on sampled token rows
    from fasth3inc_amd import pack as P
    for L in range(N_BLOCKS):
        raws = dict(zip(F.LAYER_TENSORS, P.synth_dit_block(specs, 21, L)))
        sub = _tokens(100 + L)
        for (name, K, N, xk), y in zip(PRODUCTS, want[L]):
            yo = H.oracle_matmul(oracle, raws[name], K, N, acts[xk][sub])
            err = H.rel_fro(_rows(F, y, N, sub), yo)
            print("  block %d %s: rel_fro %.3e over %d rows" % (L, name, err, len(sub)), flush=True)
            assert err <= TOL, (L, name, err)
    for ys in want:
        for b in ys:
            b.close()
    for b in list(dx.values()) + [b for bl in wbufs for b in bl]:
        b.close()


def test_streamed_dit_blocks_m16384_fused_block(gpu, oracle, blocks, acts):
    F = gpu
    path, specs = blocks
    d = {k: F.DeviceBuffer.from_array(acts[k]) for k in ("xa", "shift", "scale", "gate")}
    prep = F.DeviceBuffer(F.prepared_bytes(M, HIDDEN))
    act = F.DeviceBuffer(M * MLP * 4)

    def run(get_view):
        h = F.DeviceBuffer.from_array(acts["h"])
        qkvs = []
        for L in range(N_BLOCKS):
            v = get_view(L)
            qkv = F.DeviceBuffer(M * QKV * 4)
            F.prepare_x_norm_dev(h, M, HIDDEN, v.norm1.data, EPS, prep, d["shift"], d["scale"])
            F.matmul_prepared_dev(v.qkv.data, HIDDEN, QKV, prep, qkv, M)
            F.matmul_epi_dev(v.out.data, HIDDEN, HIDDEN, d["xa"], M, F.EPI_GATE_RESIDUAL, h, d["gate"])
            F.prepare_x_norm_dev(h, M, HIDDEN, v.norm2.data, EPS, prep, d["shift"], d["scale"])
            F.matmul_prepared_epi_dev(v.fc1.data, HIDDEN, 2 * MLP, prep, M, F.EPI_SWIGLU, act)
            F.matmul_epi_dev(v.fc2.data, MLP, HIDDEN, act, M, F.EPI_GATE_RESIDUAL, h, d["gate"])
            qkvs.append(qkv)
        F.synchronize()
        return h, qkvs

    print("case: DiT fused block sequence, resident", flush=True)
    views, wbufs = _resident_views(F, path, specs)
    h_want, q_want = run(lambda L: views[L])
    print("case: DiT fused block sequence, streamed through 2 device slots", flush=True)
    with F.Trunk(path, 1 << 40) as tr:
        tr.attach_device(0)
        h_got, q_got = run(lambda L: _streamed(F, tr, L))
    assert _equal_on_device(F, h_got.ptr, h_want.ptr, M * HIDDEN * 4)
    for L in range(N_BLOCKS):
        assert _equal_on_device(F, q_got[L].ptr, q_want[L].ptr, M * QKV * 4), L

    # the oracle's CPU sequence on sampled tokens (each row evolves alone)
    from fasth3inc_amd import pack as P
    sub = _tokens(7)
    r = acts["h"][sub].copy()
    sh, sc, gt, xa = (acts[k][sub] for k in ("shift", "scale", "gate", "xa"))
    n = len(sub)
    for L in range(N_BLOCKS):
        raws = dict(zip(F.LAYER_TENSORS, P.synth_dit_block(specs, 21, L)))
        xn = r.copy()
        H.elementwise(oracle, "fh3_oracle_", "rmsnorm", xn, raws["norm1"].view(np.float32), n, HIDDEN, EPS)
        H.elementwise(oracle, "fh3_oracle_", "modulate", xn, sh, sc, n, HIDDEN)
        qkv = H.oracle_matmul(oracle, raws["qkv"], HIDDEN, QKV, xn)
        err = H.rel_fro(_rows(F, q_want[L], QKV, sub), qkv)
        print("  block %d qkv (fused prep): rel_fro %.3e" % (L, err), flush=True)
        assert err <= TOL, (L, err)
        y = H.oracle_matmul(oracle, raws["out"], HIDDEN, HIDDEN, xa)
        H.elementwise(oracle, "fh3_oracle_", "gate_residual", r, gt, y, n, HIDDEN)
        xn = r.copy()
        H.elementwise(oracle, "fh3_oracle_", "rmsnorm", xn, raws["norm2"].view(np.float32), n, HIDDEN, EPS)
        H.elementwise(oracle, "fh3_oracle_", "modulate", xn, sh, sc, n, HIDDEN)
        y1 = H.oracle_matmul(oracle, raws["fc1"], HIDDEN, 2 * MLP, xn)
        a = np.zeros((n, MLP), np.float32)
        H.elementwise(oracle, "fh3_oracle_", "swiglu", y1, a, n, MLP)
        y2 = H.oracle_matmul(oracle, raws["fc2"], MLP, HIDDEN, a)
        H.elementwise(oracle, "fh3_oracle_", "gate_residual", r, gt, y2, n, HIDDEN)
    h0 = acts["h"][sub]
    got = _rows(F, h_want, HIDDEN, sub)
    err = H.rel_fro(got - h0, r - h0)
    print("  final h after %d fused blocks: rel_fro of the update %.3e" % (N_BLOCKS, err), flush=True)
    assert err <= TOL
    for b in [h_got, h_want, prep, act] + q_got + q_want + list(d.values()) + [b for bl in wbufs for b in bl]:
        b.close()


# ---------------------------------------------------------------------------
# The real model's block (src/cli/fh3_cli.c:935-941): hidden 5376, inner 7168,
# qkv 21504, gate_compress 7168 (Q4_K), fc1 28672, fc2 14336 -> 5376:
# 238,480,384 bytes of Q4_K per block (docs/data/census.json:17), at the CLI's
# default sequence of 3016 tokens (6 text, 130 audio, 2880 video).
# ---------------------------------------------------------------------------
RM = 3016


@pytest.fixture(scope="module")
def real_blocks(tmp_path_factory):
    from fasth3inc_amd import pack as P
    specs = P.real_dit_block_specs()
    path = str(tmp_path_factory.mktemp("dit_real") / "dit_real.fh3p")
    P.write_pack(path, N_BLOCKS, specs, lambda L: P.synth_dit_block(specs, 23, L))
    return path, specs


def test_streamed_real_dit_blocks_m3016(gpu, oracle, real_blocks):
    """Three real-size blocks (the five Q4_K products, gate_compress
    included) streamed from disk through the host ring and from page-locked
    host memory through the two device slots: every output bit for bit
    equal to the resident run, and sampled token rows against the oracle."""
    F = gpu
    from fasth3inc_amd import pack as P
    path, specs = real_blocks
    q4 = [s for s in specs if s.qtype == F.FH3_QUANT_Q4_K]
    # the census's per-block bytes: 238,436,352 of Q4_K plus 44,032 of fp32 norm weights
    assert sum(s.nbytes for s in specs) == 238480384 and sum(s.nbytes for s in q4) == 238436352
    ins = sorted({s.ne0 for s in q4})
    host_x = {K: F.synth_x("outliers" if K == 5376 else "silu_gated" if K == 14336 else "normal", 23, K, RM, K)
              for K in ins}
    dx = {K: F.DeviceBuffer.from_array(v) for K, v in host_x.items()}
    names = ["qkv", "gate_compress", "out", "fc1", "fc2"]

    def run(get_view):
        outs = []
        for L in range(N_BLOCKS):
            v = get_view(L)
            ys = []
            for name in names:
                w = getattr(v, name)
                y = F.DeviceBuffer(RM * w.out * 4)
                F.matmul_dev(w.data, w.in_, w.out, dx[w.in_], y, RM)
                ys.append((y, w.out))
            outs.append(ys)
        F.synchronize()
        return outs

    print("case: real DiT blocks resident, %d blocks M=%d" % (N_BLOCKS, RM), flush=True)
    bufs = [[F.DeviceBuffer.from_array(a) for a in P.synth_dit_block(specs, 23, L)] for L in range(N_BLOCKS)]
    with F.Pack(path) as p:
        pviews = [p.layer(L, None) for L in range(N_BLOCKS)]
    views = []
    for L in range(N_BLOCKS):
        v = F.Fh3LayerView()
        for t, n in enumerate(F.LAYER_TENSORS):
            w = getattr(pviews[L], n)
            setattr(v, n, F.Fh3W(w.type, w.in_, w.out, bufs[L][t].ptr))
        views.append(v)
    want = run(lambda L: views[L])
    for host_budget, label in ((0, "disk -> host ring -> 2 device slots"),
                               (1 << 40, "page-locked host blocks -> 2 device slots")):
        print("case: real DiT blocks streamed (%s)" % label, flush=True)
        with F.Trunk(path, host_budget) as tr:
            tr.attach_device(0)
            assert tr.info().dpin == 0 and tr.info().dev_slot_size >= 238480384
            got = run(lambda L: _streamed(F, tr, L))
            ds = tr.dev_stats()
            assert ds.uploads == N_BLOCKS and ds.misses == N_BLOCKS
        for L in range(N_BLOCKS):
            for name, (g, N), (w, _) in zip(names, got[L], want[L]):
                assert _equal_on_device(F, g.ptr, w.ptr, RM * N * 4), (label, L, name)
        for ys in got:
            for b, _ in ys:
                b.close()
    rng = np.random.default_rng(3016)
    sub = np.unique(np.concatenate([[0, 5, 6, 135, 136, RM - 1], rng.choice(RM, 26, replace=False)]))
    for L in range(N_BLOCKS):
        raws = dict(zip(F.LAYER_TENSORS, P.synth_dit_block(specs, 23, L)))
        for name, (y, N) in zip(names, want[L]):
            w = getattr(views[L], name)
            yo = H.oracle_matmul(oracle, raws[name], w.in_, N, host_x[w.in_][sub])
            err = H.rel_fro(_rows(F, y, N, sub), yo)
            print("  block %d %s (%d -> %d): rel_fro %.3e over %d rows" % (L, name, w.in_, N, err, len(sub)),
                  flush=True)
            assert err <= TOL, (L, name, err)
    for ys in want:
        for b, _ in ys:
            b.close()
    for b in list(dx.values()) + [b for bl in bufs for b in bl]:
        b.close()
