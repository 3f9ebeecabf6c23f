"""Video sparse attention on the GPU (fh3_hip_vsa_attention_dev,
fh3_hip_vsa_attention_qkv_dev, fh3_vsa_attention) against the oracle's
restatement of src/core/fh3_vsa.c and the reference's own VSA fixtures,
through the C-ABI.

Bars: the tile choice is exact (the tile statistics are computed in the
reference's order, so the selected key tiles are the CPU's -- checked through
an output whose support is the selection); the attention output within
rel-Frobenius 2e-3 of the CPU result (fp16 operands, fp32 accumulation).
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _say(msg):
    print(msg, flush=True)


def _buf(F, a):
    return F.DeviceBuffer.from_array(np.ascontiguousarray(a, dtype=np.float32))


def _gpu_vsa(F, q, k, v, gate, seq, sparsity, tile=64):
    n, heads, hd = q.shape
    dq, dk, dv = _buf(F, q), _buf(F, k), _buf(F, v)
    dg = _buf(F, gate) if gate is not None else None
    do = F.DeviceBuffer(q.nbytes)
    F.vsa_attention_dev(dq, dk, dv, dg, do, F.seq_of(*seq[:4], grid=seq[4:]), heads, hd, sparsity, tile)
    F.synchronize()
    return do.download(np.float32, q.shape)


@pytest.mark.parametrize("name", ["vsa_n784", "vsa_padded", "vsa_sparsity0"])
def test_reference_vsa_fixtures(gpu, name):
    F = gpu
    f = H.read_vsa_fixture(name)
    seq = (f["n"], f["num_text"], f["num_audio"], f["num_video"], f["grid_t"], f["grid_h"], f["grid_w"])
    o = _gpu_vsa(F, f["q"], f["k"], f["v"], f["gate"], seq, f["sparsity"])
    err = H.rel_fro(o, f["ref"])
    _say("%s: rel_fro %.3e" % (name, err))
    assert err <= TOL


CASES = [
    # (n, text, audio, video, gt, gh, gw, heads, hd, sparsity, gate)
    (784, 0, 0, 784, 7, 8, 14, 2, 64, 0.8, True),
    (268, 35, 23, 210, 5, 6, 7, 3, 64, 0.8, False),
    (300, 100, 0, 200, 2, 10, 10, 2, 128, 0.5, True),
    (130, 0, 0, 130, 0, 0, 0, 1, 64, 0.9, True),       # no grid: 1 x 1 x V
    (90, 40, 10, 41, 2, 2, 10, 2, 64, 0.8, True),      # counts do not sum to n: all video
    (512, 64, 64, 384, 6, 8, 8, 2, 64, 0.0, True),
    (2304, 77, 0, 2227, 0, 0, 0, 2, 128, 0.8, True),
    (4096 + 120, 120, 0, 4096, 16, 16, 16, 2, 128, 0.8, True),
]


@pytest.mark.parametrize("case", CASES)
def test_vsa_vs_oracle(gpu, oracle, case):
    F = gpu
    n, T, A, V, gt, gh, gw, heads, hd, sp, has_gate = case
    rng = np.random.default_rng(n + heads * 10 + hd)
    q, k, v, g = ((rng.standard_normal((n, heads, hd)) * 0.7).astype(np.float32) for _ in range(4))
    gate = g if has_gate else None
    seq = (n, T, A, V, gt, gh, gw)
    o = _gpu_vsa(F, q, k, v, gate, seq, sp)
    ref = H.vsa_oracle(oracle, q, k, v, gate, seq, sp)
    err = H.rel_fro(o, ref)
    _say("vsa n=%d T=%d A=%d grid=%s heads=%d hd=%d sp=%.2f gate=%d: rel_fro %.3e"
         % (n, T, A, (gt, gh, gw), heads, hd, sp, has_gate, err))
    assert np.isfinite(o).all()
    assert err <= TOL


@pytest.mark.parametrize("sparsity", [0.8, 0.5, 0.95])
def test_vsa_tile_choice_exact(gpu, oracle, sparsity):
    """Key tile j carries v = e_j (one-hot on channel j), no gate: a query's
    output row is then sum over its selected tiles of (weight) e_j, so the
    nonzero channels are exactly the selected tiles.  Tile scores are made
    close (small q, k) so the top-k choice is sensitive to rounding."""
    F = gpu
    n_text, gt, gh, gw = 50, 8, 16, 16          # 1 text tile + 2*4*4 = 32 video tiles
    n = n_text + gt * gh * gw
    heads, hd = 2, 128
    rng = np.random.default_rng(int(sparsity * 100))
    q = (rng.standard_normal((n, heads, hd)) * 0.3).astype(np.float32)
    k = (rng.standard_normal((n, heads, hd)) * 0.3).astype(np.float32)
    # tile of each token, from the oracle's geometry
    import ctypes
    tok = np.zeros(n, np.int32)
    off = np.zeros(n + 9, np.int32)
    npre = ctypes.c_int()
    f = oracle.fh3_oracle_vsa_geometry
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_int] * 8 + [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
    T = f(n, n_text, 0, n - n_text, gt, gh, gw, 64, H._ptr(tok), H._ptr(off), n + 8, ctypes.byref(npre))
    assert T == 33
    v = np.zeros((n, heads, hd), np.float32)
    for j in range(T):
        v[tok[off[j]:off[j + 1]], :, j] = 1.0
    seq = (n, n_text, 0, n - n_text, gt, gh, gw)
    o = _gpu_vsa(F, q, k, v, None, seq, sparsity)
    ref = H.vsa_oracle(oracle, q, k, v, None, seq, sparsity)
    sel_gpu = np.abs(o[..., :T]) > 1e-6
    sel_cpu = np.abs(ref[..., :T]) > 1e-6
    _say("sparsity %.2f: %d selected (token, head, tile) triples; differences %d"
         % (sparsity, sel_cpu.sum(), (sel_gpu != sel_cpu).sum()))
    assert np.array_equal(sel_gpu, sel_cpu)
    assert H.rel_fro(o, ref) <= TOL


def test_vsa_sparsity0_without_gate_is_dense(gpu):
    """test_vsa.c's structural check on the device: sparsity 0, no gate ==
    dense attention (here the GPU dense path)."""
    F = gpu
    f = H.read_vsa_fixture("vsa_sparsity0")
    seq = (f["n"], f["num_text"], f["num_audio"], f["num_video"], f["grid_t"], f["grid_h"], f["grid_w"])
    o = _gpu_vsa(F, f["q"], f["k"], f["v"], None, seq, 0.0)
    n, heads, hd = f["q"].shape
    dq, dk, dv = _buf(F, f["q"]), _buf(F, f["k"]), _buf(F, f["v"])
    dd = F.DeviceBuffer(f["q"].nbytes)
    F.attention_dev(dq, dk, dv, dd, n, heads, hd)
    F.synchronize()
    assert H.rel_fro(o, dd.download(np.float32, f["q"].shape)) <= TOL


def test_vsa_deterministic_and_host_wrapper(gpu):
    F = gpu
    rng = np.random.default_rng(3)
    n, heads, hd = 784, 2, 64
    q, k, v, g = (rng.standard_normal((n, heads, hd)).astype(np.float32) for _ in range(4))
    seq = (n, 0, 0, n, 7, 8, 14)
    a = _gpu_vsa(F, q, k, v, g, seq, 0.8)
    b = _gpu_vsa(F, q, k, v, g, seq, 0.8)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    c = F.vsa_attention_host(q, k, v, g, F.seq_of(n, 0, 0, n, grid=(7, 8, 14)), 0.8)
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
    # a different sequence shape replaces the cached geometry, then the first returns
    _gpu_vsa(F, q[:300], k[:300], v[:300], g[:300], (300, 100, 0, 200, 2, 10, 10), 0.8)
    d = _gpu_vsa(F, q, k, v, g, seq, 0.8)
    assert np.array_equal(a.view(np.uint32), d.view(np.uint32))


def test_vsa_qkv_branch(gpu, oracle):
    """fh3_dit.c:390-409 with VSA: q/k rmsnorm + rope3 from the qkv output,
    then VSA -- against the CPU sequence through the oracle."""
    F = gpu
    n_text, gt, gh, gw = 64, 4, 8, 12
    n = n_text + gt * gh * gw
    heads, hd, rot = 2, 128, 96
    inner = heads * hd
    rng = np.random.default_rng(21)
    qkv = (rng.standard_normal((n, 3 * inner)) * 2).astype(np.float32)
    qw = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    kw = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    ang = rng.uniform(0, 50, (n, rot // 2))
    ang = np.concatenate([ang, ang], axis=1)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    gate = rng.standard_normal((n, heads, hd)).astype(np.float32)
    q = np.ascontiguousarray(qkv[:, :inner]).reshape(n, heads, hd)
    k = np.ascontiguousarray(qkv[:, inner:2 * inner]).reshape(n, heads, hd)
    v = np.ascontiguousarray(qkv[:, 2 * inner:]).reshape(n, heads, hd)
    H.elementwise(oracle, "fh3_oracle_", "rmsnorm", q, qw, n * heads, hd, 1e-5)
    H.elementwise(oracle, "fh3_oracle_", "rmsnorm", k, kw, n * heads, hd, 1e-5)
    H.elementwise(oracle, "fh3_oracle_", "rope3", q, cos, sin, n, heads, hd, rot)
    H.elementwise(oracle, "fh3_oracle_", "rope3", k, cos, sin, n, heads, hd, rot)
    seq = (n, n_text, 0, n - n_text, gt, gh, gw)
    ref = H.vsa_oracle(oracle, q, k, v, gate, seq, 0.8)
    do = F.DeviceBuffer(n * inner * 4)
    F.vsa_attention_qkv_dev(_buf(F, qkv), _buf(F, gate), do, F.seq_of(n, n_text, 0, grid=(gt, gh, gw)), heads, hd,
                            0.8, 64, _buf(F, qw), _buf(F, kw), 1e-5, _buf(F, cos), _buf(F, sin), rot)
    F.synchronize()
    err = H.rel_fro(do.download(np.float32, (n, heads, hd)), ref)
    _say("vsa qkv branch: rel_fro %.3e" % err)
    assert err <= TOL


def test_vsa_argument_errors(gpu):
    F = gpu
    b = F.DeviceBuffer(64 * 2 * 128 * 4)
    sq = F.seq_of(64, grid=(1, 8, 8))
    with pytest.raises(F.Fh3Error):          # head dim 96 is not supported
        F.vsa_attention_dev(b, b, b, None, b, sq, 1, 96)
    with pytest.raises(F.Fh3Error):          # tiles above 64 slots
        F.vsa_attention_dev(b, b, b, None, b, sq, 1, 64, 0.8, 128)
    with pytest.raises(F.Fh3Error):          # rope needs both tables
        F.vsa_attention_qkv_dev(b, None, b, sq, 1, 64, 0.8, 64, None, None, 1e-5, b, None, 64)
    with pytest.raises(F.Fh3Error):          # misaligned
        F.vsa_attention_dev(b.ptr + 4, b, b, None, b, sq, 1, 64)


def test_vsa_after_shutdown_and_reinit(gpu):
    """fh3_hip_shutdown frees the library's buffers, the kept tile geometry
    included; the next call after re-initialisation rebuilds it."""
    F = gpu
    rng = np.random.default_rng(8)
    n, heads, hd = 268, 2, 64
    q, k, v, g = (rng.standard_normal((n, heads, hd)).astype(np.float32) for _ in range(4))
    seq = (n, 35, 23, 210, 5, 6, 7)
    a = _gpu_vsa(F, q, k, v, g, seq, 0.8)
    F.lib().fh3_hip_shutdown()
    F.init(0)
    b = _gpu_vsa(F, q, k, v, g, seq, 0.8)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
