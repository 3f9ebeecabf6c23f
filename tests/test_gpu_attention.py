"""Dense attention and the DiT block's attention branch on the GPU
(fh3_hip_attention_dev, fh3_hip_attention_qkv_dev, fh3_attention) against the
oracle's restatement of src/core/fh3_ops.c:458-505,589-695 and the
reference's own attention fixture, through the C-ABI.

Bar: rel-Frobenius <= 2e-3 of the output against the CPU result (fp16
operands, fp32 accumulation and softmax), the same gate as the linear layer.
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


def _oracle_attn(oracle, q, k, v, rows=None):
    """The oracle's result for query rows `rows` (all when None)."""
    qs = q if rows is None else np.ascontiguousarray(q[rows])
    o = np.zeros_like(qs)
    heads, hd = q.shape[1], q.shape[2]
    oracle.fh3_oracle_attention_rows(H._ptr(qs), qs.shape[0], H._ptr(k), H._ptr(v), k.shape[0], H._ptr(o),
                                     heads, hd)
    return o


def _gpu_attn(F, q, k, v):
    n, heads, hd = q.shape
    dq, dk, dv = _buf(F, q), _buf(F, k), _buf(F, v)
    do = F.DeviceBuffer(q.nbytes)
    F.attention_dev(dq, dk, dv, do, n, heads, hd)
    F.synchronize()
    return do.download(np.float32, q.shape)


def test_reference_attention_fixture(gpu):
    """The reference's attention.bin (n = 777, not a multiple of the 64-key
    tile), reduced to heads 0 and 3 and every fourth query: the other query
    rows are zero (a query's output depends only on its own row)."""
    F = gpu
    f = H.read_ops_fixture("attention_sub")
    q = np.zeros_like(f["k"])
    q[f["q_idx"]] = f["q"]
    o = _gpu_attn(F, q, f["k"], f["v"])[f["q_idx"]]
    err = H.rel_fro(o, f["ref"])
    _say("attention fixture: rel_fro %.3e, check_close %.3e" % (err, H.check_close(o, f["ref"])))
    assert err <= TOL


@pytest.mark.parametrize("n,heads,hd,sigma", [(1, 1, 128, 1.0), (64, 2, 128, 1.0), (100, 3, 64, 1.0),
                                              (777, 2, 128, 0.5), (1024, 1, 128, 1.2), (2050, 2, 64, 1.0),
                                              (130, 4, 128, 0.05)])
def test_attention_vs_oracle(gpu, oracle, n, heads, hd, sigma):
    F = gpu
    rng = np.random.default_rng(n * 7 + heads + hd)
    q, k, v = ((rng.standard_normal((n, heads, hd)) * sigma).astype(np.float32) for _ in range(3))
    v = (v / sigma).astype(np.float32)
    o = _gpu_attn(F, q, k, v)
    ref = _oracle_attn(oracle, q, k, v)
    err = H.rel_fro(o, ref)
    _say("attention n=%d heads=%d hd=%d sigma=%.2f: rel_fro %.3e" % (n, heads, hd, sigma, err))
    assert np.isfinite(o).all()
    assert err <= TOL


def test_attention_large_n_rows(gpu, oracle):
    """n = 8192 keys (a DiT-length sequence per head): 96 seeded query rows
    against the oracle; every row is a convex combination of v (row sums of
    the weights are 1), so |o| <= max |v| on every channel."""
    F = gpu
    n, heads, hd = 8192, 2, 128
    rng = np.random.default_rng(11)
    q, k, v = (rng.standard_normal((n, heads, hd)).astype(np.float32) for _ in range(3))
    o = _gpu_attn(F, q, k, v)
    rows = np.sort(rng.choice(n, 96, replace=False))
    rows[-1] = n - 1
    err = H.rel_fro(o[rows], _oracle_attn(oracle, q, k, v, rows))
    _say("attention n=8192: rel_fro on 96 rows %.3e" % err)
    assert err <= TOL
    vmax = np.abs(v).max(axis=0)
    assert (np.abs(o) <= vmax[None] * (1 + 1e-3) + 1e-6).all()


def test_attention_closed_forms(gpu):
    """Identical keys: uniform weights, o = mean(v).  One key: o = v."""
    F = gpu
    rng = np.random.default_rng(5)
    n, heads, hd = 200, 2, 128
    q = rng.standard_normal((n, heads, hd)).astype(np.float32)
    k = np.repeat(rng.standard_normal((1, heads, hd)).astype(np.float32), n, axis=0)
    v = rng.standard_normal((n, heads, hd)).astype(np.float32)
    o = _gpu_attn(F, q, k, v)
    assert H.rel_fro(o, np.broadcast_to(v.mean(axis=0), o.shape)) <= TOL
    o1 = _gpu_attn(F, q[:1], k[:1], v[:1])
    assert H.rel_fro(o1, v[:1]) <= 1e-3    # v rounded to fp16 once


def test_attention_deterministic_and_host_wrapper(gpu):
    F = gpu
    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal((300, 3, 128)).astype(np.float32) for _ in range(3))
    a = _gpu_attn(F, q, k, v)
    b = _gpu_attn(F, q, k, v)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    c = F.attention_host(q, k, v)
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32))


def _rope_tables(rng, n, rot):
    ang = rng.uniform(0, 100, (n, rot // 2)).astype(np.float64)
    ang = np.concatenate([ang, ang], axis=1)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


@pytest.mark.parametrize("n,heads,hd,norm,rot", [(300, 3, 128, True, 96), (777, 2, 128, False, 96),
                                                 (65, 4, 64, True, 0), (129, 2, 128, True, 128)])
def test_attention_qkv_branch(gpu, oracle, n, heads, hd, norm, rot):
    """fh3_dit.c:390-411 from the qkv projection output: split, q/k rmsnorm
    per head, rope3, attention -- on the CPU through the oracle, on the GPU in
    one call reading qkv in place."""
    F = gpu
    rng = np.random.default_rng(n + heads + rot)
    inner = heads * hd
    qkv = (rng.standard_normal((n, 3 * inner)) * 2).astype(np.float32)
    qw = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    kw = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    eps = 1e-5
    cos, sin = _rope_tables(rng, n, rot) if rot else (None, None)
    # CPU: the reference's sequence through the oracle
    q = np.ascontiguousarray(qkv[:, :inner]).reshape(n, heads, hd)
    k = np.ascontiguousarray(qkv[:, inner:2 * inner]).reshape(n, heads, hd)
    v = np.ascontiguousarray(qkv[:, 2 * inner:]).reshape(n, heads, hd)
    if norm:
        H.elementwise(oracle, "fh3_oracle_", "rmsnorm", q, qw, n * heads, hd, eps)
        H.elementwise(oracle, "fh3_oracle_", "rmsnorm", k, kw, n * heads, hd, eps)
    if rot:
        H.elementwise(oracle, "fh3_oracle_", "rope3", q, cos, sin, n, heads, hd, rot)
        H.elementwise(oracle, "fh3_oracle_", "rope3", k, cos, sin, n, heads, hd, rot)
    ref = _oracle_attn(oracle, q, k, v)
    # GPU
    dqkv = _buf(F, qkv)
    do = F.DeviceBuffer(n * inner * 4)
    dn = (_buf(F, qw), _buf(F, kw)) if norm else (None, None)
    dr = (_buf(F, cos), _buf(F, sin)) if rot else (None, None)
    F.attention_qkv_dev(dqkv, n, heads, hd, do, dn[0], dn[1], eps, dr[0], dr[1], rot)
    F.synchronize()
    o = do.download(np.float32, (n, heads, hd))
    err = H.rel_fro(o, ref)
    _say("qkv branch n=%d heads=%d hd=%d norm=%d rot=%d: rel_fro %.3e" % (n, heads, hd, norm, rot, err))
    assert err <= TOL


def test_attention_argument_errors(gpu):
    F = gpu
    b = F.DeviceBuffer(4 * 96 * 4)
    with pytest.raises(F.Fh3Error):          # head dim 96 is not supported
        F.attention_dev(b, b, b, b, 4, 1, 96)
    with pytest.raises(F.Fh3Error):          # rope needs both tables and an even rot_dim <= hd
        F.attention_qkv_dev(b, 1, 1, 64, b, None, None, 1e-5, b, None, 64)
    with pytest.raises(F.Fh3Error):
        F.attention_qkv_dev(b, 1, 1, 64, b, None, None, 1e-5, b, b, 65)
    with pytest.raises(F.Fh3Error):          # norm weights come in pairs
        F.attention_qkv_dev(b, 1, 1, 64, b, b, None)
    with pytest.raises(F.Fh3Error):          # misaligned pointers
        F.attention_dev(b.ptr + 4, b, b, b, 1, 1, 64)
