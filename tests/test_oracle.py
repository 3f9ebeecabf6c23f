"""Pins the CPU oracle (oracle/fh3_oracle.c) before it is trusted as the
checker: golden fixtures of the reference's own tests, the reference build
itself, and closed forms that a plausible slip (wrong nibble, swapped scale
bits, dropped term, transposed operand) would fail.
"""
import os
import zlib

import numpy as np
import pytest

import helpers as H


# --------------------------------------------------------------------------
# Golden fixtures (reference tests/unit/test_quant.c:40-113, test_matmul.c)
# --------------------------------------------------------------------------
def test_dequant_q4k_fixture_bitexact(oracle):
    t, rows, cols, raw, ref = H.read_q4k_fixture()
    assert (t, rows, cols, raw.size) == (12, 4, 512, 1152)
    assert H.load_oracle().fh3_oracle_row_bytes(12, cols) * rows == raw.size
    out = H.oracle_dequant(oracle, raw, rows, cols)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("name", sorted(H.QTYPES))
def test_dequant_fixture_bitexact_every_type(oracle, name):
    """reference tests/unit/test_quant.c:40-130 for each decodable type; the
    fixtures were written by gguf-py's own dequantize, an implementation
    independent of the reference's C."""
    t, rows, cols, raw, ref = H.read_quant_fixture(name)
    assert (t, rows, cols) == (H.QTYPES[name][0], 4, 512)
    assert oracle.fh3_oracle_row_bytes(t, cols) * rows == raw.size
    out = H.oracle_dequant(oracle, raw, rows, cols, qtype=t)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("name", sorted(H.QTYPES))
@pytest.mark.parametrize("finite", [True, False])
def test_dequant_bitwise_vs_reference_build(oracle, ref, name, finite):
    """Random blocks (with raw, possibly Inf/NaN scale fields when not
    `finite`), odd lengths that leave a partial block unwritten."""
    rng = np.random.default_rng(zlib.crc32(("%s/%d" % (name, finite)).encode()))
    t, bl, bb, _ = H.QTYPES[name]
    rows, cols = 7, 1024
    raw = H.random_blocks(rng, name, rows, cols, finite=finite)
    if not finite and name not in ("F16", "BF16"):
        raw = rng.integers(0, 256, size=raw.size, dtype=np.uint8)
    for n in (cols, cols - 1, bl):
        a = np.full((rows, cols), 7.0, np.float32)
        b = np.full((rows, cols), 7.0, np.float32)
        rb = oracle.fh3_oracle_row_bytes(t, cols)
        for r in range(rows):
            p = raw[r * rb:]
            oracle.fh3_oracle_dequant(t, p.ctypes.data, a[r].ctypes.data, n)
            ref.fh3_dequant(t, p.ctypes.data, b[r].ctypes.data, n)
        same = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
        assert same.all(), (name, n)
        written = n if bl == 1 else (n // bl) * bl
        assert (a[:, written:] == 7.0).all()


def test_dequant_unsupported_types_write_nothing(oracle):
    """src/core/fh3_quant.c:314-316: Q4_0/Q4_1/Q5_0/Q5_1/Q8_1/Q8_K have row sizes
    but no decoder."""
    raw = np.arange(4096, dtype=np.uint8)
    for t in (2, 3, 6, 7, 9, 15, 99):
        out = np.full(256, 3.0, np.float32)
        oracle.fh3_oracle_dequant(t, raw.ctypes.data, out.ctypes.data, 256)
        assert (out == 3.0).all()


def test_q8_0_closed_form(oracle):
    """w = q * d with q int8 and d the block's fp16 scale."""
    raw = np.zeros(34 * 2, np.uint8)
    raw[0:2] = np.array([0.5], np.float16).view(np.uint8)
    raw[2:34] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    raw[34:36] = np.array([-3.0], np.float16).view(np.uint8)
    raw[36:68] = np.array([127, -128] * 16, dtype=np.int8).view(np.uint8)
    out = np.zeros(64, np.float32)
    oracle.fh3_oracle_dequant(8, raw.ctypes.data, out.ctypes.data, 64)
    assert np.array_equal(out[:32], np.arange(-16, 16) * 0.5)
    assert np.array_equal(out[32:], np.array([127, -128] * 16) * -3.0)


def test_matmul_fixture_vs_fp64(oracle):
    """reference tests/unit/test_matmul.c:143-156: rel-L2 <= 1e-6 vs NumPy fp64."""
    t, K, N, M, raw, x, bias, y = H.read_matmul_fixture()
    assert (t, K, N, M) == (12, 5376, 192, 37)
    yo = H.oracle_matmul(oracle, raw, K, N, x, bias)
    assert H.rel_fro(yo, y) <= 1e-6


# --------------------------------------------------------------------------
# The reference build (oracle/_ref) and the vectors it wrote
# --------------------------------------------------------------------------
def _golden():
    return np.load(os.path.join(H.GOLDEN, "ref_vectors.npz"), allow_pickle=False)


@pytest.mark.parametrize("case", range(5))
def test_matmul_bitwise_vs_reference_vectors(oracle, case):
    g = _golden()
    K, N, M, use_bias = (int(v) for v in g["c%d_shape" % case])
    bias = g["c%d_bias" % case] if use_bias else None
    y = H.oracle_matmul(oracle, g["c%d_w" % case], K, N, g["c%d_x" % case], bias)
    yr = g["c%d_y" % case]
    same = (y.view(np.uint32) == yr.view(np.uint32)) | (np.isnan(y) & np.isnan(yr))
    assert same.all()
    deq = H.oracle_dequant(oracle, g["c%d_w" % case], N, K)
    dr = g["c%d_deq" % case]
    same = (deq.view(np.uint32) == dr.view(np.uint32)) | (np.isnan(deq) & np.isnan(dr))
    assert same.all()


@pytest.mark.parametrize("K,N,M", [(256, 1, 1), (512, 70, 9), (2048, 129, 4)])
def test_matmul_bitwise_vs_reference_build(oracle, ref, K, N, M):
    rng = np.random.default_rng(K + N + M)
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    for b in (None, bias):
        yo = H.oracle_matmul(oracle, raw, K, N, x, b)
        for fn in ("fh3_matmul", "fh3_matmul_scalar", "fh3_matmul_avx2"):
            yr = H.matmul_with(ref, fn, raw, K, N, x, b)
            assert np.array_equal(yo.view(np.uint32), yr.view(np.uint32)), fn


def test_matmul_rows_subset_equals_full(oracle):
    rng = np.random.default_rng(5)
    K, N, M = 512, 200, 3
    raw = H.random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    full = H.oracle_matmul(oracle, raw, K, N, x)
    part = H.oracle_matmul_rows(oracle, raw, K, N, x, 37, 150)
    assert np.array_equal(part[:, 37:150].view(np.uint32), full[:, 37:150].view(np.uint32))
    assert np.isnan(part[:, :37]).all() and np.isnan(part[:, 150:]).all()


# --------------------------------------------------------------------------
# Closed forms
# --------------------------------------------------------------------------
def test_f16_decode_all_patterns(oracle):
    """Every fp16 bit pattern decodes to NumPy's exact float16 -> float32."""
    f = oracle.fh3_oracle_f16_to_f32
    hs = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = np.array([f(int(h)) for h in hs], dtype=np.float32)
    theirs = hs.view(np.float16).astype(np.float32)
    fin = np.isfinite(theirs) | np.isinf(theirs)
    assert np.array_equal(ours[fin].view(np.uint32), theirs[fin].view(np.uint32))
    assert np.isnan(ours[~fin]).all()
    # F16C quiets signalling NaNs: 0x7C01 -> 0x7FC02000
    assert np.float32(f(0x7C01)).view(np.uint32) == 0x7FC02000


def _pack_scales(sc, mn):
    """6-bit scale/min packing built bit by bit from the format description."""
    s = np.zeros(12, dtype=np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return s


def _block(d_bits, dmin_bits, sc, mn, q):
    """One super-block from field values; q[g][l] is the nibble of weight l of group g."""
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = np.array([d_bits], dtype=np.uint16).view(np.uint8)
    blk[2:4] = np.array([dmin_bits], dtype=np.uint16).view(np.uint8)
    blk[4:16] = _pack_scales(sc, mn)
    for c in range(4):
        blk[16 + 32 * c:48 + 32 * c] = (q[2 * c] | (q[2 * c + 1] << 4)).astype(np.uint8)
    return blk


def test_scale_min_layout_exhaustive(oracle):
    """d = dmin = 1 and q = 15 make every weight of group g equal to 15*sc_g - m_g
    exactly; sweep all 64 x 64 (sc, m) values through all 8 group slots."""
    q = np.full((8, 32), 15, dtype=np.uint8)
    blocks, expect = [], []
    vals = np.arange(64)
    rng = np.random.default_rng(1)
    for rep in range(64):
        sc = rng.permutation(vals)[:8] if rep else np.arange(8)
        mn = rng.permutation(vals)[:8]
        sc[rep % 8] = rep
        blocks.append(_block(0x3C00, 0x3C00, sc, mn, q))
        expect.append(np.repeat(15.0 * sc - mn, 32))
    # every (slot, sc) and (slot, m) pair
    for slot in range(8):
        for v in range(64):
            sc = np.zeros(8, dtype=np.int64); mn = np.zeros(8, dtype=np.int64)
            sc[slot] = v; mn[(slot + 3) % 8] = v
            blocks.append(_block(0x3C00, 0x3C00, sc, mn, q))
            expect.append(np.repeat(15.0 * sc - mn, 32))
    raw = np.concatenate(blocks)
    out = H.oracle_dequant(oracle, raw, len(blocks), 256)
    assert np.array_equal(out, np.array(expect, dtype=np.float32))


def test_nibble_order(oracle):
    """q = position pattern: chunk c byte l carries group 2c (low) and 2c+1 (high)."""
    q = np.array([[(g * 7 + l) % 16 for l in range(32)] for g in range(8)], dtype=np.uint8)
    blk = _block(0x3C00, 0x0000, np.ones(8, dtype=np.int64), np.zeros(8, dtype=np.int64), q)
    out = H.oracle_dequant(oracle, blk, 1, 256)[0]
    assert np.array_equal(out, q.reshape(-1).astype(np.float32))


def test_matmul_exact_integers(oracle):
    """Integer-valued weights and activations small enough that every fp32 sum
    is exact: the product must equal the int64 matrix product exactly."""
    rng = np.random.default_rng(3)
    K, N, M = 512, 23, 5
    blocks, wint = [], np.zeros((N, K), dtype=np.int64)
    for o in range(N):
        for b in range(K // 256):
            sc = rng.integers(0, 4, 8); mn = rng.integers(0, 8, 8)
            q = rng.integers(0, 16, (8, 32)).astype(np.uint8)
            blocks.append(_block(0x3C00, 0x3C00, sc, mn, q))
            wint[o, b * 256:(b + 1) * 256] = (sc[:, None] * q - mn[:, None]).reshape(-1)
    raw = np.concatenate(blocks)
    x = rng.integers(-3, 4, (M, K))
    bias = rng.integers(-9, 10, N).astype(np.float32)
    y = H.oracle_matmul(oracle, raw, K, N, x.astype(np.float32), bias)
    assert np.array_equal(y, (x @ wint.T + bias).astype(np.float32))


@pytest.mark.parametrize("name", ["F16", "BF16", "Q8_0", "Q2_K", "Q3_K", "Q5_K", "Q6_K"])
def test_matmul_other_types_bitwise_vs_reference_build(oracle, ref, name):
    """src/core/fh3_ops.c:317-404 decodes any type through fh3_dequant; the
    oracle's product must match the reference build bit for bit for each."""
    t = H.QTYPES[name][0]
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    K, N, M = 512, 70, 5
    raw = H.random_blocks(rng, name, N, K, scale_lo=-12, scale_hi=-8)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    for b in (None, bias):
        yo = H.matmul_with(oracle, "fh3_oracle_matmul", raw, K, N, x, b, qtype=t)
        yr = H.matmul_with(ref, "fh3_matmul", raw, K, N, x, b, qtype=t)
        assert np.isfinite(yo).all()
        assert np.array_equal(yo.view(np.uint32), yr.view(np.uint32))


def _general_rows(rng, name, N, K):
    if name == "F32":
        return (rng.standard_normal((N, K)) * 0.02).astype(np.float32).view(np.uint8).reshape(-1)
    return H.random_blocks(rng, name, N, K, scale_lo=-12, scale_hi=-8)


@pytest.mark.parametrize("name,K", [("F32", 7), ("F32", 33), ("F16", 32), ("F16", 96), ("BF16", 200),
                                    ("F16", 1000), ("Q8_0", 32), ("Q8_0", 96), ("Q8_0", 224)])
def test_matmul_short_rows_bitwise_vs_reference_build(oracle, ref, name, K):
    """Rows that are not whole 256-value super-blocks (the DiT's 32- and
    96-value patch projections, src/model/fh3_dit.c:352-353; any length for
    the element types, whole 32-blocks for Q8_0): the 8-lane part and the
    fmaf tail of src/core/fh3_ops.c:19-207, bitwise against the build."""
    t = 0 if name == "F32" else H.QTYPES[name][0]
    rng = np.random.default_rng(zlib.crc32(("%s%d" % (name, K)).encode()))
    N, M = 37, 5
    raw = _general_rows(rng, name, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    for b in (None, bias):
        yo = H.matmul_with(oracle, "fh3_oracle_matmul", raw, K, N, x, b, qtype=t)
        for fn in ("fh3_matmul", "fh3_matmul_scalar"):
            yr = H.matmul_with(ref, fn, raw, K, N, x, b, qtype=t)
            assert np.isfinite(yo).all()
            assert np.array_equal(yo.view(np.uint32), yr.view(np.uint32)), fn


@pytest.mark.parametrize("K", [1, 7, 13, 96])
def test_matmul_short_rows_exact_integers(oracle, K):
    """Small integers in fp32 weights and activations: every product and
    partial sum is exact, so the oracle must return the integer product for
    any row length, tail included (a dropped or doubled tail element fails)."""
    rng = np.random.default_rng(K)
    N, M = 11, 3
    w = rng.integers(-8, 9, size=(N, K)).astype(np.float32)
    x = rng.integers(-8, 9, size=(M, K)).astype(np.float32)
    bias = rng.integers(-100, 101, size=N).astype(np.float32)
    y = H.matmul_with(oracle, "fh3_oracle_matmul", w.view(np.uint8).reshape(-1), K, N, x, bias, qtype=0)
    assert np.array_equal(y, (x.astype(np.int64) @ w.astype(np.int64).T + bias.astype(np.int64)).astype(np.float32))


# --------------------------------------------------------------------------
# The DiT block's elementwise ops (src/core/fh3_ops.c:410-585) vs the build
# --------------------------------------------------------------------------
@pytest.mark.parametrize("n,dim", [(3, 5120), (2, 1000), (5, 13), (1, 7)])
def test_elementwise_ops_bitwise_vs_reference_build(oracle, ref, n, dim):
    rng = np.random.default_rng(n * 100 + dim)
    x = (rng.standard_normal((n, dim)) * 3).astype(np.float32)
    w = rng.standard_normal(dim).astype(np.float32)
    shift = rng.standard_normal((n, dim)).astype(np.float32)
    scale = (rng.standard_normal((n, dim)) * 0.3).astype(np.float32)
    gate = rng.standard_normal((n, dim)).astype(np.float32)
    res = []
    for lib, pre in ((oracle, "fh3_oracle_"), (ref, "fh3_")):
        a = x.copy()
        H.elementwise(lib, pre, "rmsnorm", a, w, n, dim, 1e-6)
        b = a.copy()
        H.elementwise(lib, pre, "modulate", b, shift, scale, n, dim)
        h = x.copy()
        H.elementwise(lib, pre, "gate_residual", h, gate, b, n, dim)
        F = dim // 2 if dim % 2 == 0 else dim
        sw_in = np.ascontiguousarray(np.concatenate([x, gate], axis=1)[:, : 2 * F] * 10).astype(np.float32)
        sw = np.zeros((n, F), np.float32)
        H.elementwise(lib, pre, "swiglu", sw_in, sw, n, F)
        res.append((a, b, h, sw))
    for o, r in zip(res[0], res[1]):
        assert np.array_equal(o.view(np.uint32), r.view(np.uint32))


def test_elementwise_closed_forms(oracle):
    """rmsnorm of a constant row is w; modulate by (shift 0, scale 0) is the
    identity; swiglu of gate 0 is 0 and of a very negative gate is exactly 0;
    gate_residual with gate 0 leaves h."""
    dim = 64
    x = np.full((1, dim), 3.0, np.float32)
    w = np.arange(dim, dtype=np.float32) / 7
    H.elementwise(oracle, "fh3_oracle_", "rmsnorm", x, w, 1, dim, 0.0)
    assert np.allclose(x[0], w, rtol=1e-6)
    y = np.random.default_rng(0).standard_normal((2, dim)).astype(np.float32)
    z = y.copy()
    H.elementwise(oracle, "fh3_oracle_", "modulate", z, np.zeros_like(y), np.zeros_like(y), 2, dim)
    assert np.array_equal(z, y)
    sw_in = np.zeros((1, 2 * dim), np.float32)
    sw_in[0, :dim] = 5.0
    sw_in[0, dim:] = np.linspace(-100, 0, dim, dtype=np.float32)
    out = np.ones((1, dim), np.float32)
    H.elementwise(oracle, "fh3_oracle_", "swiglu", sw_in, out, 1, dim)
    assert out[0, -1] == 0.0 and (out[0, sw_in[0, dim:] < -80] == 0.0).all()
    h = y.copy()
    H.elementwise(oracle, "fh3_oracle_", "gate_residual", h, np.zeros_like(y), z, 2, dim)
    assert np.array_equal(h, y)


# --------------------------------------------------------------------------
# The reference's own op fixtures (tests/unit/test_ops.c: check_close <= 1e-5)
# --------------------------------------------------------------------------
def test_elementwise_fixtures(oracle):
    f = H.read_ops_fixture("rmsnorm")
    x = f["x"].copy()
    H.elementwise(oracle, "fh3_oracle_", "rmsnorm", x, f["w"], f["n"], f["dim"], f["eps"])
    assert H.check_close(x, f["ref"]) <= 1e-5
    f = H.read_ops_fixture("modulate")
    x = f["x"].copy()
    H.elementwise(oracle, "fh3_oracle_", "modulate", x, f["shift"], f["scale"], f["n"], f["dim"])
    assert H.check_close(x, f["ref"]) <= 1e-5
    # the plausible slip x*scale + shift fails it (test_ops.c's own invariant)
    assert H.check_close(f["x"] * f["scale"] + f["shift"], f["ref"]) > 1.0
    f = H.read_ops_fixture("gate_residual")
    h = f["h"].copy()
    H.elementwise(oracle, "fh3_oracle_", "gate_residual", h, f["gate"], f["y"], f["n"], f["dim"])
    assert H.check_close(h, f["ref"]) <= 1e-5
    f = H.read_ops_fixture("swiglu")
    out = np.zeros_like(f["ref"])
    H.elementwise(oracle, "fh3_oracle_", "swiglu", f["inp"], out, f["n"], f["F"])
    assert H.check_close(out, f["ref"]) <= 1e-5
    swapped = np.ascontiguousarray(np.concatenate([f["inp"][:, f["F"]:], f["inp"][:, :f["F"]]], axis=1))
    H.elementwise(oracle, "fh3_oracle_", "swiglu", swapped, out, f["n"], f["F"])
    assert H.check_close(out, f["ref"]) > 1.0


def test_rope3_fixture(oracle):
    f = H.read_ops_fixture("rope3")
    n, heads, hd, rot = f["n"], f["heads"], f["hd"], f["rot"]
    x = f["x"].copy()
    H.elementwise(oracle, "fh3_oracle_", "rope3", x, f["cos"], f["sin"], n, heads, hd, rot)
    assert H.check_close(x, f["ref"]) <= 1e-5
    assert np.array_equal(x[..., rot:], f["x"][..., rot:])      # channels past rot_dim untouched
    # rotating all 128 channels (cos 1, sin 0 past 96) must fail, as test_ops.c checks
    c = np.concatenate([f["cos"], np.ones((n, hd - rot), np.float32)], axis=1)
    s = np.concatenate([f["sin"], np.zeros((n, hd - rot), np.float32)], axis=1)
    xb = f["x"].copy()
    H.elementwise(oracle, "fh3_oracle_", "rope3", xb, np.ascontiguousarray(c), np.ascontiguousarray(s),
                  n, heads, hd, hd)
    assert np.abs(xb - f["ref"]).max() > 1.0


def test_attention_fixture(oracle):
    """attention.bin (n = 777: not a multiple of the 64-key tile), reduced to
    heads 0 and 3 and every fourth query by make_ops_fixtures.py."""
    f = H.read_ops_fixture("attention_sub")
    o = np.zeros_like(f["ref"])
    oracle.fh3_oracle_attention_rows(H._ptr(f["q"]), f["nq"], H._ptr(f["k"]), H._ptr(f["v"]), f["n"],
                                     H._ptr(o), f["heads"], f["hd"])
    assert H.check_close(o, f["ref"]) <= 1e-5
    assert f["q_idx"][-1] == f["n"] - 1          # the last query row is covered


@pytest.mark.parametrize("n,heads,hd", [(130, 2, 128), (70, 3, 75), (1, 1, 8), (64, 1, 64)])
def test_attention_rope3_bitwise_vs_reference_build(oracle, ref, n, heads, hd):
    rng = np.random.default_rng(n + hd)
    q, k, v = ((rng.standard_normal((n, heads, hd)) * 1.5).astype(np.float32) for _ in range(3))
    outs = []
    for lib, pre in ((oracle, "fh3_oracle_"), (ref, "fh3_")):
        o = np.zeros_like(q)
        H.elementwise(lib, pre, "attention", q, k, v, o, n, heads, hd)
        outs.append(o)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    rot = hd - hd % 4 if hd >= 4 else 2
    cos = rng.standard_normal((n, rot)).astype(np.float32)
    sin = rng.standard_normal((n, rot)).astype(np.float32)
    xs = []
    for lib, pre in ((oracle, "fh3_oracle_"), (ref, "fh3_")):
        x = q.copy()
        H.elementwise(lib, pre, "rope3", x, cos, sin, n, heads, hd, rot)
        xs.append(x)
    assert np.array_equal(xs[0].view(np.uint32), xs[1].view(np.uint32))


def test_attention_closed_forms(oracle):
    """One key: o = v exactly.  Identical keys: uniform weights, o = mean(v).
    A key whose score dominates by far: o = its v."""
    hd, heads = 64, 2
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, heads, hd)).astype(np.float32)
    v1 = rng.standard_normal((1, heads, hd)).astype(np.float32)
    o = np.zeros_like(q)
    oracle.fh3_oracle_attention_rows(H._ptr(q), 1, H._ptr(q), H._ptr(v1), 1, H._ptr(o), heads, hd)
    assert np.array_equal(o, v1)
    n = 150
    kk = np.repeat(rng.standard_normal((1, heads, hd)).astype(np.float32), n, axis=0)
    vv = rng.standard_normal((n, heads, hd)).astype(np.float32)
    oracle.fh3_oracle_attention_rows(H._ptr(q), 1, H._ptr(kk), H._ptr(vv), n, H._ptr(o), heads, hd)
    assert np.allclose(o[0], vv.mean(axis=0), rtol=1e-5, atol=1e-6)
    kd = rng.standard_normal((n, heads, hd)).astype(np.float32) * 0.01
    kd[97] = q[0] * 50.0
    oracle.fh3_oracle_attention_rows(H._ptr(q), 1, H._ptr(kd), H._ptr(vv), n, H._ptr(o), heads, hd)
    assert np.allclose(o[0], vv[97], rtol=1e-6, atol=1e-6)


# --------------------------------------------------------------------------
# Video sparse attention (src/core/fh3_vsa.c; tests/unit/test_vsa.c)
# --------------------------------------------------------------------------
def _fix_seq(f):
    return (f["n"], f["num_text"], f["num_audio"], f["num_video"], f["grid_t"], f["grid_h"], f["grid_w"])


@pytest.mark.parametrize("name", ["vsa_n784", "vsa_padded", "vsa_sparsity0"])
def test_vsa_fixtures(oracle, name):
    """The reference's three VSA fixtures (rel-L2 <= 1e-5, as test_vsa.c),
    cut to two heads."""
    f = H.read_vsa_fixture(name)
    o = H.vsa_oracle(oracle, f["q"], f["k"], f["v"], f["gate"], _fix_seq(f), f["sparsity"])
    assert H.rel_fro(o, f["ref"]) <= 1e-5


def test_vsa_sparsity0_without_gate_is_dense(oracle):
    """test_vsa.c's structural check: sparsity 0 and no gate equals dense attention."""
    f = H.read_vsa_fixture("vsa_sparsity0")
    o = H.vsa_oracle(oracle, f["q"], f["k"], f["v"], None, _fix_seq(f), 0.0)
    d = np.zeros_like(o)
    H.elementwise(oracle, "fh3_oracle_", "attention", f["q"], f["k"], f["v"], d, f["n"], f["heads"], f["head_dim"])
    assert H.rel_fro(o, d) <= 1e-5


VSA_CASES = [
    # (n, text, audio, video, gt, gh, gw, heads, hd, sparsity, gate)
    (784, 0, 0, 784, 7, 8, 14, 2, 64, 0.8, True),
    (268, 35, 23, 210, 5, 6, 7, 3, 64, 0.8, False),
    (300, 100, 0, 200, 2, 10, 10, 2, 128, 0.5, True),
    (130, 0, 0, 130, 0, 0, 0, 1, 32, 0.9, True),      # no grid: 1 x 1 x V
    (90, 40, 10, 41, 2, 2, 10, 2, 16, 0.8, True),     # counts do not sum to n: all video
    (512, 64, 64, 384, 6, 8, 8, 2, 64, 0.0, True),
    (1000, 16, 24, 960, 6, 10, 16, 1, 64, 0.95, True),
]


@pytest.mark.parametrize("case", VSA_CASES)
def test_vsa_bitwise_vs_reference_build(oracle, ref, case):
    n, T, A, V, gt, gh, gw, heads, hd, sp, has_gate = case
    rng = np.random.default_rng(n + heads * 10 + hd)
    q, k, v, g = ((rng.standard_normal((n, heads, hd)) * 0.7).astype(np.float32) for _ in range(4))
    gate = g if has_gate else None
    seq = (n, T, A, V, gt, gh, gw)
    a = H.vsa_oracle(oracle, q, k, v, gate, seq, sp)
    b = H.vsa_ref(ref, q, k, v, gate, seq, sp)
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_vsa_geometry_closed_form(oracle):
    """Tiles partition the sequence; text and audio runs come first in runs of
    64; a full 4x4x4 video cube is 64 consecutive-in-(t,h,w) tokens."""
    import ctypes
    n, T, A, gt, gh, gw = 35 + 70 + 8 * 8 * 8, 35, 70, 8, 8, 8
    tok = np.zeros(n, np.int32)
    off = np.zeros(n + 9, np.int32)
    npre = ctypes.c_int()
    f = oracle.fh3_oracle_vsa_geometry
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_int] * 8 + [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
    nt = f(n, T, A, n - T - A, gt, gh, gw, 64, H._ptr(tok), H._ptr(off), n + 8, ctypes.byref(npre))
    assert npre.value == 1 + 2 and nt == 3 + 8
    assert sorted(tok.tolist()) == list(range(n))
    assert list(off[:4]) == [0, 35, 99, 105]
    cube = tok[off[3]:off[4]] - (T + A)
    t, h, w = cube // 64, (cube // 8) % 8, cube % 8
    assert (t < 4).all() and (h < 4).all() and (w < 4).all() and len(cube) == 64
