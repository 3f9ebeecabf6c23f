"""Shared test helpers: ctypes loaders for the oracle and the reference build,
readers for the reference's golden fixtures, and seeded input generators.

The oracle (oracle/libfh3_oracle.so) is the checker; nothing here is a compute
path of the product.
"""
import ctypes
import os
import struct
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
ORACLE_SO = os.path.join(ROOT, "oracle", "libfh3_oracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libfh3_ref.so")

Q4_K = 12
F32 = 0


class OracleW(ctypes.Structure):
    """Layout of Fh3W (reference include/fh3/fh3.h:82-87)."""
    _fields_ = [("type", ctypes.c_int), ("in_", ctypes.c_int64),
                ("out", ctypes.c_int64), ("data", ctypes.c_void_p)]


_F = ctypes.POINTER(ctypes.c_float)


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def load_oracle():
    if not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    lib = ctypes.CDLL(ORACLE_SO)
    lib.fh3_oracle_f16_to_f32.restype = ctypes.c_float
    lib.fh3_oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.fh3_oracle_row_bytes.restype = ctypes.c_size_t
    lib.fh3_oracle_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int64]
    lib.fh3_oracle_dequant.restype = None
    lib.fh3_oracle_dequant.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    lib.fh3_oracle_matmul.restype = None
    lib.fh3_oracle_matmul.argtypes = [ctypes.POINTER(OracleW), ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_int, ctypes.c_void_p]
    lib.fh3_oracle_matmul_rows.restype = None
    lib.fh3_oracle_matmul_rows.argtypes = [ctypes.POINTER(OracleW), ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64]
    lib.fh3_oracle_threads.restype = ctypes.c_int
    _bind_elementwise(lib, "fh3_oracle_")
    return lib


def _bind_elementwise(lib, prefix):
    P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    for name, args in (("rmsnorm", [P, P, I, I, F]), ("modulate", [P, P, P, I, I]), ("swiglu", [P, P, I, I]),
                       ("gate_residual", [P, P, P, I, I]), ("rope3", [P, P, P, I, I, I, I]),
                       ("attention", [P, P, P, P, I, I, I])):
        f = getattr(lib, prefix + name)
        f.restype = None
        f.argtypes = args
    if hasattr(lib, prefix + "attention_rows"):
        f = getattr(lib, prefix + "attention_rows")
        f.restype = None
        f.argtypes = [P, I, P, P, I, P, I, I]


OPS_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ops")


def read_ops_fixture(name):
    """The reference's op fixtures copied by tests/golden/make_ops_fixtures.py:
    a dict of header fields and float32 arrays."""
    raw = open(os.path.join(OPS_DIR, name + ".bin"), "rb").read()
    u32 = lambda i: int(np.frombuffer(raw, "<u4", 1, 4 * i)[0])
    f32 = lambda off, cnt: np.frombuffer(raw, "<f4", cnt, off).copy()
    if name == "rmsnorm":
        n, dim = u32(0), u32(1)
        eps = float(np.frombuffer(raw, "<f4", 1, 8)[0])
        o = 12
        x = f32(o, n * dim).reshape(n, dim); o += 4 * n * dim
        w = f32(o, dim); o += 4 * dim
        return dict(n=n, dim=dim, eps=eps, x=x, w=w, ref=f32(o, n * dim).reshape(n, dim))
    if name in ("modulate", "gate_residual"):
        n, dim = u32(0), u32(1)
        arrs = [f32(8 + 4 * n * dim * i, n * dim).reshape(n, dim) for i in range(4)]
        keys = ("x", "shift", "scale", "ref") if name == "modulate" else ("h", "gate", "y", "ref")
        return dict(n=n, dim=dim, **dict(zip(keys, arrs)))
    if name == "swiglu":
        n, F = u32(0), u32(1)
        return dict(n=n, F=F, inp=f32(8, n * 2 * F).reshape(n, 2 * F),
                    ref=f32(8 + 8 * n * F, n * F).reshape(n, F))
    if name == "rope3":
        n, heads, hd, rot = u32(0), u32(1), u32(2), u32(3)
        cx, cr = n * heads * hd, n * rot
        o = 16
        x = f32(o, cx).reshape(n, heads, hd); o += 4 * cx
        c = f32(o, cr).reshape(n, rot); o += 4 * cr
        sn = f32(o, cr).reshape(n, rot); o += 4 * cr
        return dict(n=n, heads=heads, hd=hd, rot=rot, x=x, cos=c, sin=sn, ref=f32(o, cx).reshape(n, heads, hd))
    if name == "attention_sub":
        n, heads, hd, nq = u32(0), u32(1), u32(2), u32(3)
        o = 16
        hidx = np.frombuffer(raw, "<i4", heads, o).copy(); o += 4 * heads
        qidx = np.frombuffer(raw, "<i4", nq, o).copy(); o += 4 * nq
        out = dict(n=n, heads=heads, hd=hd, nq=nq, head_idx=hidx, q_idx=qidx)
        for key, rows in (("q", nq), ("k", n), ("v", n), ("ref", nq)):
            cnt = rows * heads * hd
            out[key] = f32(o, cnt).reshape(rows, heads, hd)
            o += 4 * cnt
        return out
    raise ValueError(name)


VSA_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "vsa")


def read_vsa_fixture(name):
    """A VSA fixture cut to two heads by tests/golden/make_ops_fixtures.py."""
    raw = open(os.path.join(VSA_DIR, name + ".bin"), "rb").read()
    h = struct.unpack("<IIIIIIIIIfI", raw[:44])
    keys = ("n", "num_text", "num_audio", "num_video", "grid_t", "grid_h", "grid_w", "heads", "head_dim",
            "sparsity", "has_gate")
    out = dict(zip(keys, h))
    n, heads, hd = out["n"], out["heads"], out["head_dim"]
    cnt = n * heads * hd
    names = ("q", "k", "v", "gate", "ref") if out["has_gate"] else ("q", "k", "v", "ref")
    for i, key in enumerate(names):
        out[key] = np.frombuffer(raw, "<f4", cnt, 44 + 4 * cnt * i).reshape(n, heads, hd).copy()
    if not out["has_gate"]:
        out["gate"] = None
    return out


class VsaCfg(ctypes.Structure):      # reference include/fh3/fh3.h:41-44
    _fields_ = [("tile", ctypes.c_int), ("sparsity", ctypes.c_float)]


class Seq(ctypes.Structure):         # reference src/model/fh3_seq.h:32-45
    _fields_ = [("seq_len", ctypes.c_int), ("num_text", ctypes.c_int), ("num_audio", ctypes.c_int),
                ("num_video", ctypes.c_int), ("grid_t", ctypes.c_int), ("grid_h", ctypes.c_int),
                ("grid_w", ctypes.c_int), ("tags", ctypes.c_void_p), ("pair_index", ctypes.c_void_p),
                ("pos", ctypes.c_void_p), ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p)]


def _vsa_args(q, k, v, gate):
    return [_ptr(np.ascontiguousarray(a, dtype=np.float32)) if a is not None else None for a in (q, k, v, gate)]


def vsa_oracle(oracle, q, k, v, gate, seq, sparsity=0.8, tile=64):
    """fh3_oracle_vsa_attention; seq = (n, num_text, num_audio, num_video, gt, gh, gw)."""
    q, k, v = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v))
    g = None if gate is None else np.ascontiguousarray(gate, dtype=np.float32)
    o = np.full_like(q, np.nan)
    n, heads, hd = q.shape
    f = oracle.fh3_oracle_vsa_attention
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_int, ctypes.c_float] + [ctypes.c_void_p] * 5 + [ctypes.c_int] * 9
    rc = f(tile, sparsity, _ptr(q), _ptr(k), _ptr(v), None if g is None else _ptr(g), _ptr(o), *seq, heads, hd)
    assert rc == 0
    return o


def vsa_ref(ref, q, k, v, gate, seq, sparsity=0.8, tile=64):
    """The reference build's fh3_vsa_attention."""
    q, k, v = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v))
    g = None if gate is None else np.ascontiguousarray(gate, dtype=np.float32)
    o = np.full_like(q, np.nan)
    n, heads, hd = q.shape
    cfg = VsaCfg(tile, sparsity)
    sq = Seq(*seq, None, None, None, None, None)
    f = ref.fh3_vsa_attention
    f.restype = None
    f.argtypes = [ctypes.POINTER(VsaCfg)] + [ctypes.c_void_p] * 5 + [ctypes.POINTER(Seq), ctypes.c_int, ctypes.c_int]
    f(ctypes.byref(cfg), _ptr(q), _ptr(k), _ptr(v), None if g is None else _ptr(g), _ptr(o), ctypes.byref(sq),
      heads, hd)
    return o


def check_close(actual, ref):
    """The reference's test_ops.c check_close metric: max |a - r| / max(|r|, 1)."""
    a = np.asarray(actual, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    return float(np.max(np.abs(a - r) / np.maximum(np.abs(r), 1.0)))


def load_ref():
    """The reference's own fh3_quant.c/fh3_ops.c built by oracle/Makefile, or None."""
    if not os.path.exists(REF_SO):
        return None
    lib = ctypes.CDLL(REF_SO)
    lib.fh3_dequant.restype = None
    lib.fh3_dequant.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    for name in ("fh3_matmul", "fh3_matmul_scalar", "fh3_matmul_avx2"):
        f = getattr(lib, name)
        f.restype = None
        f.argtypes = [ctypes.POINTER(OracleW), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.fh3_row_bytes.restype = ctypes.c_size_t
    lib.fh3_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int64]
    lib.fh3_rng_normal.restype = None
    lib.fh3_rng_normal.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_size_t]
    _bind_elementwise(lib, "fh3_")
    return lib


def elementwise(lib, prefix, op, *arrays_and_sizes):
    """Call <prefix><op> on numpy arrays (passed by pointer) and ints/floats;
    arrays are modified in place as the C function does."""
    args = [a.ctypes.data_as(ctypes.c_void_p) if isinstance(a, np.ndarray) else a for a in arrays_and_sizes]
    getattr(lib, prefix + op)(*args)


def oracle_dequant(lib, raw, n_rows, n_cols, qtype=Q4_K, fn="fh3_oracle_dequant"):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.zeros((n_rows, n_cols), dtype=np.float32)
    rb = raw.size // n_rows
    f = getattr(lib, fn)
    for r in range(n_rows):
        f(qtype, raw[r * rb:].ctypes.data_as(ctypes.c_void_p),
          out[r].ctypes.data_as(ctypes.c_void_p), n_cols)
    return out


def matmul_with(lib, fn, raw, K, N, x, bias=None, qtype=Q4_K):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M = x.shape[0]
    y = np.full((M, N), np.nan, dtype=np.float32)
    w = OracleW(qtype, K, N, raw.ctypes.data)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    getattr(lib, fn)(ctypes.byref(w), _ptr(x), _ptr(y), M, None if b is None else _ptr(b))
    return y


def oracle_matmul(lib, raw, K, N, x, bias=None):
    return matmul_with(lib, "fh3_oracle_matmul", raw, K, N, x, bias)


def oracle_matmul_rows(lib, raw, K, N, x, o_begin, o_end, bias=None):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M = x.shape[0]
    y = np.full((M, N), np.nan, dtype=np.float32)
    w = OracleW(Q4_K, K, N, raw.ctypes.data)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib.fh3_oracle_matmul_rows(ctypes.byref(w), _ptr(x), _ptr(y), M,
                               None if b is None else _ptr(b), o_begin, o_end)
    return y


def read_q4k_fixture():
    """tests/golden/Q4_K.bin: <IIII> type, rows, cols, raw_nbytes; raw; fp32 dequant
    (layout written by the reference's tools/emit_quant_fixtures.py:84-91)."""
    with open(os.path.join(GOLDEN, "Q4_K.bin"), "rb") as f:
        buf = f.read()
    t, rows, cols, nraw = struct.unpack_from("<IIII", buf, 0)
    raw = np.frombuffer(buf, dtype=np.uint8, count=nraw, offset=16).copy()
    ref = np.frombuffer(buf, dtype=np.float32, count=rows * cols, offset=16 + nraw).reshape(rows, cols).copy()
    return t, rows, cols, raw, ref


# Type ids (reference include/fh3/fh3.h:23-39) -> (block length, block bytes,
# byte offsets of the fp16 scale fields).  The decodable set of
# src/core/fh3_quant.c:284-318.
QTYPES = {
    "F16": (1, 1, 2, ()),
    "BF16": (30, 1, 2, ()),
    "Q8_0": (8, 32, 34, (0,)),
    "Q2_K": (10, 256, 84, (80, 82)),
    "Q3_K": (11, 256, 110, (108,)),
    "Q4_K": (12, 256, 144, (0, 2)),
    "Q5_K": (13, 256, 176, (0, 2)),
    "Q6_K": (14, 256, 210, (208,)),
}


def read_quant_fixture(name):
    """tests/golden/quant/<name>.bin (Q4_K: tests/golden/Q4_K.bin), same layout
    as read_q4k_fixture."""
    path = os.path.join(GOLDEN, "Q4_K.bin" if name == "Q4_K" else os.path.join("quant", name + ".bin"))
    with open(path, "rb") as f:
        buf = f.read()
    t, rows, cols, nraw = struct.unpack_from("<IIII", buf, 0)
    raw = np.frombuffer(buf, dtype=np.uint8, count=nraw, offset=16).copy()
    ref = np.frombuffer(buf, dtype=np.float32, count=rows * cols, offset=16 + nraw).reshape(rows, cols).copy()
    return t, rows, cols, raw, ref


def random_blocks(rng, name, rows, cols, scale_lo=-14, scale_hi=-4, finite=True):
    """Random rows of format `name`: uniform random bytes, then every fp16 scale
    field overwritten with +-2^e * (1 + m/1024), e in [scale_lo, scale_hi]
    (`finite`), so the decoded values are finite and of DiT-like magnitude.
    F16/BF16 payloads get finite halves of magnitude 2^-8..2^8."""
    t, bl, bb, scale_offs = QTYPES[name]
    nblk = cols // bl
    raw = rng.integers(0, 256, size=(rows, nblk, bb), dtype=np.uint8)
    if name in ("F16", "BF16"):
        v = (rng.standard_normal((rows, cols)) * 4.0).astype(np.float32)
        bits = v.astype(np.float16).view(np.uint16) if name == "F16" else (v.view(np.uint32) >> 16).astype(np.uint16)
        return bits.reshape(rows, -1).view(np.uint8).reshape(-1).copy()
    for off in scale_offs:
        e = rng.integers(scale_lo, scale_hi + 1, size=(rows, nblk))
        m = rng.integers(0, 1024, size=(rows, nblk))
        s = rng.integers(0, 2, size=(rows, nblk))
        h = np.asarray(np.ldexp(1.0 + m / 1024.0, e) * np.where(s, -1.0, 1.0), dtype=np.float16)
        raw[:, :, off:off + 2] = h.view(np.uint8).reshape(rows, nblk, 2) if finite else raw[:, :, off:off + 2]
    return raw.reshape(-1)


def read_matmul_fixture():
    """tests/golden/matmul_ref.bin: <IIIII> type, in, out, n_tok, w_bytes; W; X; bias;
    y_ref computed in fp64 (reference tools/emit_quant_fixtures.py:125-132)."""
    with open(os.path.join(GOLDEN, "matmul_ref.bin"), "rb") as f:
        buf = f.read()
    t, K, N, M, wb = struct.unpack_from("<IIIII", buf, 0)
    off = 20
    raw = np.frombuffer(buf, dtype=np.uint8, count=wb, offset=off).copy(); off += wb
    x = np.frombuffer(buf, dtype=np.float32, count=M * K, offset=off).reshape(M, K).copy(); off += 4 * M * K
    bias = np.frombuffer(buf, dtype=np.float32, count=N, offset=off).copy(); off += 4 * N
    y = np.frombuffer(buf, dtype=np.float32, count=M * N, offset=off).reshape(M, N).copy()
    return t, K, N, M, raw, x, bias, y


def rel_fro(y, yref):
    y = np.asarray(y, dtype=np.float64)
    yref = np.asarray(yref, dtype=np.float64)
    return float(np.linalg.norm(y - yref) / np.linalg.norm(yref))


REF_IO_SO = os.path.join(ROOT, "oracle", "_ref", "libfh3_ref_io.so")
REF_TRUNK_BYTES = 1 << 16  # generous room for the reference's struct Fh3Trunk


class TrunkStats(ctypes.Structure):
    """Layout of Fh3TrunkStats (reference include/fh3/fh3.h:134-140)."""
    _fields_ = [("hits", ctypes.c_uint64), ("misses", ctypes.c_uint64), ("bytes_read", ctypes.c_uint64),
                ("read_s", ctypes.c_double), ("wait_s", ctypes.c_double)]


def load_ref_io():
    """The reference's own fh3_pack.c/fh3_trunk.c built by oracle/Makefile, or None."""
    if not os.path.exists(REF_IO_SO):
        return None
    lib = ctypes.CDLL(REF_IO_SO)
    lib.fh3_trunk_open.restype = ctypes.c_int
    lib.fh3_trunk_open.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_void_p]
    lib.fh3_trunk_close.restype = None
    lib.fh3_trunk_close.argtypes = [ctypes.c_void_p]
    lib.fh3_trunk_prefetch.restype = None
    lib.fh3_trunk_prefetch.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.fh3_trunk_acquire.restype = ctypes.c_void_p
    lib.fh3_trunk_acquire.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.fh3_trunk_stats.restype = TrunkStats
    lib.fh3_trunk_stats.argtypes = [ctypes.c_void_p]
    return lib


def write_pattern_pack(path, sizes, pattern_base=0xA0, truncate_last=0):
    """A synthetic FH3P pack whose layer L is sizes[L] bytes of (pattern_base + L),
    laid out as the reference's trunk test writes it (tests/unit/test_trunk.c:45-131:
    index at 4096, descriptors of the full in-memory size, nine F32 tensor
    descriptors per layer).  truncate_last cuts that many bytes off the file end."""
    from fasth3inc_amd import fh3 as F
    n = len(sizes)
    hdr = F.Fh3PackHeader()
    hdr.magic, hdr.version, hdr.num_layers, hdr.layer_alignment = F.FH3_PACK_MAGIC, F.FH3_PACK_VERSION, n, 4096
    hdr.index_offset = 4096
    hdr.index_bytes = n * ctypes.sizeof(F.Fh3PackLayerDesc)
    data_off = (hdr.index_offset + hdr.index_bytes + 4095) // 4096 * 4096
    hdr.data_offset = data_off
    hdr.total_bytes = data_off + sum(sizes)
    descs = (F.Fh3PackLayerDesc * n)()
    at = data_off
    for L, sz in enumerate(sizes):
        descs[L].file_offset, descs[L].size_bytes, descs[L].n_tensors = at, sz, 9
        for t in range(9):
            td = descs[L].tensors[t]
            td.name = b"tensor_%d_%d" % (L, t)
            td.type, td.n_dims = F32, 2
            td.shape[0] = td.shape[1] = 64
            td.offset_in_layer, td.size_bytes = t * 4096, 4096
            td.in_dim = td.out_dim = 64
        at += sz
    with open(path, "wb") as f:
        f.write(bytes(hdr))
        f.write(b"\0" * (hdr.index_offset - ctypes.sizeof(hdr)))
        f.write(bytes(descs))
        f.write(b"\0" * (data_off - hdr.index_offset - hdr.index_bytes))
        for L, sz in enumerate(sizes):
            f.write(bytes([(pattern_base + L) & 0xFF]) * sz)
        if truncate_last:
            f.truncate(hdr.total_bytes - truncate_last)
    return path


def random_q4k(rng, n_rows, K, d_range=(0.1, 0.45), dmin_range=(0.02, 0.06)):
    """Random Q4_K bytes with normal positive fp16 d/dmin (the reference fixtures'
    recipe, tools/emit_quant_fixtures.py:113-119) -- every 6-bit scale/min and
    nibble pattern is reachable."""
    nsb = n_rows * (K // 256)
    blocks = rng.integers(0, 256, size=(nsb, 144), dtype=np.uint8)
    d = rng.uniform(*d_range, size=nsb).astype(np.float16)
    dm = rng.uniform(*dmin_range, size=nsb).astype(np.float16)
    blocks[:, 0:2] = d.view(np.uint8).reshape(nsb, 2)
    blocks[:, 2:4] = dm.view(np.uint8).reshape(nsb, 2)
    return blocks.reshape(-1)
