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
    return lib


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
    return lib


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
