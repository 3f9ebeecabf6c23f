"""The C-ABI library loads and exports every entry point include/fh3/*.h
declares (no compute calls: these run without a GPU)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include", "fh3")


def declared_functions():
    names = set()
    for fn in sorted(os.listdir(INC)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(INC, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        text = re.sub(r"typedef[^;]*;", "", text)
        text = re.sub(r"#[^\n]*", "", text)
        for m in re.finditer(r"\b(fh3_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_headers_declare_entry_points():
    names = declared_functions()
    for must in ("fh3_row_bytes", "fh3_dequant", "fh3_matmul", "fh3_matmul_scalar", "fh3_matmul_avx2",
                 "fh3_hip_matmul_dev", "fh3_hip_dequant_dev", "fh3_hip_init"):
        assert must in names


def test_library_exports_every_declared_symbol(fh3):
    lib = fh3.lib()
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def _dynsyms(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib], capture_output=True, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if len(l.split()) == 3 and l.split()[1] in "TtWw"}


LIB = os.path.join(ROOT, "fasth3inc_amd", "lib", "libfh3hip.so")


def test_library_exports_exactly_the_headers():
    """Nothing beyond the header API is exported: no kernel launcher
    (fh3k_*), no internal helper (fh3i_*)."""
    assert _dynsyms(LIB) == declared_functions()


def test_library_calls_between_its_own_functions_are_not_interposable():
    """The library's calls to its own exported functions (fh3_matmul ->
    fh3_hip_matmul_dev, fh3_trunk_acquire_dev -> fh3_trunk_acquire, ...) bind
    inside it (-Bsymbolic): no PLT slot names a symbol the library defines, so
    a program that also defines fh3_trunk_acquire or fh3_pack_open (the
    reference's fh3_core) cannot redirect them."""
    rel = subprocess.run(["readelf", "-r", "--wide", LIB], capture_output=True, text=True, check=True).stdout
    own = declared_functions()
    slots = set()
    for line in rel.splitlines():
        parts = line.split()
        if len(parts) >= 5 and "JUMP_SLOT" in parts[2]:
            slots.add(parts[4].split("@")[0])
    assert not (slots & own), sorted(slots & own)


def test_binding_table_matches_headers(fh3):
    declared = declared_functions()
    extra = [n for n in fh3.SIGNATURES if n not in declared]
    assert not extra, extra
    undeclared = [n for n in declared if n not in fh3.SIGNATURES]
    assert not undeclared, undeclared


def test_library_is_gfx950_only_and_has_no_cpu_matmul():
    lib = os.path.join(ROOT, "fasth3inc_amd", "lib", "libfh3hip.so")
    out = subprocess.run(["nm", "-D", "--defined-only", lib], capture_output=True, text=True).stdout
    # no oracle symbols leak into the product
    assert "fh3_oracle" not in out
    bundle = subprocess.run(["strings", "-n", "8", lib], capture_output=True, text=True).stdout
    assert "gfx950" in bundle


def test_row_bytes_table(fh3):
    """Same table as reference src/core/fh3_quant.c:14-34."""
    rb = fh3.row_bytes
    assert rb(fh3.FH3_QUANT_Q4_K, 5120) == 2880
    assert rb(fh3.FH3_QUANT_Q4_K, 4096) == 2304
    assert rb(fh3.FH3_QUANT_Q4_K, 13824) == 7776
    assert rb(fh3.FH3_QUANT_Q4_K, 1) == 144
    assert rb(fh3.FH3_QUANT_F32, 10) == 40
    assert rb(fh3.FH3_QUANT_Q6_K, 512) == 420
    assert rb(fh3.FH3_QUANT_Q4_K, 0) == 0 and rb(fh3.FH3_QUANT_Q4_K, -5) == 0
    assert rb(99, 256) == 0


def test_row_bytes_matches_reference_build(fh3, ref):
    for t in (0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 30, 99):
        for n in (1, 31, 32, 255, 256, 5120, 13824):
            assert fh3.row_bytes(t, n) == ref.fh3_row_bytes(t, n), (t, n)


def test_matmul_path_selection(fh3):
    """Kernel family per shape (host-side decision, no GPU call): the int8
    kernel takes one to four tokens while its window fits (K <= 20480 for one
    or two tokens, K <= 12288 for three or four), the persistent fp16 sweep up
    to 16 tokens for 512 <= K <= 32768 and up to 64 from K = 5120 (long rows
    in K slices), the fp16 GEMV up to 64 tokens on shorter rows, the
    GEMM above; a forced path that cannot take a shape falls back to the
    automatic choice."""
    F = fh3
    G8, SK, GM, SW = F.PATH_GEMV8, F.PATH_SKINNY, F.PATH_GEMM, F.PATH_SWEEP
    assert F.matmul_path(1, 5120) == G8 and F.matmul_path(2, 5120) == G8
    assert F.matmul_path(1, 20480) == G8 and F.matmul_path(1, 20736) == SW
    assert F.matmul_path(2, 20480) == G8 and F.matmul_path(2, 20736) == SW
    assert F.matmul_path(3, 12288) == G8 and F.matmul_path(4, 12288) == G8 and F.matmul_path(4, 12544) == SW
    assert F.matmul_path(4, 13824) == SW and F.matmul_path(1, 25600) == SW and F.matmul_path(1, 200) == SK
    assert F.matmul_path(5, 5120) == SW and F.matmul_path(16, 5120) == SW and F.matmul_path(16, 6144) == SW
    assert F.matmul_path(16, 6400) == SW and F.matmul_path(16, 8192) == SW and F.matmul_path(16, 32768) == SW
    assert F.matmul_path(5, 256) == SK and F.matmul_path(17, 5120) == SW and F.matmul_path(32, 25600) == SW
    assert F.matmul_path(33, 5120) == SW and F.matmul_path(64, 5120) == SW and F.matmul_path(64, 256) == SK
    assert F.matmul_path(17, 4864) == SK and F.matmul_path(64, 4096) == SK and F.matmul_path(16, 4096) == SW
    assert F.matmul_path(17, 2560) == SK and F.matmul_path(64, 512) == SK and F.matmul_path(33, 2816) == SK
    assert F.matmul_path(65, 5120) == GM
    MD = F.PATH_MIDM
    assert F.matmul_path(33, 8192) == SW and F.matmul_path(64, 13824) == SW and F.matmul_path(17, 8192) == SW
    assert F.matmul_path(16, 13824) == SW and F.matmul_path(33, 7936) == SW and F.matmul_path(65, 13824) == GM
    try:
        F.set_path(MD)
        assert F.matmul_path(1, 5120) == MD and F.matmul_path(64, 256) == MD and F.matmul_path(65, 5120) == GM
        F.set_path(SK)
        assert F.matmul_path(1, 5120) == SK
        F.set_path(G8)
        assert F.matmul_path(4, 5120) == G8 and F.matmul_path(5, 5120) == SW
        F.set_path(SW)
        assert F.matmul_path(1, 5120) == SW and F.matmul_path(16, 512) == SW
        assert F.matmul_path(65, 5120) == GM and F.matmul_path(64, 8192) == SW and F.matmul_path(16, 256) == SK
        F.set_path(GM)
        assert F.matmul_path(1, 5120) == GM
    finally:
        F.set_path(F.PATH_AUTO)
