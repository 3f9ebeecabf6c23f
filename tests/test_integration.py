"""The drop-in at link level, on the CPU (no compute calls).

The integration recipe is built by `make -C oracle integration` from the
reference's own sources where they lie: fh3_core with
the CPU matmul, dequant, attention and pack reader renamed and the trunk
streamer left out, then the reference's CLI main and its bench_matmul linked
against that archive and libfh3hip.so.  Checked here:
  - no symbol is defined twice: nothing the renamed archive defines is
    exported by the library;
  - every fh3_* the reference's CLI and benchmark take from outside the
    archive is exported by the library (the products, dequant, attention,
    pack reader, trunk streamer and memory plan);
  - the structs callers hold by value (Fh3Trunk on the CLI's stack, Fh3Pack,
    Fh3File, Fh3W, Fh3LayerView, the pack descriptors) have the reference's
    size and field offsets.
Skipped where the reference tree is absent.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
INT = os.path.join(ROOT, "oracle", "_ref", "integration")
LIB = os.path.join(ROOT, "fasth3inc_amd", "lib", "libfh3hip.so")

pytestmark = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src")), reason="reference tree absent")


@pytest.fixture(scope="module")
def built():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "integration", "REF=" + REF], check=True,
                   stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    return INT


def _syms(args, path):
    out = subprocess.run(["nm"] + args + [path], capture_output=True, text=True, check=True).stdout
    return out.splitlines()


def _defined_globals(path):
    return {l.split()[-1] for l in _syms(["-g", "--defined-only"], path) if len(l.split()) == 3}


def _exports():
    return {l.split()[-1] for l in _syms(["-D", "--defined-only"], LIB) if len(l.split()) == 3}


def _undefined_fh3(path):
    return {l.split()[-1] for l in _syms(["-D", "--undefined-only"], path) if l.split()[-1].startswith("fh3_")}


def test_no_symbol_defined_twice(built):
    core = _defined_globals(os.path.join(built, "libfh3_core.a"))
    assert "fh3_cpu_matmul" in core and "fh3_dit_forward" in core
    clash = core & _exports()
    assert not clash, sorted(clash)


@pytest.mark.parametrize("exe", ["fh3", "bench_matmul"])
def test_reference_programs_take_the_layer_from_the_library(built, exe):
    need = _undefined_fh3(os.path.join(built, exe))
    assert "fh3_matmul" in need
    if exe == "fh3":
        assert {"fh3_trunk_open", "fh3_trunk_acquire", "fh3_trunk_prefetch", "fh3_pack_open",
                "fh3_vsa_attention", "fh3_dequant"} <= need
    missing = need - _exports()
    assert not missing, sorted(missing)


def test_struct_layouts_match_the_reference(built, tmp_path):
    exe = str(tmp_path / "layout_ours")
    subprocess.run(["gcc", "-std=gnu99", "-D_GNU_SOURCE", "-I" + os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "c", "layout_probe.c"), "-o", exe], check=True)
    ours = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    want = open(os.path.join(built, "layout_reference.txt")).read()
    assert "sizeof Fh3Trunk" in want
    assert ours == want
