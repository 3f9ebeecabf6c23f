"""A C99 program calls the library (tests/c/fh3_c_caller.c, built by
fasth3inc_amd/build.py against include/fh3/*.h and linked to libfh3hip.so):
the reference's test_matmul.c checks on its own fixture, the calls of its
bench_matmul.c with an output check, the DiT's run-once patch projections,
and the trunk held by value on the stack as the reference CLI holds it."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "c", "fh3_c_caller")


def _run(*args):
    if not os.path.exists(EXE):
        pytest.fail("tests/c/fh3_c_caller is not built (python -m fasth3inc_amd.build)")
    print("case: fh3_c_caller %s" % " ".join(args), flush=True)
    r = subprocess.run([EXE] + list(args), capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    return r.stdout


def test_c_caller_matmul_ref():
    out = _run("matmul_ref", os.path.join(ROOT, "tests", "golden", "matmul_ref.bin"))
    assert out.count("PASS") == 3


@pytest.mark.parametrize("n_tok", ["1024", "16"])
def test_c_caller_bench_matmul(n_tok):
    out = _run("bench", n_tok, "3")
    assert "PASS bench_matmul output" in out


def test_c_caller_dit_patch_projections():
    """src/model/fh3_dit.c:352-353 replayed by a C99 caller: 32- and 96-value
    F16 rows with bias written into h behind the text rows."""
    out = _run("patch", "6", "130", "2880")
    assert out.count("PASS patch projection") == 2


def test_c_caller_trunk_by_value():
    out = _run("trunk", os.path.join(ROOT, "tests", "golden", "tiny_trunk.bin"))
    assert out.count("PASS") == 2
