"""Build recipe for libfh3hip.so (gfx950) and the CPU oracle.

    python -m fasth3inc_amd.build          # build everything in-tree
    python -m fasth3inc_amd.build --check  # also print kernel resource usage

C99 host files are compiled with gcc (-std=gnu99, OpenMP), HIP sources with
hipcc for gfx950 only, and linked into fasth3inc_amd/lib/libfh3hip.so; the
calibration program (MFMA and HBM rates) goes to fasth3inc_amd/lib/fh3_calib.  The
oracle (oracle/libfh3_oracle.so) and, when the reference tree is present, the
reference build (oracle/_ref/libfh3_ref.so) are made by oracle/Makefile.
"""
import argparse
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INC = os.path.join(ROOT, "include")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libfh3hip.so")
OBJ = os.path.join(ROOT, "_build", "obj")
REFERENCE = "/root/reference"

HIPCC = os.environ.get("HIPCC", "hipcc")
CC = os.environ.get("CC", "gcc")

C_SOURCES = ["fh3_synth.c", "fh3_pack.c", "fh3_trunk.c"]
HIP_SOURCES = ["fh3_kernels.hip", "fh3_attn.hip", "fh3_hip.cpp"]

C_FLAGS = ["-std=gnu99", "-O3", "-fPIC", "-fopenmp", "-Wall", "-Wextra", "-D_GNU_SOURCE",
           "-ffp-contract=off", "-I" + INC, "-I" + CSRC]
# -packed-fp32-ops: no v_pk_*_f32 in device code (host pass warns it does not know the feature)
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
             "-Wall", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I" + INC, "-I" + CSRC]


def _run(cmd, quiet=False):
    if not quiet:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if out.strip():
        print(out, flush=True)
    if res.returncode != 0:
        raise RuntimeError("build step failed: " + " ".join(cmd))
    return out


def build_oracle(quiet=False):
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], quiet)
    if os.path.isdir(os.path.join(REFERENCE, "src", "core")):
        _run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref", "REF=" + REFERENCE], quiet)


def build_lib(check=False, quiet=False):
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    objs = []
    for src in C_SOURCES:
        path = os.path.join(CSRC, src)
        if not os.path.exists(path):
            continue
        obj = os.path.join(OBJ, src + ".o")
        _run([CC] + C_FLAGS + ["-c", path, "-o", obj], quiet)
        objs.append(obj)
    for src in HIP_SOURCES:
        obj = os.path.join(OBJ, src + ".o")
        extra = ["-Rpass-analysis=kernel-resource-usage"] if (check and src.endswith(".hip")) else []
        _run([HIPCC] + HIP_FLAGS + extra + ["-c", os.path.join(CSRC, src), "-o", obj], quiet)
        objs.append(obj)
    tmp = LIB + ".tmp"
    # exports: exactly the header API (libfh3hip.map); -Bsymbolic binds the
    # library's calls between its own exported functions inside it
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs +
         ["-lgomp", "-lpthread", "-Wl,--no-undefined", "-Wl,-soname,libfh3hip.so", "-Wl,-Bsymbolic",
          "-Wl,--version-script=" + os.path.join(CSRC, "libfh3hip.map")], quiet)
    os.replace(tmp, LIB)
    return LIB


CALIB_SRC = os.path.join(CSRC, "fh3_calib.hip")
CALIB = os.path.join(LIBDIR, "fh3_calib")


def build_calib(quiet=False):
    """The calibration program (fp16 / bf16 / int8 MFMA rates and the clock
    they imply; the load-only HBM stream), which the profiles quote beside the
    kernels."""
    os.makedirs(LIBDIR, exist_ok=True)
    _run([HIPCC] + HIP_FLAGS + [CALIB_SRC, "-o", CALIB], quiet)
    return CALIB


C_CALLER_SRC = os.path.join(ROOT, "tests", "c", "fh3_c_caller.c")
C_CALLER = os.path.join(ROOT, "tests", "c", "fh3_c_caller")


def build_c_caller(quiet=False):
    """The C99 caller the GPU tests run: compiled against include/fh3/*.h
    only and linked to the library, as a C program of the reference would be."""
    _run([CC, "-std=gnu99", "-O2", "-Wall", "-Wextra", "-Werror", "-D_GNU_SOURCE", "-I" + INC, C_CALLER_SRC,
          "-o", C_CALLER, "-L" + LIBDIR, "-lfh3hip", "-Wl,-rpath,$ORIGIN/../../fasth3inc_amd/lib", "-lm"], quiet)
    return C_CALLER


def build(check=False, quiet=False):
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    build_oracle(quiet)
    lib = build_lib(check, quiet)
    build_c_caller(quiet)
    build_calib(quiet)
    return lib


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--check", action="store_true", help="print kernel resource usage")
    args = ap.parse_args()
    print(build(check=args.check))
    sys.exit(0)
