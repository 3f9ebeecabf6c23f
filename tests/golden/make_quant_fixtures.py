"""Copy the reference's dequantisation golden fixtures into tests/golden/quant/.

Each file (reference tests/fixtures/quant/<TYPE>.bin, written by its
tools/emit_quant_fixtures.py from gguf-py 0.19.0 `dequantize`) is data:
16-byte header <IIII> type, rows, cols, raw_nbytes; the raw blocks; then the
rows*cols fp32 dequantised values.  Q4_K.bin already lives in tests/golden/.

    python tests/golden/make_quant_fixtures.py [/root/reference]
"""
import os
import shutil
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
TYPES = ("F16", "BF16", "Q8_0", "Q2_K", "Q3_K", "Q5_K", "Q6_K")


def main(ref):
    src = os.path.join(ref, "tests", "fixtures", "quant")
    dst = os.path.join(HERE, "quant")
    os.makedirs(dst, exist_ok=True)
    for t in TYPES:
        shutil.copyfile(os.path.join(src, t + ".bin"), os.path.join(dst, t + ".bin"))
    print("copied %d fixtures into %s" % (len(TYPES), dst))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
