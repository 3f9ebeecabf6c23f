"""Write the FH3P pack fixtures used by tests/test_trunk.py.

Reads two data files the reference's own pack test uses
(tests/unit/test_pack.c:47-165):
  tests/fixtures/pack/tiny_trunk.bin  a 2-layer FH3P pack, copied verbatim
  tests/fixtures/pack/tiny_dit.gguf   the GGUF it was packed from
and writes
  tiny_trunk.bin       (copy)
  pack_vectors.json    per tensor blocks.{L}.<suffix>: ggml type, dims,
                       byte count and sha256 of its data in the GGUF
so that the pack views can be checked against the original tensor bytes
without the GGUF reader.  The GGUF is parsed here as data (GGUF v2/v3 layout:
header, key/value section, tensor infos, data section at general.alignment).

    python tests/golden/make_pack_vectors.py [/root/reference]
"""
import hashlib
import json
import os
import shutil
import struct
import sys

HERE = os.path.dirname(os.path.abspath(__file__))

# bytes per block, elements per block (ggml type table)
BLOCK = {0: (4, 1), 1: (2, 1), 2: (18, 32), 3: (20, 32), 6: (22, 32), 7: (24, 32), 8: (34, 32),
         9: (36, 32), 10: (84, 256), 11: (110, 256), 12: (144, 256), 13: (176, 256), 14: (210, 256),
         15: (292, 256), 30: (2, 1)}
SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


class Reader:
    def __init__(self, data):
        self.d, self.p = data, 0

    def take(self, fmt):
        v = struct.unpack_from(fmt, self.d, self.p)
        self.p += struct.calcsize(fmt)
        return v[0]

    def string(self):
        n = self.take("<Q")
        s = self.d[self.p:self.p + n].decode("utf-8")
        self.p += n
        return s

    def value(self, vt):
        if vt in SCALAR:
            return self.take(SCALAR[vt])
        if vt == 8:
            return self.string()
        if vt == 9:
            et, n = self.take("<I"), self.take("<Q")
            return [self.value(et) for _ in range(n)]
        raise ValueError("unknown GGUF value type %d" % vt)


def parse_gguf(path):
    data = open(path, "rb").read()
    r = Reader(data)
    if data[:4] != b"GGUF":
        raise ValueError("not a GGUF file")
    r.p = 4
    version = r.take("<I")
    if version < 2:
        raise ValueError("GGUF v%d not supported" % version)
    n_tensors, n_kv = r.take("<Q"), r.take("<Q")
    kv = {}
    for _ in range(n_kv):
        key = r.string()
        kv[key] = r.value(r.take("<I"))
    infos = []
    for _ in range(n_tensors):
        name = r.string()
        nd = r.take("<I")
        dims = [r.take("<Q") for _ in range(nd)]
        qtype, off = r.take("<I"), r.take("<Q")
        infos.append((name, dims, qtype, off))
    align = int(kv.get("general.alignment", 32))
    base = (r.p + align - 1) // align * align
    out = {}
    for name, dims, qtype, off in infos:
        bb, be = BLOCK[qtype]
        rows = 1
        for d in dims[1:]:
            rows *= d
        nbytes = (dims[0] + be - 1) // be * bb * rows
        blob = data[base + off:base + off + nbytes]
        if len(blob) != nbytes:
            raise ValueError("%s: data runs past the end of the file" % name)
        out[name] = {"type": qtype, "dims": dims, "nbytes": nbytes, "sha256": hashlib.sha256(blob).hexdigest()}
    return out


def main(ref):
    src = os.path.join(ref, "tests", "fixtures", "pack")
    shutil.copyfile(os.path.join(src, "tiny_trunk.bin"), os.path.join(HERE, "tiny_trunk.bin"))
    tensors = parse_gguf(os.path.join(src, "tiny_dit.gguf"))
    blocks = {k: v for k, v in tensors.items() if k.startswith("blocks.")}
    with open(os.path.join(HERE, "pack_vectors.json"), "w") as f:
        json.dump({"source": "tests/fixtures/pack/tiny_dit.gguf", "tensors": blocks}, f, indent=1, sort_keys=True)
    print("wrote tiny_trunk.bin and %d tensor digests" % len(blocks))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
