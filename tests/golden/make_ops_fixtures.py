"""Copy the reference's elementwise-op and attention golden fixtures into
tests/golden/ops/.

The reference's tests/fixtures/ops/*.bin were written by its
tools/emit_fixtures.py from a numpy model of each op; they are data (inputs
and expected outputs):

  rmsnorm.bin        <IIf> n, dim, eps; x[n][dim], w[dim], ref[n][dim]
  modulate.bin       <II> n, dim; x, shift, scale, ref  (each [n][dim])
  swiglu.bin         <II> n, F; in[n][2F], ref[n][F]
  gate_residual.bin  <II> n, dim; h, gate, y, ref  (each [n][dim])
  rope3.bin          <IIII> n, heads, head_dim, rot_dim; x[n][heads][hd],
                     cos[n][rot], sin[n][rot], ref[n][heads][hd]

These five are copied unchanged.  attention.bin (n = 777, heads = 4,
hd = 128, 6.3 MB) is cut down, exactly, to what two heads and every fourth
query need: heads are independent, and one query's output depends only on
its own q row and all k/v rows of its head.  attention_sub.bin holds

  <IIII> n (keys), heads (2), hd, nq; int32 head_idx[2]; int32 q_idx[nq];
  q[nq][2][hd], k[n][2][hd], v[n][2][hd], ref[nq][2][hd]

The VSA fixtures (reference tests/fixtures/vsa/*.bin: a 44-byte header
<IIIIIIIIIfI> n, num_text, num_audio, num_video, grid_t, grid_h, grid_w,
heads, head_dim, sparsity, has_gate; then q, k, v, [gate], ref, each
[n][heads][head_dim]) are cut to heads 0 and 3 (heads are independent in
every step of the call) and written to tests/golden/vsa/<name>.bin with the
same header (heads = 2).

    python tests/golden/make_ops_fixtures.py [/root/reference]
"""
import os
import shutil
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
COPY = ("rmsnorm", "modulate", "swiglu", "gate_residual", "rope3")
HEADS = (0, 3)
QSTEP = 4
VSA = ("vsa_n784", "vsa_padded", "vsa_sparsity0")


def main(ref):
    src = os.path.join(ref, "tests", "fixtures", "ops")
    dst = os.path.join(HERE, "ops")
    os.makedirs(dst, exist_ok=True)
    for name in COPY:
        shutil.copyfile(os.path.join(src, name + ".bin"), os.path.join(dst, name + ".bin"))
    with open(os.path.join(src, "attention.bin"), "rb") as f:
        n, heads, hd = struct.unpack("<III", f.read(12))
        arr = np.frombuffer(f.read(), dtype="<f4").reshape(4, n, heads, hd)
    q, k, v, r = arr
    qi = np.arange(0, n, QSTEP, dtype=np.int32)
    hi = np.array(HEADS, dtype=np.int32)
    with open(os.path.join(dst, "attention_sub.bin"), "wb") as f:
        f.write(struct.pack("<IIII", n, len(HEADS), hd, len(qi)))
        f.write(hi.tobytes())
        f.write(qi.tobytes())
        for a in (q[qi][:, hi], k[:, hi], v[:, hi], r[qi][:, hi]):
            f.write(np.ascontiguousarray(a, dtype="<f4").tobytes())
    print("copied %d fixtures and attention_sub.bin (%d queries, heads %s) into %s"
          % (len(COPY), len(qi), HEADS, dst))
    vsrc = os.path.join(ref, "tests", "fixtures", "vsa")
    vdst = os.path.join(HERE, "vsa")
    os.makedirs(vdst, exist_ok=True)
    for name in VSA:
        with open(os.path.join(vsrc, name + ".bin"), "rb") as f:
            hdr = list(struct.unpack("<IIIIIIIIIfI", f.read(44)))
            n, heads, hd, has_gate = hdr[0], hdr[7], hdr[8], hdr[10]
            cnt = 5 if has_gate else 4
            arr = np.frombuffer(f.read(), dtype="<f4").reshape(cnt, n, heads, hd)
        hdr[7] = len(HEADS)
        with open(os.path.join(vdst, name + ".bin"), "wb") as f:
            f.write(struct.pack("<IIIIIIIIIfI", *hdr))
            for a in arr:
                f.write(np.ascontiguousarray(a[:, list(HEADS)], dtype="<f4").tobytes())
    print("wrote %d VSA fixtures (heads %s) into %s" % (len(VSA), HEADS, vdst))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
