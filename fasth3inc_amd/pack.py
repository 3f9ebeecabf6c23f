"""Writer of FH3P packs (the format fh3_pack_open reads; reference layout
src/io/fh3_pack.h:41-71, writer tools/pack_dit.py:110-160).

  [0, 128)           header
  [4096, ...)        one 24 + 168*n_tensors byte descriptor per layer
  data_offset        layer runs, each 4096-aligned and padded to 4096;
                     tensors 32-aligned inside a run, in the run order
                     qkv, gate_compress, out, fc1, fc2, norm1, norm2, q_norm, k_norm

Layers are produced one at a time by a callback, so packs larger than host
memory can be written.  Used for synthetic trunks (tests, benchmark).
"""
import ctypes
import os

import numpy as np

from . import fh3

INDEX_OFFSET = 4096
RUN_ALIGN = fh3.FH3_PACK_ALIGNMENT
TENSOR_ALIGN = 32
DESC_HEAD = 24


def _up(n, a):
    return (n + a - 1) // a * a


class TensorSpec:
    """One tensor of every layer: GGUF-style dims (ne0 = in, ne1 = out)."""

    def __init__(self, suffix, qtype, ne0, ne1=1):
        self.suffix, self.qtype, self.ne0, self.ne1 = suffix, qtype, ne0, ne1
        self.nbytes = fh3.row_bytes(qtype, ne0) * ne1


def layout(specs):
    """(offset_in_layer per tensor, run bytes)."""
    offs, at = [], 0
    for s in specs:
        at = _up(at, TENSOR_ALIGN)
        offs.append(at)
        at += s.nbytes
    return offs, _up(at, RUN_ALIGN)


def write_pack(path, n_layers, specs, make_layer, name_fmt="blocks.{L}.{suffix}"):
    """Write an n_layers pack whose layers hold `specs`; make_layer(L) returns
    one uint8 array (or bytes) per spec."""
    offs, run = layout(specs)
    nt = len(specs)
    desc_bytes = DESC_HEAD + nt * ctypes.sizeof(fh3.Fh3PackTensorDesc)
    index_bytes = n_layers * desc_bytes
    data_off = _up(INDEX_OFFSET + index_bytes, RUN_ALIGN)

    hdr = fh3.Fh3PackHeader()
    hdr.magic, hdr.version, hdr.num_layers = fh3.FH3_PACK_MAGIC, fh3.FH3_PACK_VERSION, n_layers
    hdr.layer_alignment = RUN_ALIGN
    hdr.index_offset, hdr.index_bytes = INDEX_OFFSET, index_bytes
    hdr.data_offset, hdr.total_bytes = data_off, data_off + n_layers * run

    index = bytearray()
    for L in range(n_layers):
        ld = fh3.Fh3PackLayerDesc()
        ld.file_offset, ld.size_bytes, ld.n_tensors = data_off + L * run, run, nt
        for i, s in enumerate(specs):
            td = ld.tensors[i]
            td.name = name_fmt.format(L=L, suffix=s.suffix).encode()[:63]
            td.type, td.n_dims = s.qtype, 2 if s.ne1 > 1 else 1
            td.shape[0], td.shape[1] = s.ne0, s.ne1
            td.offset_in_layer, td.size_bytes = offs[i], s.nbytes
            td.in_dim, td.out_dim = s.ne0, s.ne1
        index += bytes(ld)[:desc_bytes]

    with open(path, "wb") as f:
        f.write(bytes(hdr))
        f.write(b"\0" * (INDEX_OFFSET - ctypes.sizeof(hdr)))
        f.write(index)
        f.write(b"\0" * (data_off - INDEX_OFFSET - index_bytes))
        for L in range(n_layers):
            arrays = make_layer(L)
            if len(arrays) != nt:
                raise ValueError("make_layer(%d) returned %d tensors, expected %d" % (L, len(arrays), nt))
            buf = np.zeros(run, dtype=np.uint8)
            for s, o, a in zip(specs, offs, arrays):
                a = np.frombuffer(a, dtype=np.uint8) if isinstance(a, (bytes, bytearray)) else a.view(np.uint8)
                if a.size != s.nbytes:
                    raise ValueError("%s: %d bytes, expected %d" % (s.suffix, a.size, s.nbytes))
                buf[o:o + s.nbytes] = a.reshape(-1)
            f.write(buf.tobytes())
    return hdr.total_bytes


def dit_block_specs(hidden, qkv_out, mlp_hidden, qtype=fh3.FH3_QUANT_Q4_K, inner=None, gate_compress=False):
    """The nine tensors of a DiT block in run order.  fc1 holds the value and
    gate halves of the gated MLP as one (2*mlp_hidden x hidden) matrix; the
    norm weights are fp32 vectors.  inner (default hidden) is the attention
    width: the out projection maps inner -> hidden.  gate_compress=True makes
    the VSA gate projection a (inner x hidden) matrix of type qtype, as in the
    real model (src/model/fh3_dit.c:404-407); otherwise it is an fp32 vector of
    hidden entries, which the product never reads."""
    f32 = fh3.FH3_QUANT_F32
    inner = hidden if inner is None else inner
    gc = (TensorSpec("attn.to_gate_compress.weight", qtype, hidden, inner) if gate_compress
          else TensorSpec("attn.to_gate_compress.weight", f32, hidden, 1))
    return [TensorSpec("attn.qkv_proj.weight", qtype, hidden, qkv_out),
            gc,
            TensorSpec("attn.out_proj.weight", qtype, inner, hidden),
            TensorSpec("mlp.fc1.weight", qtype, hidden, 2 * mlp_hidden),
            TensorSpec("mlp.fc2.weight", qtype, mlp_hidden, hidden),
            TensorSpec("norm1.weight", f32, hidden),
            TensorSpec("norm2.weight", f32, hidden),
            TensorSpec("attn.q_norm.weight", f32, 128),
            TensorSpec("attn.k_norm.weight", f32, 128)]


# The real fh3 DiT block (src/cli/fh3_cli.c:935-941): hidden 5376, 56 heads of
# 128 (inner 7168), feed-forward 14336; 238,480,384 bytes per block in the
# reference's census (docs/data/census.json:17).
REAL_DIT = dict(hidden=5376, qkv_out=21504, mlp_hidden=14336, inner=7168, gate_compress=True)


def real_dit_block_specs(qtype=fh3.FH3_QUANT_Q4_K):
    return dit_block_specs(qtype=qtype, **REAL_DIT)


def synth_dit_block(specs, seed, L, sigma=0.02):
    """Seeded contents of block L: matrices quantised to Q4_K from N(0, sigma),
    fp32 vectors 1 + 0.1 N(0, 1) (norm weights).  Stream ids are
    0x100*L + tensor index."""
    out = []
    for i, s in enumerate(specs):
        if s.qtype == fh3.FH3_QUANT_Q4_K:
            out.append(fh3.synth_q4k_weights(seed, 0x100 * L + i, s.ne1, s.ne0, sigma))
        else:
            v = fh3.synth_x("normal", seed, 0x100 * L + i, 1, s.ne0 * s.ne1)[0]
            out.append((1.0 + 0.1 * v).astype(np.float32).view(np.uint8))
    return out
