"""FH3P reader and layer streamer, host side (runs without a GPU).

Mirrors the reference's tests/unit/test_pack.c:47-253 (layout, tensor bytes
against the GGUF they were packed from, error codes) and
tests/unit/test_trunk.c:133-357 (pinned-prefix hit rate, never-LRU, prefetch
overlap, two-slot pointer identity, plan refusal), then replays random call
sequences through the reference's own streamer (its fh3_pack.c and
fh3_trunk.c, built from source by oracle/Makefile) and this library's,
comparing every counter and slot choice step by step.
"""
import ctypes
import hashlib
import json
import os
import shutil
import struct
import time

import numpy as np
import pytest

import helpers

MB = 1 << 20
GOLDEN_PACK = os.path.join(helpers.GOLDEN, "tiny_trunk.bin")
SUFFIXES = ("attn.qkv_proj.weight", "attn.to_gate_compress.weight", "attn.out_proj.weight", "mlp.fc1.weight",
            "mlp.fc2.weight", "norm1.weight", "norm2.weight", "attn.q_norm.weight", "attn.k_norm.weight")


@pytest.fixture
def pattern_pack(tmp_path):
    return helpers.write_pattern_pack(str(tmp_path / "synthetic_10layer.bin"), [MB] * 10)


def assert_pattern(fh3, addr, L, size):
    assert addr is not None
    b = fh3.host_bytes(addr, size)
    assert b[0] == 0xA0 + L and b[size - 1] == 0xA0 + L
    assert np.all(b == 0xA0 + L)


# ---------------------------------------------------------------------------
# pack reader (reference tests/unit/test_pack.c)
# ---------------------------------------------------------------------------
def test_pack_layer_offsets_aligned(fh3):
    with fh3.Pack(GOLDEN_PACK) as p:
        assert p.header.magic == fh3.FH3_PACK_MAGIC and p.header.version == fh3.FH3_PACK_VERSION
        assert p.num_layers == 2 and p.header.layer_alignment == 4096
        for L in range(p.num_layers):
            ld = p.layer_desc(L)
            assert ld.file_offset % 4096 == 0 and ld.size_bytes % 4096 == 0
            assert ld.n_tensors == 9
            for t in range(ld.n_tensors):
                assert ld.tensors[t].offset_in_layer % 32 == 0 and ld.tensors[t].size_bytes > 0


def _tensor_digest(addr, n):
    return hashlib.sha256(ctypes.string_at(addr, n)).hexdigest()


def test_pack_layer_tensor_bytes_match_gguf(fh3):
    """Views over a host copy of each layer run, and over the mapping, hold the
    GGUF tensor bytes (sha256 digests in tests/golden/pack_vectors.json)."""
    golden = json.load(open(os.path.join(helpers.GOLDEN, "pack_vectors.json")))["tensors"]
    raw = open(GOLDEN_PACK, "rb").read()
    with fh3.Pack(GOLDEN_PACK) as p:
        for L in range(p.num_layers):
            ld = p.layer_desc(L)
            run = np.frombuffer(raw, dtype=np.uint8, count=ld.size_bytes, offset=ld.file_offset).copy()
            base = run.ctypes.data
            for view in (p.layer(L, base), p.layer(L, None)):
                for t, name in enumerate(fh3.LAYER_TENSORS):
                    g = golden["blocks.%d.%s" % (L, SUFFIXES[t])]
                    w = getattr(view, name)
                    td = ld.tensors[t]
                    assert td.size_bytes == g["nbytes"]
                    assert w.type == g["type"] == td.type
                    assert (w.in_, w.out) == (td.in_dim, td.out_dim)
                    assert w.in_ == g["dims"][0]
                    assert _tensor_digest(w.data, g["nbytes"]) == g["sha256"], (L, name)
            # the host-copy view points into the copy at the descriptor offsets
            v = p.layer(L, base)
            assert [getattr(v, n).data - base for n in fh3.LAYER_TENSORS] == \
                [ld.tensors[t].offset_in_layer for t in range(9)]


def _patched(tmp_path, name, edits=(), cut=None):
    path = str(tmp_path / name)
    shutil.copyfile(GOLDEN_PACK, path)
    with open(path, "r+b") as f:
        for off, fmt, val in edits:
            f.seek(off)
            f.write(struct.pack(fmt, val))
        if cut is not None:
            f.truncate(cut)
    return path


def test_pack_robustness(fh3, tmp_path):
    lib = fh3.lib()
    p = fh3.Fh3Pack()
    assert lib.fh3_pack_open(None, ctypes.byref(p)) == fh3.FH3_ERR
    assert lib.fh3_pack_open(GOLDEN_PACK.encode(), None) == fh3.FH3_ERR
    assert lib.fh3_pack_open(str(tmp_path / "non_existent_file.bin").encode(), ctypes.byref(p)) == fh3.FH3_E_IO
    cases = [
        ("short.bin", (), 100, fh3.FH3_E_TRUNCATED),
        ("magic.bin", ((0, "<I", 0x12345678),), None, fh3.FH3_E_BAD_MAGIC),
        ("version.bin", ((4, "<I", 2),), None, fh3.FH3_E_BAD_VERSION),
        ("align.bin", ((12, "<I", 512),), None, fh3.FH3_E_INVALID),
        ("nolayers.bin", ((8, "<I", 0),), None, fh3.FH3_E_INVALID),
        ("index_past_eof.bin", ((16, "<Q", 1 << 40),), None, fh3.FH3_E_TRUNCATED),
        ("tiny_index.bin", ((24, "<Q", 2 * 23),), None, fh3.FH3_E_TRUNCATED),
    ]
    for name, edits, cut, want in cases:
        path = _patched(tmp_path, name, edits, cut)
        assert lib.fh3_pack_open(path.encode(), ctypes.byref(p)) == want, name


def test_pack_layer_out_of_range_is_empty(fh3):
    with fh3.Pack(GOLDEN_PACK) as p:
        for L in (-1, p.num_layers, 1 << 20):
            v = p.layer(L, None)
            assert all(getattr(v, n).data is None and getattr(v, n).in_ == 0 for n in fh3.LAYER_TENSORS)


def test_pack_writer_round_trip(fh3, tmp_path):
    """Packs written by fasth3inc_amd.pack (24 + 9*168-byte descriptors, as the
    reference's packer writes) read back with the same descriptors and bytes."""
    from fasth3inc_amd import pack as P
    specs = P.dit_block_specs(hidden=512, qkv_out=768, mlp_hidden=1024)
    layers = [P.synth_dit_block(specs, seed=7, L=L) for L in range(3)]
    path = str(tmp_path / "dit.bin")
    P.write_pack(path, 3, specs, lambda L: layers[L])
    offs, run = P.layout(specs)
    with fh3.Pack(path) as p:
        assert p.num_layers == 3 and p.header.index_bytes == 3 * 1536
        for L in range(3):
            ld = p.layer_desc(L)
            assert ld.size_bytes == run and ld.file_offset % 4096 == 0 and ld.n_tensors == 9
            v = p.layer(L, None)
            for t, (s, name) in enumerate(zip(specs, fh3.LAYER_TENSORS)):
                w = getattr(v, name)
                assert (w.type, w.in_, w.out) == (s.qtype, s.ne0, s.ne1)
                assert ld.tensors[t].offset_in_layer == offs[t]
                assert ld.tensors[t].name.decode() == "blocks.%d.%s" % (L, s.suffix)
                assert ctypes.string_at(w.data, s.nbytes) == layers[L][t].tobytes()


# ---------------------------------------------------------------------------
# trunk streamer (reference tests/unit/test_trunk.c)
# ---------------------------------------------------------------------------
def test_trunk_pinned_prefix_hit_rate(fh3, pattern_pack):
    with fh3.Trunk(pattern_pack, 8 * MB) as tr:
        inf = tr.info()
        assert inf.num_layers == 10 and inf.npin == 6 and inf.slot_size == MB
        for _ in range(3):
            for L in range(10):
                assert_pattern(fh3, tr.acquire(L), L, MB)
        s = tr.stats()
        assert (s.hits, s.misses, s.bytes_read) == (18, 12, 12 * MB)


def test_trunk_never_lru(fh3, pattern_pack):
    lru, lru_hits = [], 0
    for _ in range(3):
        for L in range(10):
            if L in lru:
                lru_hits += 1
                lru.remove(L)
            elif len(lru) == 8:
                lru.pop(0)
            lru.append(L)
    assert lru_hits == 0
    with fh3.Trunk(pattern_pack, 8 * MB) as tr:
        for _ in range(3):
            for L in range(10):
                assert tr.acquire(L) is not None
        assert tr.stats().hits == 18


def test_trunk_prefetch_overlaps(fh3, pattern_pack):
    with fh3.Trunk(pattern_pack, 8 * MB) as tr:
        tr.prefetch(6)
        time.sleep(0.025)
        assert_pattern(fh3, tr.acquire(6), 6, MB)
        s = tr.stats()
        assert s.read_s > 0.0 and s.wait_s < s.read_s


def test_trunk_multi_slot_acquisition(fh3, pattern_pack):
    with fh3.Trunk(pattern_pack, 8 * MB) as tr:
        a1 = tr.acquire(6)
        assert_pattern(fh3, a1, 6, MB)
        assert (tr.stats().misses, tr.stats().hits) == (1, 0)
        tr.prefetch(7)
        assert tr.acquire(6) == a1
        assert (tr.stats().misses, tr.stats().hits) == (1, 1)
        b1 = tr.acquire(7)
        assert b1 != a1
        assert_pattern(fh3, b1, 7, MB)
        assert (tr.stats().misses, tr.stats().hits) == (2, 1)
        for i, (L, want) in enumerate([(6, a1), (7, b1), (6, a1), (7, b1)]):
            assert tr.acquire(L) == want
            assert (tr.stats().hits, tr.stats().misses) == (2 + i, 2)


def test_plan_refuses_when_short(fh3):
    avail = fh3.mem_available()
    assert avail > 0
    assert fh3.plan_check(fh3.plan(total_bytes=avail + (20 << 30))) == fh3.FH3_E_NOMEM
    assert fh3.plan_check(fh3.plan(min_bytes=2 << 30, budget_bytes=536870912)) == fh3.FH3_E_NOMEM
    ok = fh3.plan(min_bytes=MB, budget_bytes=32 * MB)
    assert fh3.plan_check(ok) == fh3.FH3_OK and fh3.plan_bytes(ok) == 32 * MB
    comp = fh3.plan(pinned_bytes=1000, ring_bytes=2000, activation_bytes=3000, table_bytes=4000,
                    total_bytes=50000, budget_bytes=99999)
    assert fh3.plan_bytes(comp) == 10000
    assert fh3.plan_bytes(fh3.plan(total_bytes=50000, budget_bytes=99999)) == 50000
    assert fh3.lib().fh3_plan_check(None) == fh3.FH3_ERR


def test_trunk_short_read_returns_null(fh3, tmp_path):
    path = helpers.write_pattern_pack(str(tmp_path / "cut.bin"), [MB] * 10, truncate_last=4096)
    with fh3.Trunk(path, 4 * MB) as tr:
        assert tr.info().npin == 2
        assert tr.acquire(9) is None
        assert tr.stats().misses == 0
        assert_pattern(fh3, tr.acquire(8), 8, MB)
        assert tr.stats().misses == 1
    # a pinned layer that cannot be read whole fails the open
    with pytest.raises(fh3.Fh3Error) as e:
        fh3.Trunk(path, 64 * MB)
    assert e.value.code == fh3.FH3_E_IO


def test_trunk_open_errors(fh3, tmp_path):
    lib = fh3.lib()
    buf = ctypes.create_string_buffer(lib.fh3_trunk_struct_bytes())
    assert lib.fh3_trunk_open(None, MB, ctypes.addressof(buf)) == fh3.FH3_ERR
    assert lib.fh3_trunk_open(GOLDEN_PACK.encode(), MB, None) == fh3.FH3_ERR
    assert lib.fh3_trunk_open(str(tmp_path / "missing.bin").encode(), MB, ctypes.addressof(buf)) == fh3.FH3_E_IO
    # out-of-range layers and NULL trunks are refused without side effects
    with fh3.Trunk(GOLDEN_PACK, 0) as tr:
        assert tr.acquire(-1) is None and tr.acquire(2) is None
        tr.prefetch(5)
        assert tr.stats().misses == 0
    assert lib.fh3_trunk_acquire(None, 0) is None
    # the device calls refuse a trunk that was never attached
    with fh3.Trunk(GOLDEN_PACK, 0) as tr:
        assert tr.acquire_dev(0) is None
        tr.prefetch_dev(0)


@pytest.mark.parametrize("sizes,budget", [
    ([MB] * 10, 8 * MB), ([MB] * 10, 0), ([MB] * 10, 2 * MB - 1), ([MB] * 10, 64 * MB),
    ([3 * MB, MB, MB, 2 * MB, MB, 4 * MB, MB], 9 * MB),
    ([100000, 300000, 5000, 250000, 4096, 123456], 700000),
    ([MB, 2 * MB, 3 * MB, 4 * MB], 11 * MB), ([4 * MB, 3 * MB, 2 * MB, MB], 11 * MB),
])
def test_trunk_prefix_split_is_a_fixed_point(fh3, tmp_path, sizes, budget):
    """The prefix/slot split is a fixed point: slots are exactly as large as the
    biggest streamed layer (page-rounded), and the prefix is the longest one
    that fits beside two such slots.  It is the first fixed point reached from
    "slot = biggest layer", not always the longest prefix possible: [4,3,2,1] MB
    under 11 MB pins nothing although 4 MB + 2 x 3 MB would fit, exactly as the
    reference's iteration (src/io/fh3_trunk.c:161-200) decides."""
    page = lambda n: -(-n // 4096) * 4096
    path = helpers.write_pattern_pack(str(tmp_path / "v.bin"), sizes)
    with fh3.Trunk(path, budget) as tr:
        inf = tr.info()
        npin, slot = inf.npin, inf.slot_size
        assert slot == page(max(sizes[npin:] or sizes))
        avail = max(budget - 2 * slot, 0)
        assert sum(sizes[:npin]) <= avail
        assert npin == len(sizes) or sum(sizes[:npin + 1]) > avail
        for L in range(len(sizes)):
            assert_pattern(fh3, tr.acquire(L), L, sizes[L])
    if sizes == [4 * MB, 3 * MB, 2 * MB, MB]:
        assert npin == 0


# ---------------------------------------------------------------------------
# step-by-step agreement with the reference's own streamer
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def ref_io():
    lib = helpers.load_ref_io()
    if lib is None:
        pytest.skip("oracle/_ref/libfh3_ref_io.so not built (reference tree absent)")
    return lib


class RefTrunk:
    def __init__(self, lib, path, budget):
        self.lib = lib
        self.buf = ctypes.create_string_buffer(helpers.REF_TRUNK_BYTES)
        self.t = ctypes.addressof(self.buf)
        rc = lib.fh3_trunk_open(path.encode(), budget, self.t)
        assert rc == 0, rc

    def prefetch(self, L):
        self.lib.fh3_trunk_prefetch(self.t, L)

    def acquire(self, L):
        return self.lib.fh3_trunk_acquire(self.t, L)

    def stats(self):
        return self.lib.fh3_trunk_stats(self.t)

    def close(self):
        self.lib.fh3_trunk_close(self.t)


SEQ_CASES = [
    ([MB] * 10, 8 * MB), ([MB] * 10, 0), ([MB] * 6, 5 * MB),
    ([3 * MB, MB, MB, 2 * MB, MB, 4 * MB, MB], 9 * MB),
    ([100000, 300000, 5000, 250000, 4096, 123456], 700000),
]


@pytest.mark.parametrize("case", range(len(SEQ_CASES)))
def test_trunk_matches_reference_streamer(fh3, ref_io, tmp_path, case):
    """Same pack, budget and call sequence (scans with and without prefetch,
    random prefetch/acquire mixes, out-of-range layers) through both streamers:
    identical hit/miss/byte counters after every call, identical slot choice
    (the order in which distinct addresses appear) and identical bytes."""
    sizes, budget = SEQ_CASES[case]
    n = len(sizes)
    path = helpers.write_pattern_pack(str(tmp_path / "seq.bin"), sizes)
    rng = np.random.default_rng(1000 + case)
    ops = []
    for _ in range(2):
        for L in range(n):
            ops += [("acquire", L), ("prefetch", (L + 1) % n)]
    for L in range(n):
        ops.append(("acquire", L))
    for _ in range(300):
        ops.append(("prefetch" if rng.random() < 0.4 else "acquire", int(rng.integers(-1, n + 1))))
    mine, theirs = fh3.Trunk(path, budget), RefTrunk(ref_io, path, budget)
    ids_m, ids_r = {}, {}
    try:
        for i, (op, L) in enumerate(ops):
            if op == "prefetch":
                mine.prefetch(L)
                theirs.prefetch(L)
            else:
                a, b = mine.acquire(L), theirs.acquire(L)
                assert (a is None) == (b is None), (i, op, L)
                if a is not None:
                    assert ids_m.setdefault(a, len(ids_m)) == ids_r.setdefault(b, len(ids_r)), (i, L)
                    assert ctypes.string_at(a, sizes[L]) == ctypes.string_at(b, sizes[L])
            sm, sr = mine.stats(), theirs.stats()
            assert (sm.hits, sm.misses, sm.bytes_read) == (sr.hits, sr.misses, sr.bytes_read), (i, op, L)
    finally:
        mine.close()
        theirs.close()
