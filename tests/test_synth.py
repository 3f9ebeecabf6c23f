"""Host-side seeded generators and the Q4_K encoder of libfh3hip.so (CPU)."""
import numpy as np
import pytest

import helpers as H


def test_philox_known_answers(fh3):
    """Random123 known-answer vectors for Philox4x32-10."""
    kat = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for ctr, key, want in kat:
        assert fh3.philox4x32_10(ctr, key).tolist() == want


def test_rng_normal_matches_reference_vectors(fh3):
    g = np.load(H.os.path.join(H.GOLDEN, "ref_vectors.npz"), allow_pickle=False)
    ours = fh3.rng_normal(7, 3, 1001)
    assert np.array_equal(ours.view(np.uint32), g["rng_seed7_stream3"].view(np.uint32))


def test_rng_normal_moments(fh3):
    z = fh3.rng_normal(0, 0, 1 << 20).astype(np.float64)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1) < 5e-3


def test_f32_to_f16_matches_numpy(fh3):
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)
    vals = np.concatenate([bits.view(np.float32),
                           np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 6.1e-5, 5.96e-8, 2.98e-8,
                                     2.9802322e-08, 1e-9, np.inf, -np.inf], dtype=np.float32)])
    for v in vals:
        ours = fh3.f32_to_f16_bits(v)
        with np.errstate(over="ignore"):  # values past the fp16 range round to infinity, as intended
            want = int(np.array([v], dtype=np.float32).astype(np.float16).view(np.uint16)[0])
        if np.isnan(v):
            assert (ours & 0x7C00) == 0x7C00 and (ours & 0x3FF)
        else:
            assert ours == want, (v, hex(ours), hex(want))


def test_quantizer_round_trip(fh3, oracle):
    """Encoded rows decode (oracle) within the 4-bit step of each group."""
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((16, 1024)) * 0.02).astype(np.float32)
    raw = fh3.q4k_quantize(w)
    assert raw.size == 16 * 4 * 144
    deq = H.oracle_dequant(oracle, raw, 16, 1024)
    g = w.reshape(-1, 32)
    step = (g.max(1) - np.minimum(g.min(1), 0)) / 15
    err = np.abs(deq.reshape(-1, 32) - g)
    # rounding to the nearest level costs <= step/2; 6-bit scale rounding adds a little
    assert (err <= 0.75 * step[:, None] + 1e-6).mean() > 0.999
    rel = np.linalg.norm(deq - w) / np.linalg.norm(w)
    assert rel < 0.12


def test_quantizer_fields_valid(fh3):
    rng = np.random.default_rng(2)
    w = rng.standard_normal((4, 512)).astype(np.float32)
    raw = fh3.q4k_quantize(w).reshape(-1, 144)
    d = raw[:, 0:2].copy().view(np.float16).astype(np.float32)
    dm = raw[:, 2:4].copy().view(np.float16).astype(np.float32)
    assert (d > 0).all() and (dm >= 0).all() and np.isfinite(d).all()


def test_quantizer_constant_and_zero_rows(fh3, oracle):
    w = np.zeros((2, 256), dtype=np.float32)
    w[1] = 0.5
    raw = fh3.q4k_quantize(w)
    deq = H.oracle_dequant(oracle, raw, 2, 256)
    assert np.array_equal(deq[0], np.zeros(256, np.float32))
    assert np.allclose(deq[1], 0.5, rtol=2e-3)


def test_synth_generators(fh3):
    x = fh3.synth_x("outliers", 0, 11, 64, 4096)
    frac = np.mean(np.abs(x) == 8.0)
    assert 0.008 < frac < 0.012
    y = fh3.synth_x("silu_gated", 0, 12, 64, 4096).astype(np.float64)
    # E[a * silu(b)] = 0, E[(a silu b)^2] = E[silu(b)^2] ~ 0.356
    assert abs(y.mean()) < 0.01 and 0.3 < (y ** 2).mean() < 0.42
    w1 = fh3.synth_q4k_weights(0, 1, 8, 512, 0.02, 0.0)
    w2 = fh3.synth_q4k_weights(0, 1, 8, 512, 0.02, 0.0)
    assert np.array_equal(w1, w2)
    w3 = fh3.synth_q4k_weights(0, 1, 300, 512, 0.02, 2.0)
    d = w3.reshape(-1, 144)[:, 0:2].copy().view(np.float16).astype(np.float64)
    spread = np.log10(np.percentile(d, 95) / np.percentile(d, 5))
    assert spread > 1.2


def test_synth_weights_chunking_invisible(fh3):
    """Rows beyond the 256-row generation chunk continue the same stream."""
    a = fh3.synth_q4k_weights(3, 9, 300, 256, 0.02, 2.0)
    b = fh3.synth_q4k_weights(3, 9, 260, 256, 0.02, 2.0)
    assert np.array_equal(a[:b.size], b)
