"""Products at the shapes of the reference's real call sites.

DiT block (src/model/fh3_dit.c:388,406,414,435,437; hidden 5376, 56 heads of
128, feed-forward 14336 at src/cli/fh3_cli.c:935-941):
  qkv 5376 -> 21504, gate_compress 5376 -> 7168 (the VSA gate, a Q4_K
  product), out 7168 -> 5376, fc1 5376 -> 28672 ([val | gate], with the
  SwiGLU epilogue too), fc2 14336 -> 5376,
at the CLI's default sequence length (640x384, 39 frames: n = 3016 tokens),
64 seeded token rows of each against the oracle.  qkv and gate_compress read
one normalised, modulated prepared buffer as the fused block does.

Text encoder (src/model/fh3_te.c:455-487; hidden 5120, 64 query heads and
8 key/value heads of 128, intermediate 25600 at src/model/fh3_te.h:12-22):
  q 5120 -> 8192, k and v 5120 -> 1024, o 8192 -> 5120, gate and up
  5120 -> 25600, down 25600 -> 5120,
at prompt lengths 1, 2, 4, 16 and 64 tokens, every row against the oracle, and
65, 128, 300 and 600 tokens on sampled rows.
K = 25600 with one or two tokens is past the integer-MFMA kernel's LDS and
runs the small-M fp16 kernel.
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu
TOL = 2e-3
EPS = 1e-6

DIT_HIDDEN, DIT_INNER, DIT_FFN = 5376, 7168, 14336
DIT_N = 3016
DIT = [("qkv", DIT_HIDDEN, 3 * DIT_INNER), ("gate_compress", DIT_HIDDEN, DIT_INNER),
       ("out", DIT_INNER, DIT_HIDDEN), ("fc1", DIT_HIDDEN, 2 * DIT_FFN), ("fc2", DIT_FFN, DIT_HIDDEN)]

TE = [("q", 5120, 8192), ("k", 5120, 1024), ("v", 5120, 1024), ("o", 8192, 5120), ("gate", 5120, 25600),
      ("up", 5120, 25600), ("down", 25600, 5120)]


def _sub(M, seed, n=64):
    """n token rows of M (M >= n): the first and last, the two either side of
    a 256-token tile edge when M has one, and seeded others."""
    rng = np.random.default_rng(seed)
    edges = {t for t in (0, 255, 256, M - 1) if t < M}
    pick = set(int(t) for t in rng.choice(M, n - len(edges), replace=False)) | edges
    return np.array(sorted(pick))


def _rows(F, buf, N, rows):
    out = np.empty((len(rows), N), np.float32)
    for i, t in enumerate(rows):
        F._check(F.lib().fh3_hip_memcpy_dtoh(out[i].ctypes.data, buf.ptr + int(t) * N * 4, N * 4), "dtoh")
    return out


@pytest.mark.parametrize("name,K,N", DIT, ids=[d[0] for d in DIT])
def test_dit_real_products(gpu, oracle, name, K, N):
    F = gpu
    M = DIT_N
    print("case: DiT %s M=%d K=%d N=%d path=%d" % (name, M, K, N, F.matmul_path(M, K)), flush=True)
    raw = F.synth_q4k_weights(31, K + N, N, K, 0.02, 0.0)
    x = F.synth_x("outliers" if name != "fc2" else "silu_gated", 31, K, M, K)
    dw, dx, dy = F.DeviceBuffer.from_array(raw), F.DeviceBuffer.from_array(x), F.DeviceBuffer(M * N * 4)
    F.matmul_dev(dw, K, N, dx, dy, M)
    F.synchronize()
    sub = _sub(M, K + N)
    yo = H.oracle_matmul(oracle, raw, K, N, x[sub])
    err = H.rel_fro(_rows(F, dy, N, sub), yo)
    print("  rel_fro %.3e" % err, flush=True)
    assert err <= TOL
    if name == "fc1":      # the SwiGLU epilogue writes [M][ffn] directly
        act = F.DeviceBuffer(M * DIT_FFN * 4)
        F.matmul_epi_dev(dw, K, N, dx, M, F.EPI_SWIGLU, act)
        F.synchronize()
        ref = np.zeros((len(sub), DIT_FFN), np.float32)
        H.elementwise(oracle, "fh3_oracle_", "swiglu", yo, ref, len(sub), DIT_FFN)
        err = H.rel_fro(_rows(F, act, DIT_FFN, sub), ref)
        print("  swiglu epilogue rel_fro %.3e" % err, flush=True)
        assert err <= TOL


def test_dit_qkv_and_gate_compress_share_one_prep(gpu, oracle):
    """The VSA branch: one rmsnorm+modulate prep feeds both qkv and
    gate_compress (src/model/fh3_dit.c:383-407)."""
    F = gpu
    M, K = DIT_N, DIT_HIDDEN
    print("case: DiT fused prep -> qkv + gate_compress, M=%d" % M, flush=True)
    h = F.synth_x("normal", 32, 1, M, K)
    nw = (1 + 0.1 * F.synth_x("normal", 32, 2, 1, K)[0]).astype(np.float32)
    shift = (0.1 * F.synth_x("normal", 32, 3, M, K)).astype(np.float32)
    scale = (0.2 * F.synth_x("normal", 32, 4, M, K)).astype(np.float32)
    d = {k: F.DeviceBuffer.from_array(v) for k, v in dict(h=h, nw=nw, shift=shift, scale=scale).items()}
    prep = F.DeviceBuffer(F.prepared_bytes(M, K))
    F.prepare_x_norm_dev(d["h"], M, K, d["nw"], EPS, prep, d["shift"], d["scale"])
    sub = _sub(M, 5)
    xn = h[sub].copy()
    H.elementwise(oracle, "fh3_oracle_", "rmsnorm", xn, nw, len(sub), K, EPS)
    H.elementwise(oracle, "fh3_oracle_", "modulate", xn, shift[sub], scale[sub], len(sub), K)
    for name, N in (("qkv", 3 * DIT_INNER), ("gate_compress", DIT_INNER)):
        raw = F.synth_q4k_weights(32, N, N, K, 0.02, 0.0)
        dw, dy = F.DeviceBuffer.from_array(raw), F.DeviceBuffer(M * N * 4)
        F.matmul_prepared_dev(dw, K, N, prep, dy, M)
        F.synchronize()
        err = H.rel_fro(_rows(F, dy, N, sub), H.oracle_matmul(oracle, raw, K, N, xn))
        print("  %s rel_fro %.3e" % (name, err), flush=True)
        assert err <= TOL


@pytest.mark.parametrize("name,K,N", TE, ids=[t[0] for t in TE])
def test_te_real_products(gpu, oracle, name, K, N):
    F = gpu
    raw = F.synth_q4k_weights(33, K + N, N, K, 0.02, 0.0)
    dw = F.DeviceBuffer.from_array(raw)
    for M in (1, 2, 4, 16, 64):
        path = F.matmul_path(M, K)
        print("case: TE %s M=%d K=%d N=%d path=%d" % (name, M, K, N, path), flush=True)
        if K == 25600 and M <= 16:
            assert path == F.PATH_SWEEP      # past k_gemv8's window: the sweep in five K slices
        x = F.synth_x("silu_gated" if name == "down" else "normal", 33, 100 * M + K, M, K)
        dx, dy = F.DeviceBuffer.from_array(x), F.DeviceBuffer(M * N * 4)
        F.matmul_dev(dw, K, N, dx, dy, M)
        F.synchronize()
        y = dy.download(np.float32, (M, N))
        yo = H.oracle_matmul(oracle, raw, K, N, x)
        err = H.rel_fro(y, yo)
        worst = max(H.rel_fro(y[t], yo[t]) for t in range(M))
        print("  rel_fro %.3e, worst row %.3e" % (err, worst), flush=True)
        assert err <= TOL and worst <= TOL, (M, err, worst)


@pytest.mark.parametrize("name,K,N", TE, ids=[t[0] for t in TE])
def test_te_prompt_lengths(gpu, oracle, name, K, N):
    """The text encoder's prompt lengths past 64 tokens (prompts run about
    6-600 tokens through src/model/fh3_te.c:455-487): 65, 128, 300 and 600
    tokens, including the 25600-long down rows, on 48 sampled token rows
    against the oracle, the worst row within the gate too."""
    F = gpu
    raw = F.synth_q4k_weights(34, K + N, N, K, 0.02, 0.0)
    dw = F.DeviceBuffer.from_array(raw)
    for M in (65, 128, 300, 600):
        print("case: TE %s M=%d K=%d N=%d path=%d" % (name, M, K, N, F.matmul_path(M, K)), flush=True)
        x = F.synth_x("silu_gated" if name == "down" else "normal", 34, 100 * M + K, M, K)
        dx, dy = F.DeviceBuffer.from_array(x), F.DeviceBuffer(M * N * 4)
        F.matmul_dev(dw, K, N, dx, dy, M)
        F.synchronize()
        sub = _sub(M, M + K, n=48)
        y = _rows(F, dy, N, sub)
        yo = H.oracle_matmul(oracle, raw, K, N, x[sub])
        err = H.rel_fro(y, yo)
        worst = max(H.rel_fro(y[i], yo[i]) for i in range(len(sub)))
        print("  rel_fro %.3e, worst row %.3e" % (err, worst), flush=True)
        assert err <= TOL and worst <= TOL, (M, err, worst)
