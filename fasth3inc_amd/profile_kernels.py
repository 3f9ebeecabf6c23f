"""Launch the hot kernels at the benchmark shapes, for rocprofv3.

    rocprofv3 --kernel-trace --stats -d OUT -- python3 -m fasth3inc_amd.profile_kernels gemv
    rocprofv3 --pmc FETCH_SIZE -d OUT -- python3 -m fasth3inc_amd.profile_kernels gemv
    rocprofv3 --pmc WRITE_SIZE -d OUT -- python3 -m fasth3inc_amd.profile_kernels copy

Workloads (each launch sequence is preceded by one untimed warmup launch):
  gemv   the six small-M shapes (M in {1,4,16}, K=5120, N in {5120,17408}):
         fh3_hip_matmul_prepared_dev -> k_gemv8 (M <= 4) and k_sweep
         (M = 16, after k_xprep), weights rotated over more than 256 MB of
         device copies so they come from HBM
  gemm   the DiT attention shapes (M=8192, K=5120, N in {15360,5120}):
         fh3_hip_matmul_prepared_dev -> k_gemm, and the activation prep k_xprep
  mlp    the DiT MLP shapes (M=32768: up and gate K=5120 -> N=13824 with a
         2-decade per-super-block scale spread, down K=13824 -> N=5120 on
         SiLU-gated activations): fh3_hip_matmul_prepared_dev -> k_gemm, and
         the activation prep k_xprep_r8
  te     the text encoder's long Q4_K rows at M = 1 and 16 (o-projection
         K=8192 -> N=5120, down-projection K=25600 -> N=5120):
         fh3_hip_matmul_prepared_dev -> k_gemv8 (M = 1, K = 8192) or k_sweep in
         K slices then k_midm_sum; weights rotated as for gemv
  prompt 17 to 64 tokens at K = 5120 (M in {17, 32, 48, 64}, N in {5120,
         17408}): fh3_hip_matmul_prepared_dev -> k_sweep with two to four
         token blocks; weights rotated as for gemv
  mid    65, 128 and 256 tokens at K = 5120 (N in {5120, 17408}):
         fh3_hip_matmul_prepared_dev -> k_gemm with 128- or 256-token tiles
         and a K split, then k_midm_sum; weights rotated as for gemv
  single the 64 x 4096 x 4096 product of the reference's bench_matmul.c, one
         weight copy (warm in the Infinity Cache after the first launch, as the
         benchmark runs it): fh3_hip_matmul_prepared_dev -> k_skinny
  q56    Q5_K and Q6_K weights read in place at the text encoder's shapes
         (Q5_K 5120 -> 1024, Q6_K 5120 -> 1024, 8192 -> 5120, 25600 -> 5120)
         at M = 1, 16 and 300: fh3_hip_matmul_prepared_dev -> k_sweep<Q6_K>
         and k_skinny<Q5_K> (K slices / windows, then k_midm_sum, where they
         split K) and k_gemm<TBW, Q5_K / Q6_K> at 300; weights rotated as for
         gemv
  copy   hipMemcpy device-to-device of 256 MiB: a copy of known size that
         calibrates FETCH_SIZE / WRITE_SIZE against the bytes moved
  attn   the DiT attention branch at n = 16384 tokens, 40 heads of 128
         (hidden 5120): fh3_hip_attention_qkv_dev from a qkv projection
         output with q/k rmsnorm and rope3 on 96 channels -> k_attn_prep,
         k_attn_fwd
  vsa    video sparse attention at the reference CLI's 1024x576, 73-frame
         shape (6 text + 244 audio tokens, video grid 22x18x32, n = 12922),
         56 heads of 128, sparsity 0.8, with q/k rmsnorm, rope3 and the gate:
         fh3_hip_vsa_attention_qkv_dev -> every VSA kernel
"""
import argparse
import sys

import numpy as np

from . import fh3 as F

MALL_BYTES = 256 << 20


def gemv(reps):
    for N in (5120, 17408):
        for M in (1, 4, 16):
            K = 5120
            raw = F.synth_q4k_weights(0, 100 + N, N, K, 0.02, 0.0)
            copies = max(2, -(-(MALL_BYTES + (64 << 20)) // raw.nbytes))
            ws = [F.DeviceBuffer.from_array(raw) for _ in range(copies)]
            dx = F.DeviceBuffer.from_array(F.synth_x("normal", 0, 200 + M, M, K))
            dy = F.DeviceBuffer(M * N * 4)
            prep = F.DeviceBuffer(F.prepared_bytes(M, K))
            F.prepare_x_dev(dx, M, K, prep)
            for i in range(reps + 1):
                F.matmul_prepared_dev(ws[i % copies], K, N, prep, dy, M)
            F.synchronize()
            print("gemv M=%d N=%d K=%d: %d launches, %d weight copies" % (M, N, K, reps, copies), flush=True)
            for b in ws + [dx, dy, prep]:
                b.close()


def te(reps):
    for K, N in ((8192, 5120), (25600, 5120)):
        for M in (1, 16):
            raw = F.synth_q4k_weights(0, 100 + N + K, N, K, 0.02, 0.0)
            copies = max(2, -(-(MALL_BYTES + (64 << 20)) // raw.nbytes))
            ws = [F.DeviceBuffer.from_array(raw) for _ in range(copies)]
            dx = F.DeviceBuffer.from_array(F.synth_x("normal", 0, 200 + M, M, K))
            dy = F.DeviceBuffer(M * N * 4)
            prep = F.DeviceBuffer(F.prepared_bytes(M, K))
            F.prepare_x_dev(dx, M, K, prep)
            for i in range(reps + 1):
                F.matmul_prepared_dev(ws[i % copies], K, N, prep, dy, M)
            F.synchronize()
            print("te M=%d N=%d K=%d path %d: %d launches" % (M, N, K, F.matmul_path(M, K), reps), flush=True)
            for b in ws + [dx, dy, prep]:
                b.close()


def _rotated_products(tag, shapes, reps):
    for M, K, N in shapes:
        raw = F.synth_q4k_weights(0, 100 + N + K, N, K, 0.02, 0.0)
        copies = max(2, -(-(MALL_BYTES + (64 << 20)) // raw.nbytes))
        ws = [F.DeviceBuffer.from_array(raw) for _ in range(copies)]
        dx = F.DeviceBuffer.from_array(F.synth_x("normal", 0, 200 + M, M, K))
        dy = F.DeviceBuffer(M * N * 4)
        prep = F.DeviceBuffer(F.prepared_bytes(M, K))
        F.prepare_x_dev(dx, M, K, prep)
        for i in range(reps + 1):
            F.matmul_prepared_dev(ws[i % copies], K, N, prep, dy, M)
        F.synchronize()
        print("%s M=%d N=%d K=%d path %d: %d launches, %d weight copies" % (tag, M, N, K, F.matmul_path(M, K), reps,
                                                                          copies), flush=True)
        for b in ws + [dx, dy, prep]:
            b.close()


def _random_q56(qt, rows, K, seed):
    """Random Q5_K (176 B) or Q6_K (210 B) super-blocks: random quant and
    scale bytes, fp16 block scales (d, and dmin for Q5_K) set to 2^-10."""
    bb = 176 if qt == F.FH3_QUANT_Q5_K else 210
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(rows, K // 256, bb), dtype=np.uint8)
    d = np.frombuffer(np.float16(2.0 ** -10).tobytes(), np.uint8)
    if qt == F.FH3_QUANT_Q5_K:
        raw[:, :, 0:2] = d
        raw[:, :, 2:4] = d
    else:
        raw[:, :, 208:210] = d
    return raw.reshape(-1)


def single(reps):
    M, K, N = 64, 4096, 4096
    raw = F.synth_q4k_weights(0, 100 + N + K, N, K, 0.02, 0.0)
    dw = F.DeviceBuffer.from_array(raw)
    dx = F.DeviceBuffer.from_array(F.synth_x("normal", 0, 200 + M, M, K))
    dy = F.DeviceBuffer(M * N * 4)
    prep = F.DeviceBuffer(F.prepared_bytes(M, K))
    F.prepare_x_dev(dx, M, K, prep)
    for i in range(reps + 1):
        F.matmul_prepared_dev(dw, K, N, prep, dy, M)
    F.synchronize()
    print("single M=%d N=%d K=%d path %d: %d launches, one weight copy" % (M, N, K, F.matmul_path(M, K), reps),
          flush=True)
    for b in (dw, dx, dy, prep):
        b.close()


def q56(reps):
    for qt, K, N in ((F.FH3_QUANT_Q5_K, 5120, 1024), (F.FH3_QUANT_Q6_K, 5120, 1024), (F.FH3_QUANT_Q6_K, 8192, 5120),
                     (F.FH3_QUANT_Q6_K, 25600, 5120)):
        raw = _random_q56(qt, N, K, seed=5)
        copies = max(2, -(-(MALL_BYTES + (64 << 20)) // raw.nbytes))
        ws = [F.DeviceBuffer.from_array(raw) for _ in range(copies)]
        for M in (1, 16, 300):
            dx = F.DeviceBuffer.from_array(F.synth_x("normal", 0, 200 + M, M, K))
            dy = F.DeviceBuffer(M * N * 4)
            prep = F.DeviceBuffer(F.prepared_bytes(M, K))
            F.prepare_x_dev(dx, M, K, prep)
            for i in range(reps + 1):
                F.matmul_prepared_dev(ws[i % copies], K, N, prep, dy, M, qtype=qt)
            F.synchronize()
            print("q56 type %d M=%d N=%d K=%d: %d launches, %d weight copies" % (qt, M, N, K, reps, copies), flush=True)
            for b in (dx, dy, prep):
                b.close()
        for b in ws:
            b.close()


def prompt(reps):
    _rotated_products("prompt", [(M, 5120, N) for N in (5120, 17408) for M in (17, 32, 48, 64)], reps)


def mid(reps):
    _rotated_products("mid", [(M, 5120, N) for N in (5120, 17408) for M in (65, 128, 256)], reps)


def gemm(reps):
    M, K = 8192, 5120
    dx = F.DeviceBuffer.from_array(F.synth_x("outliers", 1, 400 + K, M, K))
    prep = F.DeviceBuffer(F.prepared_bytes(M, K))
    for N in (15360, 5120):
        dw = F.DeviceBuffer.from_array(F.synth_q4k_weights(1, 300 + N + K, N, K, 0.02, 0.0))
        dy = F.DeviceBuffer(M * N * 4)
        for _ in range(reps + 1):
            F.prepare_x_dev(dx, M, K, prep)
            F.matmul_prepared_dev(dw, K, N, prep, dy, M)
        F.synchronize()
        print("gemm M=%d N=%d K=%d: %d launches" % (M, N, K, reps), flush=True)
        dw.close()
        dy.close()


def mlp(reps):
    M = 32768
    for K, N, xkind in ((5120, 13824, "normal"), (13824, 5120, "silu_gated")):
        dx = F.DeviceBuffer.from_array(F.synth_x(xkind, 1, 400 + K, M, K))
        prep = F.DeviceBuffer(F.prepared_bytes(M, K))
        dw = F.DeviceBuffer.from_array(F.synth_q4k_weights(1, 300 + N + K, N, K, 0.02, 2.0))
        dy = F.DeviceBuffer(M * N * 4)
        for _ in range(reps + 1):
            F.prepare_x_dev(dx, M, K, prep)
            F.matmul_prepared_dev(dw, K, N, prep, dy, M)
        F.synchronize()
        print("mlp M=%d N=%d K=%d: %d launches" % (M, N, K, reps), flush=True)
        for b in (dx, prep, dw, dy):
            b.close()


def copy(reps):
    n = 256 << 20
    a, b = F.DeviceBuffer(n), F.DeviceBuffer(n)
    a.fill(1)
    for _ in range(reps + 1):
        F._check(F.lib().fh3_hip_memcpy_dtod(b.ptr, a.ptr, n), "fh3_hip_memcpy_dtod")
    F.synchronize()
    print("copy %d bytes: %d launches" % (n, reps), flush=True)


def attn(reps, n=16384, heads=40, hd=128, rot=96):
    inner = heads * hd
    qkv = F.DeviceBuffer.from_array(F.synth_x("normal", 2, 500, n, 3 * inner))
    w = F.DeviceBuffer.from_array(np.ones(hd, np.float32))
    ang = np.outer(np.arange(n, dtype=np.float64), 1e-2 * np.arange(1, rot // 2 + 1))
    ang = np.concatenate([ang, ang], axis=1)
    cs = F.DeviceBuffer.from_array(np.cos(ang).astype(np.float32))
    sn = F.DeviceBuffer.from_array(np.sin(ang).astype(np.float32))
    o = F.DeviceBuffer(n * inner * 4)
    for _ in range(reps + 1):
        F.attention_qkv_dev(qkv, n, heads, hd, o, w, w, 1e-5, cs, sn, rot)
    F.synchronize()
    print("attn n=%d heads=%d hd=%d: %d launches" % (n, heads, hd, reps), flush=True)
    for b in (qkv, w, cs, sn, o):
        b.close()


def vsa(reps, heads=56, hd=128, rot=96):
    n_text, n_audio, grid = 6, 244, (22, 18, 32)
    n = n_text + n_audio + grid[0] * grid[1] * grid[2]
    inner = heads * hd
    qkv = F.DeviceBuffer.from_array(F.synth_x("normal", 4, 700, n, 3 * inner))
    gate = F.DeviceBuffer.from_array(F.synth_x("normal", 4, 701, n, inner))
    w = F.DeviceBuffer.from_array(np.ones(hd, np.float32))
    ang = np.outer(np.arange(n, dtype=np.float64), 1e-2 * np.arange(1, rot // 2 + 1))
    ang = np.concatenate([ang, ang], axis=1)
    cs = F.DeviceBuffer.from_array(np.cos(ang).astype(np.float32))
    sn = F.DeviceBuffer.from_array(np.sin(ang).astype(np.float32))
    o = F.DeviceBuffer(n * inner * 4)
    seq = F.seq_of(n, n_text, n_audio, grid=grid)
    for _ in range(reps + 1):
        F.vsa_attention_qkv_dev(qkv, gate, o, seq, heads, hd, 0.8, 64, w, w, 1e-5, cs, sn, rot)
    F.synchronize()
    print("vsa n=%d heads=%d hd=%d: %d launches" % (n, heads, hd, reps), flush=True)
    for b in (qkv, gate, w, cs, sn, o):
        b.close()


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("workload", choices=("gemv", "te", "prompt", "mid", "single", "q56", "gemm", "mlp", "copy", "attn", "vsa",
                                         "all"))
    ap.add_argument("--reps", type=int, default=20)
    args = ap.parse_args(argv)
    F.init(0)
    for name in (("gemv", "gemm", "copy") if args.workload == "all" else (args.workload,)):
        globals()[name](args.reps)
    return 0


if __name__ == "__main__":
    sys.exit(main())
