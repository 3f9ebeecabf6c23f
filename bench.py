#!/usr/bin/env python3
"""Benchmark of the fh3 Q4_K linear layer on one MI355X (gfx950).

Headline (`value`): small-M GEMV weight throughput on the text-encoder shapes
-- M in {1, 4, 16} tokens, K = 5120, N in {5120, 17408} -- one step = one call
of fh3_hip_matmul_dev for each of the six shapes, with the weights rotated
over distinct device copies (> 256 MB per shape) so the 256 MB MALL cannot
serve them.  value = sum of Q4_K weight bytes of a step / step time.

Also reported (`extra`): the DiT GEMMs (M = 8192 attention linears, M = 32768
MLP linears) in TFLOP/s, the M = 64 x 4096 x 4096 single matmul, kernel-only
rooflines from HIP events on the library's compute stream, and the CPU
baseline (the reference's fh3_matmul built from its sources by
oracle/Makefile, or the oracle restatement when that is absent) timed on
this host's cores on the GEMV shapes.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
import argparse
import ctypes
import json
import os
import platform
import re
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from fasth3inc_amd import fh3 as F  # noqa: E402

HBM_PEAK = 8.0e12        # B/s, MI355X HBM3E
MFMA_F16_PEAK = 2.5e15   # flop/s, MI355X dense fp16/bf16 MFMA
MALL_BYTES = 256 << 20   # Infinity Cache
METRIC = "Q4_K GEMM TFLOP/s + GEMV weight GB/s (% roofline); DiT block linear ms"

# HBM bytes per launch, measured with rocprofv3 --pmc FETCH_SIZE and --pmc
# WRITE_SIZE (one run each) over `python3 -m fasth3inc_amd.profile_kernels gemv
# --reps 5` (and `gemm` for the GEMM figures), scaled by 2.0 and 1.0: a 256 MiB
# device-to-device copy reads FETCH_SIZE = 128 MiB and WRITE_SIZE = 256 MiB.
# Summaries: profiles/gemv_k_gemv8_k_sweep_m1-16_k5120.md,
# profiles/k_gemm_dit_attention_m8192_k5120.md, profiles/hbm_counters_copy_256MiB.md.
# Re-measure when the kernels change.
TRAFFIC_GEMV_MEAN = 33641612        # mean over the six GEMV shapes (algorithmic mean 32899072)
TRAFFIC_GEMM = {"attn_qkv": 2324594574, "attn_out": 703181960}


def q4k_bytes(N, K):
    return N * (K // 256) * 144


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class HipEvents:
    """hipEvent timing on a given stream (the library's compute stream)."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def pair(self):
        a, b = ctypes.c_void_p(), ctypes.c_void_p()
        assert self.hip.hipEventCreate(ctypes.byref(a)) == 0
        assert self.hip.hipEventCreate(ctypes.byref(b)) == 0
        return a, b

    def time_ms(self, fn, iters, stream):
        a, b = self.pair()
        assert self.hip.hipEventRecord(a, stream) == 0
        for i in range(iters):
            fn(i)
        assert self.hip.hipEventRecord(b, stream) == 0
        assert self.hip.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        self.hip.hipEventDestroy(a)
        self.hip.hipEventDestroy(b)
        return ms.value / iters


# ---------------------------------------------------------------------------
# Workloads
# ---------------------------------------------------------------------------
class Gemv:
    """One small-M shape with rotated weight copies."""

    def __init__(self, M, K, N, seed):
        self.M, self.K, self.N = M, K, N
        wb = q4k_bytes(N, K)
        raw = F.synth_q4k_weights(seed, 100 + N, N, K, 0.02, 0.0)
        self.copies = max(2, -(-(MALL_BYTES + (64 << 20)) // wb))
        self.w = [F.DeviceBuffer.from_array(raw)]
        for _ in range(self.copies - 1):
            b = F.DeviceBuffer(wb)
            F.lib().fh3_hip_memcpy_dtod(b.ptr, self.w[0].ptr, wb)
            self.w.append(b)
        self.raw = raw
        self.x = F.synth_x("normal", seed, 200 + M, M, K)
        self.dx = F.DeviceBuffer.from_array(self.x)
        self.dy = F.DeviceBuffer(M * N * 4)
        self.prep = F.DeviceBuffer(F.prepared_bytes(M, K))
        F.prepare_x_dev(self.dx, M, K, self.prep)
        self.wbytes = wb
        self.alg_bytes = wb + 4 * M * K + 4 * M * N

    def call(self, i):
        F.matmul_dev(self.w[i % self.copies], self.K, self.N, self.dx, self.dy, self.M)

    def kernel(self, i):
        F.matmul_prepared_dev(self.w[i % self.copies], self.K, self.N, self.prep, self.dy, self.M)


class Gemm:
    """One large-M projection: weights ~N(0, 0.02) (optionally with a per
    super-block log-uniform scale spread), activations of a given kind."""

    def __init__(self, name, M, K, N, xkind, spread, seed, x_dev=None):
        self.name, self.M, self.K, self.N = name, M, K, N
        self.raw = F.synth_q4k_weights(seed, 300 + N + K, N, K, 0.02, spread)
        self.dw = F.DeviceBuffer.from_array(self.raw)
        if x_dev is None:
            x = F.synth_x(xkind, seed, 400 + K, M, K)
            self.dx = F.DeviceBuffer.from_array(x)
            del x
        else:
            self.dx = x_dev
        self.dy = F.DeviceBuffer(M * N * 4)
        self.prep = F.DeviceBuffer(F.prepared_bytes(M, K))
        F.prepare_x_dev(self.dx, M, K, self.prep)
        self.flop = 2.0 * M * N * K

    def call(self, i):
        F.matmul_dev(self.dw, self.K, self.N, self.dx, self.dy, self.M)

    def kernel(self, i):
        F.matmul_prepared_dev(self.dw, self.K, self.N, self.prep, self.dy, self.M)

    def free(self):
        for b in (self.dw, self.dy, self.prep):
            b.close()


def _stream_legs(ev, st, path, n_blocks, products, legs, passes, block_wbytes, block_flop, fused_block=None):
    """Time passes over n_blocks blocks of the pack at `path` through the
    trunk: per block acquire_dev(L), prefetch_dev(L+1), then the block's
    products (`products(view)` enqueues them) or `fused_block(view)`.
    legs: (label, host_budget, dev_budget, compute, fused)."""
    res = {}

    def run_pass(tr, compute, fused):
        for L in range(n_blocks):
            d = tr.acquire_dev(L)
            if d is None:
                raise F.Fh3Error(F.FH3_E_IO, F.lib().fh3_hip_last_error().decode())
            tr.prefetch_dev((L + 1) % n_blocks)
            if compute:
                (fused_block if fused else products)(tr.layer(L, d))

    for label, host_budget, dev_budget, compute, fused in legs:
        with F.Trunk(path, host_budget) as tr:
            a0 = time.perf_counter()
            tr.attach_device(dev_budget)
            attach_s = time.perf_counter() - a0
            # one untimed pass, then the timed passes right behind it with no
            # synchronisation between: the pipeline (reads, uploads, products)
            # is in its steady state when the GPU reaches the start event
            run_pass(tr, compute, fused)
            u0, h0 = tr.dev_stats().uploads, tr.stats()
            ms = ev.time_ms(lambda i: run_pass(tr, compute, fused), passes, st)
            F.synchronize()
            ups = tr.dev_stats().uploads - u0
            h1 = tr.stats()
        per_block = ms / n_blocks
        entry = {"ms_per_block": round(per_block, 3), "uploads_per_pass": ups // passes}
        if host_budget == 0:
            nb = passes * n_blocks
            entry["host_reads_per_pass"] = (h1.misses - h0.misses) // passes
            entry["read_ms_per_block"] = round((h1.read_s - h0.read_s) * 1e3 / nb, 3)
            entry["wait_ms_per_block"] = round((h1.wait_s - h0.wait_s) * 1e3 / nb, 3)
            entry["read_GBps"] = round(block_wbytes / max(1e-9, (h1.read_s - h0.read_s) / nb) / 1e9, 1)
        if dev_budget:
            entry["attach_s"] = round(attach_s, 3)
            entry["attach_GBps"] = round(n_blocks * block_wbytes / attach_s / 1e9, 1)
        if compute:
            entry["TFLOPs"] = round(block_flop / (per_block * 1e-3) / 1e12, 1)
        else:
            entry["upload_GBps"] = round(block_wbytes / (per_block * 1e-3) / 1e9, 1)
        res[label] = entry
        log("[bench] DiT blocks %s: %.3f ms/block %s" % (label, per_block, entry))
    return res


def dit_blocks_streamed(ev, st, n_blocks=8, M=16384, passes=2):
    """Eight synthetic DiT blocks (QKV 15360x5120, out 5120x5120, fc1 = up|gate
    27648x5120, fc2 = down 5120x13824; 178.4 MB of Q4_K each) written to an
    FH3P pack, held in page-locked host memory by the trunk and streamed
    through two device slots (hipMemcpyAsync on the upload stream), M = 16384
    tokens.  Per block: acquire_dev(L), prefetch_dev(L+1), the four
    fh3_hip_matmul_dev calls.  Timed beside the same blocks resident in HBM,
    beside the uploads alone, streamed as the block's fused sequence
    (norm1+modulate prep -> qkv; out-proj with the gate residual into h;
    norm2+modulate prep -> fc1 with SwiGLU -> fc2 with the gate residual, the
    attention output standing in for its input), and read from the pack file
    by the trunk's worker into the host ring (host budget 0: disk -> host ring
    -> device slots), with and without the products."""
    import tempfile
    from fasth3inc_amd import pack as P
    hidden, qkv, mlp = 5120, 15360, 13824
    specs = P.dit_block_specs(hidden=hidden, qkv_out=qkv, mlp_hidden=mlp)
    q4 = [s for s in specs if s.qtype == F.FH3_QUANT_Q4_K]
    block_wbytes = sum(s.nbytes for s in q4)
    block_flop = sum(2.0 * M * s.ne1 * s.ne0 for s in q4)
    path = os.path.join(tempfile.gettempdir(), "fh3_bench_dit_%d.fh3p" % os.getpid())
    t0 = time.perf_counter()
    P.write_pack(path, n_blocks, specs, lambda L: P.synth_dit_block(specs, 5, L))
    log("[bench] DiT pack: %d blocks x %.1f MB written in %.1fs" % (n_blocks, block_wbytes / 1e6,
                                                                     time.perf_counter() - t0))
    try:
        xa = F.DeviceBuffer.from_array(F.synth_x("outliers", 5, 1, M, hidden))
        xm = F.DeviceBuffer.from_array(F.synth_x("silu_gated", 5, 2, M, mlp))
        ys = [F.DeviceBuffer(M * n * 4) for n in (qkv, hidden, 2 * mlp, hidden)]
        h = F.DeviceBuffer.from_array(F.synth_x("normal", 5, 3, M, hidden))
        mods = [F.DeviceBuffer.from_array(0.1 * F.synth_x("normal", 5, 10 + i, M, hidden)) for i in range(3)]
        prep = F.DeviceBuffer(F.prepared_bytes(M, hidden))
        act = F.DeviceBuffer(M * mlp * 4)
        res = {"blocks": n_blocks, "M": M, "block_weight_bytes": block_wbytes, "block_flop": block_flop,
               "shapes": "qkv 5120->15360, out 5120->5120, fc1 (up|gate) 5120->27648, fc2 (down) 13824->5120"}

        shift, scale, gate = mods

        def fused_block(v):
            F.prepare_x_norm_dev(h, M, hidden, v.norm1.data, 1e-6, prep, shift, scale)
            F.matmul_prepared_dev(v.qkv.data, hidden, qkv, prep, ys[0], M)
            F.matmul_epi_dev(v.out.data, hidden, hidden, xa, M, F.EPI_GATE_RESIDUAL, h, gate)
            F.prepare_x_norm_dev(h, M, hidden, v.norm2.data, 1e-6, prep, shift, scale)
            F.matmul_prepared_epi_dev(v.fc1.data, hidden, 2 * mlp, prep, M, F.EPI_SWIGLU, act)
            F.matmul_epi_dev(v.fc2.data, mlp, hidden, act, M, F.EPI_GATE_RESIDUAL, h, gate)

        def products(v):
            for w, x, y in ((v.qkv, xa, ys[0]), (v.out, xa, ys[1]), (v.fc1, xa, ys[2]), (v.fc2, xm, ys[3])):
                F.matmul_dev(w.data, w.in_, w.out, x, y, M)

        legs = (("streamed", 1 << 40, 0, True, False), ("resident", 1 << 40, 1 << 40, True, False),
                ("uploads_only", 1 << 40, 0, False, False), ("streamed_fused_block", 1 << 40, 0, True, True),
                ("disk_ring", 0, 0, True, False), ("disk_ring_uploads_only", 0, 0, False, False))
        res.update(_stream_legs(ev, st, path, n_blocks, products, legs, passes, block_wbytes, block_flop,
                                fused_block))
        res["unhidden_upload_ms_per_block"] = round(res["streamed"]["ms_per_block"] -
                                                    res["resident"]["ms_per_block"], 3)
        res["fused_ops_ms_per_block"] = round(res["streamed_fused_block"]["ms_per_block"] -
                                              res["streamed"]["ms_per_block"], 3)
        # the disk ring's block time beyond the larger of its two inputs: the
        # products alone (resident) and reading plus uploading alone
        res["disk_ring_unhidden_ms_per_block"] = round(
            res["disk_ring"]["ms_per_block"] - max(res["resident"]["ms_per_block"],
                                                   res["disk_ring_uploads_only"]["ms_per_block"]), 3)
        for b in [xa, xm, h, prep, act] + ys + mods:
            b.close()
        return res
    finally:
        os.unlink(path)


def real_dit_blocks_streamed(ev, st, n_blocks=4, Ms=(3016, 16384), passes=2):
    """The real model's block (src/cli/fh3_cli.c:935-941: qkv 5376 -> 21504,
    gate_compress 5376 -> 7168, out 7168 -> 5376, fc1 5376 -> 28672, fc2
    14336 -> 5376; 238.4 MB of Q4_K per block, 238.5 MB with the norm weights,
    docs/data/census.json:17),
    streamed from page-locked host memory through the two device slots beside
    the same blocks resident in HBM, at the CLI's default sequence (3016
    tokens) and at 16384 tokens."""
    import tempfile
    from fasth3inc_amd import pack as P
    specs = P.real_dit_block_specs()
    q4 = [s for s in specs if s.qtype == F.FH3_QUANT_Q4_K]
    block_wbytes = sum(s.nbytes for s in q4)
    path = os.path.join(tempfile.gettempdir(), "fh3_bench_dit_real_%d.fh3p" % os.getpid())
    t0 = time.perf_counter()
    P.write_pack(path, n_blocks, specs, lambda L: P.synth_dit_block(specs, 6, L))
    log("[bench] real DiT pack: %d blocks x %.1f MB written in %.1fs" % (n_blocks, block_wbytes / 1e6,
                                                                          time.perf_counter() - t0))
    out = {"blocks": n_blocks, "block_weight_bytes": block_wbytes,
           "shapes": "qkv 5376->21504, gate_compress 5376->7168, out 7168->5376, fc1 5376->28672, "
                     "fc2 14336->5376"}
    try:
        for M in Ms:
            block_flop = sum(2.0 * M * s.ne1 * s.ne0 for s in q4)
            xs = {K: F.DeviceBuffer.from_array(F.synth_x("normal", 6, K, M, K)) for K in sorted({s.ne0 for s in q4})}
            ys = {s.suffix: F.DeviceBuffer(M * s.ne1 * 4) for s in q4}
            names = ("qkv", "gate_compress", "out", "fc1", "fc2")

            def products(v, M=M, xs=xs, ys=ys):
                for name, s in zip(names, q4):
                    w = getattr(v, name)
                    F.matmul_dev(w.data, w.in_, w.out, xs[w.in_], ys[s.suffix], M)

            legs = (("streamed", 1 << 40, 0, True, False), ("resident", 1 << 40, 1 << 40, True, False))
            r = _stream_legs(ev, st, path, n_blocks, products, legs, passes, block_wbytes, block_flop)
            r["block_flop"] = block_flop
            r["unhidden_upload_ms_per_block"] = round(r["streamed"]["ms_per_block"] -
                                                      r["resident"]["ms_per_block"], 3)
            out["M%d" % M] = r
            for b in list(xs.values()) + list(ys.values()):
                b.close()
        return out
    finally:
        os.unlink(path)


def te_other_types(ev, st, R=64):
    """The text encoder's long-row Q4_K products (o-projection 8192 -> 5120,
    down-projection 25600 -> 5120) and its Q5_K / Q6_K tensors (Q5_K 5120 ->
    1024; Q6_K 5120 -> 1024, 8192 -> 5120, 25600 -> 5120) at M = 1, 16, 64 and
    300 tokens through fh3_hip_matmul_dev (Q4_K: k_gemv8, k_sweep in K slices,
    k_skinny or k_midm by shape, k_gemm at 300; Q6_K: k_sweep, Q5_K: k_skinny,
    and both k_gemm at 300, reading the blocks in place).  Q4_K weights are the seeded N(0, 0.02) encoding, the others random
    blocks with finite scales, all rotated over more than 256 MB of device
    copies; graph of R calls."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import helpers as H
    rows = []
    for name, K, N in (("Q4_K", 8192, 5120), ("Q4_K", 25600, 5120), ("Q5_K", 5120, 1024), ("Q6_K", 5120, 1024),
                       ("Q6_K", 8192, 5120), ("Q6_K", 25600, 5120)):
        t, _, bb, _ = H.QTYPES[name]
        rng = np.random.default_rng(t * 100 + K + N)
        if name == "Q4_K":
            raw = F.synth_q4k_weights(t, K + N, N, K, 0.02, 0.0)
        else:
            raw = H.random_blocks(rng, name, N, K, scale_lo=-12, scale_hi=-8)
        wb = raw.nbytes
        copies = max(2, -(-(MALL_BYTES + (64 << 20)) // wb))
        ws = [F.DeviceBuffer.from_array(raw)]
        for _ in range(copies - 1):
            b = F.DeviceBuffer(wb)
            F.lib().fh3_hip_memcpy_dtod(b.ptr, ws[0].ptr, wb)
            ws.append(b)
        for M in (1, 16, 64, 300):
            dx = F.DeviceBuffer.from_array(rng.standard_normal((M, K)).astype(np.float32))
            dy = F.DeviceBuffer(M * N * 4)

            def call(i, dx=dx, dy=dy, M=M):
                F.matmul_dev(ws[i % copies], K, N, dx, dy, M, qtype=t)

            for i in range(2):
                call(i)
            F.synchronize()
            g = F.capture(lambda: [call(i) for i in range(R)])
            g.launch()
            t_c = ev.time_ms(lambda i: g.launch(), 8, st) / R
            g.close()
            small = F.PATH_SWEEP if name == "Q6_K" and (M <= 16 or K >= 5120) else F.PATH_SKINNY
            path = F.matmul_path(M, K) if name == "Q4_K" else (small if M <= 64 else F.PATH_GEMM)
            rows.append({"type": name, "M": M, "K": K, "N": N, "path": path, "call_us": round(t_c * 1e3, 2),
                         "weight_GBps": round(wb / (t_c * 1e-3) / 1e9, 1),
                         "hbm_frac": round((wb + 4 * M * (K + N)) / (t_c * 1e-3) / HBM_PEAK, 4)})
            log("[bench] %s M=%d K=%d N=%d call %.2f us (%.0f GB/s of weights)"
                % (name, M, K, N, t_c * 1e3, wb / (t_c * 1e-3) / 1e9))
            dx.close()
            dy.close()
        for b in ws:
            b.close()
    return rows


def dit_attention(ev, st, n=16384, heads=40, hd=128, rot=96):
    """The DiT block's attention branch at the block shapes (hidden 5120 = 40
    heads of 128, n = 16384 tokens): fh3_hip_attention_qkv_dev reading q, k,
    v in place from a qkv projection output, with per-head q/k rmsnorm and
    rope3 on 96 channels (k_attn_prep), then the online-softmax product
    (k_attn_fwd).  FLOP = 4 n^2 hd heads (Q K^T and P V)."""
    inner = heads * hd
    qkv = F.DeviceBuffer.from_array(F.synth_x("normal", 3, 600, n, 3 * inner))
    w = F.DeviceBuffer.from_array(np.ones(hd, np.float32))
    ang = np.outer(np.arange(n, dtype=np.float64), 1e-2 * np.arange(1, rot // 2 + 1))
    ang = np.concatenate([ang, ang], axis=1)
    cs = F.DeviceBuffer.from_array(np.cos(ang).astype(np.float32))
    sn = F.DeviceBuffer.from_array(np.sin(ang).astype(np.float32))
    o = F.DeviceBuffer(n * inner * 4)
    try:
        def call(i):
            F.attention_qkv_dev(qkv, n, heads, hd, o, w, w, 1e-5, cs, sn, rot)
        for i in range(3):
            call(i)
        F.synchronize()
        ms = ev.time_ms(call, 5, st)
        flop = 4.0 * n * n * hd * heads
        ach = flop / (ms * 1e-3)
        res = {"n": n, "heads": heads, "head_dim": hd, "rot_dim": rot, "call_ms": round(ms, 4),
               "TFLOPs": round(ach / 1e12, 1)}
        roof = {"bound": "mfma", "achieved": round(ach / 1e12, 1), "peak": MFMA_F16_PEAK / 1e12, "unit": "TFLOP/s",
                "frac": round(ach / MFMA_F16_PEAK, 4), "traffic": None,
                "kernel": "k_attn_prep + k_attn_fwd (fh3_hip_attention_qkv_dev)",
                "note": "4*n^2*hd*heads per call over the call time (both launches); fp16 operands, fp32 "
                        "accumulation and softmax; peak is dense fp16 MFMA"}
        log("[bench] DiT attention n=%d heads=%d: %.3f ms (%.1f TFLOP/s)" % (n, heads, ms, ach / 1e12))
        return res, roof
    finally:
        for b in (qkv, w, cs, sn, o):
            b.close()


def dit_vsa(ev, st, heads=56, hd=128, rot=96, sparsity=0.8):
    """The DiT's default attention, video sparse attention, at two sequence
    shapes from the reference CLI's dimension rules (src/cli/fh3_cli.c:217-252;
    6 text tokens): its default 640x384, 39 frames (130 audio tokens, video
    grid 12x12x20, n = 3016) and 1024x576, 73 frames (244 audio tokens, grid
    22x18x32, n = 12922); 56 heads of 128 as the real model.  One call =
    fh3_hip_vsa_attention_qkv_dev from a qkv projection output with q/k
    rmsnorm, rope3 and the gate.  dense_equiv_TFLOPs = 4 n^2 hd heads / time:
    the rate dense attention would need to match it."""
    out = []
    for label, n_text, n_audio, grid in (("640x384x39f", 6, 130, (12, 12, 20)), ("1024x576x73f", 6, 244, (22, 18, 32))):
        nv = grid[0] * grid[1] * grid[2]
        n = n_text + n_audio + nv
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
        try:
            def call(i):
                F.vsa_attention_qkv_dev(qkv, gate, o, seq, heads, hd, sparsity, 64, w, w, 1e-5, cs, sn, rot)
            for i in range(3):
                call(i)
            F.synchronize()
            ms = ev.time_ms(call, 10, st)
            dense = 4.0 * n * n * hd * heads
            out.append({"shape": label, "n": n, "text": n_text, "audio": n_audio, "video_grid": list(grid),
                        "heads": heads, "head_dim": hd, "sparsity": sparsity, "call_ms": round(ms, 4),
                        "dense_equiv_TFLOPs": round(dense / (ms * 1e-3) / 1e12, 1)})
            log("[bench] DiT VSA %s n=%d: %.3f ms" % (label, n, ms))
        finally:
            for b in (qkv, gate, w, cs, sn, o):
                b.close()
    return out


# ---------------------------------------------------------------------------
# CPU baseline
# ---------------------------------------------------------------------------
def _time_cpu(H, lib, fn, raw, K, N, x, iters):
    H.matmul_with(lib, fn, raw, K, N, x)  # warmup
    ts = []
    for _ in range(iters):
        t0 = time.perf_counter()
        H.matmul_with(lib, fn, raw, K, N, x)
        ts.append(time.perf_counter() - t0)
    return min(ts), sum(ts) / len(ts)


CALIB = os.path.join(ROOT, "fasth3inc_amd", "lib", "fh3_calib")


def load_only_ceiling(wbytes, k_bytes, k_time_ms):
    """The least time one-launch kernels need for the step's weights on this
    GPU: the calibration program (a child process on the same GPU, after the
    timed GEMV work) streams each GEMV weight matrix with load-only kernels of
    two load forms and three grid sizes, weights rotated past the Infinity
    Cache, and reports the best mean time per launch; summed over the step's
    shapes.  None when the program is not built."""
    if not os.path.exists(CALIB):
        return None
    r = subprocess.run([CALIB, "gemv"], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    if r.returncode != 0:
        return {"error": r.stdout[-400:]}
    best = {int(m.group(1)): float(m.group(2))
            for m in re.finditer(r"^\s*(\d+) B best:\s+([\d.]+) us", r.stdout, re.M)}
    if any(b not in best for b in wbytes):
        return {"error": "no stream time for every weight size: " + r.stdout[-400:]}
    us = sum(best[b] for b in wbytes)
    return {"us_per_step": round(us, 2),
            "alg_GBps": round(k_bytes / (us * 1e-6) / 1e9, 1),
            "frac": round(k_bytes / (us * 1e-6) / HBM_PEAK, 4),
            "kernels_over_ceiling": round(k_time_ms * 1e3 / us, 3),
            "best_us_per_launch": {str(b): t for b, t in sorted(best.items())},
            "source": "fasth3inc_amd/lib/fh3_calib gemv: load-only stream per weight matrix, best of 8 or 1 "
                      "loads per trip at 256/512/1024 workgroups, mean of 40 back-to-back launches"}


def cpu_baseline(cases, iters=5, big_iters=2, sample_tokens=(128, 512)):
    """fh3's CPU matmul on this host's cores, as benchmarks/bench_matmul.c
    times it (1 warmup, then best and mean of N runs): the six GEMV shapes and
    the 64 x 4096 x 4096 product with N = 5; the DiT GEMMs (M = 8192 and
    32768) with N = 2 on a sample: one 64-row output tile per thread (the
    reference schedules its tiles statically over the threads and dequantises
    each tile once per call) at two token counts, the time per tile round
    extended linearly to the full M (dequant fixed, products in M) and
    multiplied by the full shape's rounds of tiles."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import helpers as H
    ref = H.load_ref()
    if ref is not None:
        lib, fn, kind = ref, "fh3_matmul", "reference"
    else:
        lib, fn, kind = H.load_oracle(), "fh3_oracle_matmul", "port"
    threads = H.load_oracle().fh3_oracle_threads()
    total_w, total_t, per = 0, 0.0, []
    for c in cases:
        best, mean = _time_cpu(H, lib, fn, c.raw, c.K, c.N, c.x, iters)
        total_w += c.wbytes
        total_t += best
        per.append({"M": c.M, "N": c.N, "K": c.K, "ms": round(best * 1e3, 3), "mean_ms": round(mean * 1e3, 3),
                    "weight_GBps": round(c.wbytes / best / 1e9, 2)})
    configs = {}
    # single 64 x 4096 x 4096 product (same seeds as the GPU leg)
    raw = F.synth_q4k_weights(0, 300 + 4096 + 4096, 4096, 4096, 0.02, 0.0)
    x = F.synth_x("normal", 0, 400 + 4096, 64, 4096)
    best, mean = _time_cpu(H, lib, fn, raw, 4096, 4096, x, iters)
    flop = 2.0 * 64 * 4096 * 4096
    configs["single_64x4096x4096"] = {"ms": round(best * 1e3, 3), "mean_ms": round(mean * 1e3, 3),
                                      "GFLOPs": round(flop / best / 1e9, 1),
                                      "weight_GBps": round(q4k_bytes(4096, 4096) / best / 1e9, 2)}
    # DiT GEMMs on a sample (same weights and activation seeds as the GPU leg)
    big = [("attn_qkv", 8192, 5120, 15360, "outliers", 0.0), ("attn_out", 8192, 5120, 5120, "outliers", 0.0),
           ("mlp_up_gate", 32768, 5120, 13824, "normal", 2.0), ("mlp_down", 32768, 13824, 5120, "silu_gated", 2.0)]
    rows = []
    m1, m2 = sample_tokens
    for name, M, K, N, xk, spread in big:
        ns = min(N, 64 * threads)                     # one tile per thread
        rounds = -(-(-(-N // 64)) // threads)          # rounds of tiles over the threads at full N
        raw = F.synth_q4k_weights(1, 300 + N + K, N, K, 0.02, spread)[:ns * q4k_bytes(1, K)]
        x = F.synth_x(xk, 1, 400 + K, m2, K)
        t1, _ = _time_cpu(H, lib, fn, raw, K, ns, x[:m1], big_iters)
        t2, mean2 = _time_cpu(H, lib, fn, raw, K, ns, x, big_iters)
        full = (t1 + (t2 - t1) * (M - m1) / (m2 - m1)) * rounds
        rows.append({"name": name, "M": M, "K": K, "N": N, "sample_rows": ns, "sample_tokens": [m1, m2],
                     "sample_ms": [round(t1 * 1e3, 2), round(t2 * 1e3, 2)],
                     "GFLOPs": round(2.0 * M * N * K / full / 1e9, 1), "full_M_ms": round(full * 1e3, 1)})
        del raw, x
    configs["dit_gemms_sampled"] = rows
    cpu = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(total_w / total_t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": "the six GEMV shapes (best of %d after 1 warmup; value = their weight bytes over the sum "
                      "of best times), one weight copy; fh3_matmul from the reference's own fh3_quant.c and "
                      "fh3_ops.c with OMP_NUM_THREADS=%d; nproc=%d; %s; built -O3 -mavx2 -mfma -mf16c "
                      "-ffp-contract=off -fopenmp (no -march=native). configs: the 64x4096x4096 product "
                      "(best of %d) and the DiT GEMMs from one 64-row tile per thread at %d and %d tokens "
                      "(best of %d), extended linearly in M and by the rounds of tiles at full N"
                      % (iters, threads, os.cpu_count(), cpu, iters, m1, m2, big_iters),
            "per_case": per, "configs": configs}


# ---------------------------------------------------------------------------
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="skip the M=32768 MLP GEMMs")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-stream", action="store_true", help="skip the streamed DiT blocks")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(--gpus %d requested)" % args.gpus, file=sys.stderr)
        sys.exit(2)
    F.init(0)
    st = F.stream()
    ev = HipEvents()

    # ---------------- headline: small-M GEMV -------------------------------
    log("[bench] building GEMV shapes")
    gemv = [Gemv(M, 5120, N, seed=0) for N in (5120, 17408) for M in (1, 4, 16)]
    F.synchronize()

    # The timed steps are one HIP graph holding exactly `steps` consecutive
    # steps: step s is the six fh3_hip_matmul_dev calls (activation prep +
    # product kernel each) on weight copy s % copies of every shape.  Graph
    # replay removes the Python and per-call host launch cost from the timed
    # region, and one graph for all the steps removes the gap every graph
    # launch adds (about 4.7 us here, reported as ms_per_step_graph_per_step);
    # the device work is the same as eager calls (ms_per_step_eager).
    G = max(c.copies for c in gemv)

    def step(s):
        for c in gemv:
            c.call(s)

    for s in range(G):          # eager warmup (sizes the library workspace)
        step(s)
    F.synchronize()
    warm = F.capture(lambda: [step(s) for s in range(args.warmup)]) if args.warmup > 0 else None
    timed = F.capture(lambda: [step(s) for s in range(args.steps)])
    if warm is not None:
        warm.launch()
    F.synchronize()
    t0 = time.perf_counter()
    ms_step = ev.time_ms(lambda i: timed.launch(), 1, st) / args.steps
    F.synchronize()
    wall = time.perf_counter() - t0
    step_wbytes = sum(c.wbytes for c in gemv)
    value = step_wbytes / (ms_step * 1e-3) / 1e9
    log("[bench] GEMV step %.4f ms -> %.1f GB/s (wall %.2fs)" % (ms_step, value, wall))
    for g in (warm, timed):
        if g is not None:
            g.close()
    ms_eager = ev.time_ms(step, args.steps, st)
    log("[bench] GEMV step eager (python launches) %.4f ms" % ms_eager)
    graphs = [F.capture(lambda s=s: step(s)) for s in range(G)]
    for s in range(G):
        graphs[s].launch()
    ms_graph_step = ev.time_ms(lambda s: graphs[s % G].launch(), args.steps, st)
    log("[bench] GEMV step, one graph launch per step %.4f ms" % ms_graph_step)
    for g in graphs:
        g.close()

    per_gemv = []
    k_bytes, k_time = 0, 0.0
    R = 64
    for c in gemv:
        gk = F.capture(lambda c=c: [c.kernel(i) for i in range(R)])
        gc = F.capture(lambda c=c: [c.call(i) for i in range(R)])
        gk.launch()
        gc.launch()
        t_k = ev.time_ms(lambda i: gk.launch(), 8, st) / R
        t_c = ev.time_ms(lambda i: gc.launch(), 8, st) / R
        gk.close()
        gc.close()
        k_bytes += c.alg_bytes
        k_time += t_k
        per_gemv.append({"M": c.M, "K": c.K, "N": c.N, "kernel_us": round(t_k * 1e3, 2),
                         "call_us": round(t_c * 1e3, 2),
                         "kernel_weight_GBps": round(c.wbytes / (t_k * 1e-3) / 1e9, 1),
                         "kernel_alg_GBps": round(c.alg_bytes / (t_k * 1e-3) / 1e9, 1),
                         "hbm_frac": round(c.alg_bytes / (t_k * 1e-3) / HBM_PEAK, 4),
                         "copies": c.copies})
        log("[bench] GEMV M=%d N=%d kernel %.2f us call %.2f us" % (c.M, c.N, t_k * 1e3, t_c * 1e3))
    achieved = k_bytes / (k_time * 1e-3)
    roofline = {"bound": "hbm", "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK, 4), "traffic": TRAFFIC_GEMV_MEAN,
                "traffic_over_algorithmic": round(TRAFFIC_GEMV_MEAN / (k_bytes / len(gemv)), 3),
                "kernel": "k_gemv8 (n_tok<=4) and k_sweep (n_tok<=16), fh3_hip_matmul_prepared_dev",
                "note": "algorithmic bytes N*K/256*144 + 4MK + 4MN per launch over the mean launch time "
                        "(graph of 64 back-to-back launches, rotating weight copies) of the six shapes"}

    try:
        roofline["load_only_ceiling"] = load_only_ceiling([c.wbytes for c in gemv], k_bytes, k_time)
    except Exception as e:  # the calibration is context, not the measurement
        roofline["load_only_ceiling"] = {"error": repr(e)}
    if roofline["load_only_ceiling"] and "us_per_step" in roofline["load_only_ceiling"]:
        log("[bench] load-only ceiling of the six weight matrices: %.2f us per step (kernels %.2fx)" % (
            roofline["load_only_ceiling"]["us_per_step"], roofline["load_only_ceiling"]["kernels_over_ceiling"]))

    cpu = None if args.no_cpu else cpu_baseline(gemv)
    if cpu:
        log("[bench] CPU baseline %.2f GB/s (%s, %d threads)" % (cpu["value"], cpu["kind"], cpu["cores"]))
    for c in gemv:
        for b in c.w:
            b.close()
    del gemv

    # ---------------- M=64 single matmul (4096 x 4096) ---------------------
    extra = {}
    g1 = Gemm("single_64x4096x4096", 64, 4096, 4096, "normal", 0.0, seed=0)
    for i in range(10):
        g1.call(i)
    t_k = ev.time_ms(g1.kernel, 200, st)
    t_c = ev.time_ms(g1.call, 200, st)
    # roofline: HBM-bound at this size (2.1 GFLOP on 9.4 MB of weights); the
    # one weight copy is warm in the Infinity Cache after the first call
    alg1 = q4k_bytes(4096, 4096) + 4 * 64 * 4096 * 2
    extra["single_matmul_M64"] = {"M": 64, "K": 4096, "N": 4096, "path": F.matmul_path(64, 4096),
                                  "kernel_us": round(t_k * 1e3, 2), "call_us": round(t_c * 1e3, 2),
                                  "kernel_TFLOPs": round(g1.flop / (t_k * 1e-3) / 1e12, 2),
                                  "call_TFLOPs": round(g1.flop / (t_c * 1e-3) / 1e12, 2),
                                  "roofline": {"bound": "hbm", "achieved": round(alg1 / (t_k * 1e-3) / 1e9, 1),
                                               "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                                               "frac": round(alg1 / (t_k * 1e-3) / HBM_PEAK, 4),
                                               "mfma_frac": round(g1.flop / (t_k * 1e-3) / MFMA_F16_PEAK, 4),
                                               "note": "algorithmic bytes = Q4_K weights + fp32 x + fp32 y over "
                                                       "the kernel time (k_skinny, four token blocks)"}}
    g1.free()
    # the same product with the weights rotated over copies past the MALL, as
    # the GEMV shapes are timed (graph of 64 calls)
    c1 = Gemv(64, 4096, 4096, seed=0)
    c1.call(0)
    c1.kernel(0)
    F.synchronize()
    gk = F.capture(lambda: [c1.kernel(i) for i in range(64)])
    gc = F.capture(lambda: [c1.call(i) for i in range(64)])
    gk.launch()
    gc.launch()
    t_k = ev.time_ms(lambda i: gk.launch(), 4, st) / 64
    t_c = ev.time_ms(lambda i: gc.launch(), 4, st) / 64
    gk.close()
    gc.close()
    extra["single_matmul_M64"]["rotated"] = {"copies": c1.copies, "kernel_us": round(t_k * 1e3, 2),
                                             "call_us": round(t_c * 1e3, 2),
                                             "hbm_frac": round(alg1 / (t_k * 1e-3) / HBM_PEAK, 4)}
    for b in c1.w + [c1.dx, c1.dy, c1.prep]:
        b.close()
    log("[bench] 64x4096x4096: kernel %.2f us warm, %.2f us rotated" % (extra["single_matmul_M64"]["kernel_us"],
                                                                      t_k * 1e3))

    # ---------------- 17..64-token products (k_sweep with 2-4 token blocks) -
    # text-encoder prompt lengths between the headline's 16 and the GEMM's 65
    # tokens, at K = 5120 (graph of 32 calls, weights rotated past the MALL)
    prompt = []
    for N in (5120, 17408):
        for M in (17, 32, 48, 64):
            c = Gemv(M, 5120, N, seed=0)
            c.call(0)
            c.kernel(0)
            F.synchronize()
            gk = F.capture(lambda c=c: [c.kernel(i) for i in range(32)])
            gc = F.capture(lambda c=c: [c.call(i) for i in range(32)])
            gk.launch()
            gc.launch()
            t_k = ev.time_ms(lambda i: gk.launch(), 4, st) / 32
            t_c = ev.time_ms(lambda i: gc.launch(), 4, st) / 32
            gk.close()
            gc.close()
            prompt.append({"M": M, "K": 5120, "N": N, "path": F.matmul_path(M, 5120),
                           "kernel_us": round(t_k * 1e3, 2), "call_us": round(t_c * 1e3, 2),
                           "call_weight_GBps": round(c.wbytes / (t_c * 1e-3) / 1e9, 1)})
            for b in c.w + [c.dx, c.dy, c.prep]:
                b.close()
    extra["prompt_17_64_tokens"] = prompt
    log("[bench] 17..64 tokens: %s" % ", ".join("M=%d N=%d %.1f us" % (r["M"], r["N"], r["call_us"]) for r in prompt))

    # ---------------- few-hundred-token products (split-K GEMM path) -------
    # text-encoder prompt lengths: 65..512 tokens at K = 5120, where the GEMM
    # tiles alone would leave most CUs idle (128-token tiles up to 128 tokens,
    # and up to 256 while they are few; K split, then the ordered sum); graph
    # of 32 calls, weights rotated past the MALL, beside the 64-token call
    mid = []
    for N in (5120, 17408):
        for M in (64, 65, 96, 128, 192, 256, 512):
            c = Gemv(M, 5120, N, seed=0)
            c.call(0)
            c.kernel(0)
            F.synchronize()
            gk = F.capture(lambda c=c: [c.kernel(i) for i in range(32)])
            gc = F.capture(lambda c=c: [c.call(i) for i in range(32)])
            gk.launch()
            gc.launch()
            t_k = ev.time_ms(lambda i: gk.launch(), 4, st) / 32
            t_c = ev.time_ms(lambda i: gc.launch(), 4, st) / 32
            gk.close()
            gc.close()
            flop = 2.0 * M * N * 5120
            mid.append({"M": M, "K": 5120, "N": N, "path": F.matmul_path(M, 5120), "kernel_us": round(t_k * 1e3, 2),
                        "call_us": round(t_c * 1e3, 2), "call_TFLOPs": round(flop / (t_c * 1e-3) / 1e12, 1)})
            for b in c.w + [c.dx, c.dy, c.prep]:
                b.close()
    extra["gemm_few_hundred_tokens"] = mid
    log("[bench] 64..512 tokens: %s" % ", ".join("M=%d N=%d %.1f us" % (r["M"], r["N"], r["call_us"]) for r in mid))

    # ---------------- DiT GEMMs --------------------------------------------
    shapes = [("attn_qkv", 8192, 5120, 15360, "outliers", 0.0), ("attn_out", 8192, 5120, 5120, "outliers", 0.0)]
    if not args.quick:
        shapes += [("mlp_up", 32768, 5120, 13824, "normal", 2.0), ("mlp_gate", 32768, 5120, 13824, "normal", 2.0),
                   ("mlp_down", 32768, 13824, 5120, "silu_gated", 2.0)]
    gemms = []
    best_frac, sum_flop, sum_t = 0.0, 0.0, 0.0
    shared_x = {}
    for name, M, K, N, xk, spread in shapes:
        log("[bench] GEMM %s M=%d K=%d N=%d" % (name, M, K, N))
        key = (M, K, xk)
        g = Gemm(name, M, K, N, xk, spread, seed=1, x_dev=shared_x.get(key))
        shared_x[key] = g.dx
        # a few untimed launches first: the shader clock ramps up over the
        # first milliseconds of sustained MFMA work
        for i in range(3):
            g.call(i)
            g.kernel(i)
        F.synchronize()
        reps = 20
        t_k = ev.time_ms(g.kernel, reps, st)
        t_c = ev.time_ms(g.call, reps, st)
        tf_k = g.flop / (t_k * 1e-3) / 1e12
        gemms.append({"name": name, "M": M, "K": K, "N": N, "kernel_ms": round(t_k, 4), "call_ms": round(t_c, 4),
                      "kernel_TFLOPs": round(tf_k, 1), "call_TFLOPs": round(g.flop / (t_c * 1e-3) / 1e12, 1),
                      "mfma_frac": round(tf_k * 1e12 / MFMA_F16_PEAK, 4)})
        sum_flop += g.flop
        sum_t += t_k
        log("[bench]   kernel %.3f ms (%.1f TFLOP/s) call %.3f ms" % (t_k, tf_k, t_c))
        g.free()
    shared_x.clear()
    ach = sum_flop / (sum_t * 1e-3)
    roofline_gemm = {"bound": "mfma", "achieved": round(ach / 1e12, 1), "peak": MFMA_F16_PEAK / 1e12,
                     "unit": "TFLOP/s", "frac": round(ach / MFMA_F16_PEAK, 4),
                     "traffic": TRAFFIC_GEMM["attn_qkv"], "traffic_kernel": "k_gemm attn_qkv M=8192 N=15360",
                     "kernel": "k_gemm (fh3_hip_matmul_prepared_dev, n_tok>64)",
                     "note": "2*M*N*K per launch over launch time, summed over the DiT GEMMs; "
                             "fp16 operands, fp32 accumulation; peak is dense fp16 MFMA"}
    extra["dit_gemms"] = gemms
    attn = [g for g in gemms if g["name"].startswith("attn")]
    mlp = [g for g in gemms if g["name"].startswith("mlp")]
    extra["dit_attn_linears_ms"] = round(sum(g["call_ms"] for g in attn), 4)
    if mlp:
        extra["dit_mlp_linears_ms"] = round(sum(g["call_ms"] for g in mlp), 4)
    extra["gemv"] = per_gemv

    try:
        extra["te_long_rows_and_q5k_q6k"] = te_other_types(ev, st)
    except Exception as e:  # keep the headline line when this leg fails
        log("[bench] Q5_K / Q6_K leg failed: %r" % (e,))
        extra["te_long_rows_and_q5k_q6k"] = {"error": repr(e)}

    # ---------------- DiT attention branch ---------------------------------
    roofline_attn = None
    try:
        extra["dit_attention"], roofline_attn = dit_attention(ev, st)
    except Exception as e:  # keep the headline line when this leg fails
        log("[bench] DiT attention failed: %r" % (e,))
        extra["dit_attention"] = {"error": repr(e)}

    try:
        extra["dit_vsa"] = dit_vsa(ev, st)
    except Exception as e:  # keep the headline line when this leg fails
        log("[bench] DiT VSA failed: %r" % (e,))
        extra["dit_vsa"] = {"error": repr(e)}

    # ---------------- DiT blocks streamed through the trunk ----------------
    if not args.no_stream:
        try:
            extra["dit_blocks_streamed"] = dit_blocks_streamed(ev, st)
        except Exception as e:  # keep the headline line when this leg fails
            log("[bench] DiT streamed blocks failed: %r" % (e,))
            extra["dit_blocks_streamed"] = {"error": repr(e)}
        try:
            extra["real_dit_blocks_streamed"] = real_dit_blocks_streamed(ev, st)
        except Exception as e:
            log("[bench] real DiT streamed blocks failed: %r" % (e,))
            extra["real_dit_blocks_streamed"] = {"error": repr(e)}

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "ms_per_step_eager": round(ms_eager, 5),
        "ms_per_step_graph_per_step": round(ms_graph_step, 5),
        "higher_is_better": True,
        "vs_baseline": None,
        "dtype": "i8 x i8 -> i32 (1-4 tokens: Q4_K nibbles x int16 activations as two int8 planes) and "
                 "f16 x f16 -> f32 (16 tokens: exact sc*q x fp16 activations); Q4_K weights, fp32 activations "
                 "and outputs",
        "data": "synthetic: Philox-seeded N(0,0.02) weights Q4_K-encoded, N(0,1) activations",
        "config": {"workload": "small-M GEMV, text-encoder shapes: M in {1,4,16}, K=5120, N in {5120,17408}; "
                               "one step = one fh3_hip_matmul_dev per shape, weights rotated over >256 MB of "
                               "device copies", "parallelism": "single GPU"},
        "roofline": roofline,
        "roofline_gemm": roofline_gemm,
        "roofline_attention": roofline_attn,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
