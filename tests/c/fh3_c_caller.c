/*
 * fh3_c_caller.c -- a C99 caller of libfh3hip.so through the headers of include/fh3 only,
 * the way the reference's own programs call its CPU library.
 *
 *   fh3_c_caller matmul_ref <tests/golden/matmul_ref.bin>
 *       The checks of the reference's tests/unit/test_matmul.c:103-156:
 *       fh3_matmul_scalar == fh3_matmul_avx2 == fh3_matmul bit for bit, with
 *       and without bias, and rel-L2 against the fixture's fp64 reference
 *       (the GPU gate, 2e-3, in place of the CPU's 1e-6).
 *   fh3_c_caller bench [n_tok] [iters]
 *       The calls of the reference's benchmarks/bench_matmul.c: in 5376,
 *       out 14336, its constant Q4_K blocks, activation and bias patterns,
 *       one warm-up and `iters` timed fh3_matmul calls (host pointers, so W,
 *       x and y cross PCIe on every call), then the same with the weights
 *       registered once (fh3_hip_register_weights).  Every output row holds
 *       the same weights, so y[t][o] - bias[o] must be one value per token:
 *       checked, and that value against a double-precision sum over the
 *       dequantised block (rel-L2 <= 2e-3).
 *   fh3_c_caller patch [text] [audio] [video]
 *       The run-once patch embedding of the reference's DiT forward
 *       (src/model/fh3_dit.c:350-353): text rows copied into h, then
 *       fh3_matmul of 32-value audio rows and 96-value video rows (F16
 *       weights 5376 x 32 and 5376 x 96, F32 biases, as the GGUF holds them)
 *       written straight into h behind them.  Checks: the text rows are
 *       untouched, every other row of h is written, and each region against
 *       a double-precision product (rel-L2 <= 2e-3).
 *   fh3_c_caller trunk <pack.bin>
 *       fh3_trunk_open on an Fh3Trunk held by value on the stack, as the
 *       reference CLI holds it (src/cli/fh3_cli.c:750,963): the host scan,
 *       then the device extension on the same struct.
 * Prints one PASS line per check; exits non-zero on the first failure.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "fh3/fh3.h"
#include "fh3/fh3_hip.h"
#include "fh3/fh3_trunk.h"

#define CHECK(cond)                                                                         \
    do {                                                                                    \
        if (!(cond)) {                                                                      \
            fprintf(stderr, "[FAIL] %s:%d: %s (%s)\n", __FILE__, __LINE__, #cond,           \
                    fh3_hip_last_error());                                                  \
            return 1;                                                                       \
        }                                                                                   \
    } while (0)

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static double rel_l2(const float *a, const double *ref, size_t n) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < n; i++) {
        const double d = (double)a[i] - ref[i];
        num += d * d;
        den += ref[i] * ref[i];
    }
    return sqrt(num) / sqrt(den);
}

static int run_matmul_ref(const char *path) {
    FILE *fp = fopen(path, "rb");
    CHECK(fp != NULL);
    uint32_t h[5];
    CHECK(fread(h, sizeof(uint32_t), 5, fp) == 5);
    const int64_t in = h[1], out = h[2];
    const int n_tok = (int)h[3];
    CHECK(h[0] == FH3_QUANT_Q4_K && in == 5376 && out == 192 && n_tok == 37);
    const size_t yc = (size_t)n_tok * (size_t)out, xc = (size_t)n_tok * (size_t)in;
    uint8_t *wr = (uint8_t *)malloc(h[4]);
    float *x = (float *)malloc(xc * sizeof(float)), *bias = (float *)malloc((size_t)out * sizeof(float));
    float *yref = (float *)malloc(yc * sizeof(float));
    float *ys = (float *)malloc(yc * sizeof(float)), *ya = (float *)malloc(yc * sizeof(float));
    float *yo = (float *)malloc(yc * sizeof(float));
    double *yd = (double *)malloc(yc * sizeof(double));
    CHECK(wr && x && bias && yref && ys && ya && yo && yd);
    CHECK(fread(wr, 1, h[4], fp) == h[4]);
    CHECK(fread(x, sizeof(float), xc, fp) == xc);
    CHECK(fread(bias, sizeof(float), (size_t)out, fp) == (size_t)out);
    CHECK(fread(yref, sizeof(float), yc, fp) == yc);
    fclose(fp);
    Fh3W w;
    w.type = FH3_QUANT_Q4_K;
    w.in = in;
    w.out = out;
    w.data = wr;

    fh3_matmul_scalar(&w, x, ys, n_tok, bias);
    fh3_matmul_avx2(&w, x, ya, n_tok, bias);
    fh3_matmul(&w, x, yo, n_tok, bias);
    CHECK(memcmp(ys, ya, yc * sizeof(float)) == 0);
    CHECK(memcmp(ys, yo, yc * sizeof(float)) == 0);
    printf("PASS matmul_scalar_eq_avx2_eq_omp (%zu outputs bitwise identical)\n", yc);
    fh3_matmul_scalar(&w, x, ys, n_tok, NULL);
    fh3_matmul_avx2(&w, x, ya, n_tok, NULL);
    fh3_matmul(&w, x, yo, n_tok, NULL);
    CHECK(memcmp(ys, ya, yc * sizeof(float)) == 0);
    CHECK(memcmp(ys, yo, yc * sizeof(float)) == 0);
    printf("PASS matmul_scalar_eq_avx2_eq_omp (nobias)\n");
    fh3_matmul(&w, x, yo, n_tok, bias);
    for (size_t i = 0; i < yc; i++) yd[i] = (double)yref[i];
    const double err = rel_l2(yo, yd, yc);
    CHECK(err <= 2e-3);
    printf("PASS matmul_matches_numpy rel_l2=%.3e (gate 2e-3)\n", err);
    free(wr), free(x), free(bias), free(yref), free(ys), free(ya), free(yo), free(yd);
    return 0;
}

static int run_bench(int n_tok, int iters) {
    const int64_t in = 5376, out = 14336;
    const size_t rb = fh3_row_bytes(FH3_QUANT_Q4_K, in);
    const size_t wbytes = (size_t)out * rb, xc = (size_t)n_tok * (size_t)in, yc = (size_t)n_tok * (size_t)out;
    uint8_t *wd = (uint8_t *)malloc(wbytes);
    float *x = (float *)malloc(xc * sizeof(float)), *bias = (float *)malloc((size_t)out * sizeof(float));
    float *y = (float *)malloc(yc * sizeof(float));
    CHECK(wd && x && bias && y);
    const uint16_t d_val = 0x3800, dmin_val = 0x2c00; /* fp16 0.5 and 0.0625 */
    for (size_t b = 0; b < wbytes / 144; b++) {
        uint8_t *blk = wd + b * 144;
        memcpy(blk, &d_val, 2);
        memcpy(blk + 2, &dmin_val, 2);
        memset(blk + 4, 0x12, 12);
        memset(blk + 16, 0x34, 128);
    }
    for (size_t i = 0; i < xc; i++) x[i] = ((float)(i % 100) - 50.0f) * 0.001f;
    for (int64_t i = 0; i < out; i++) bias[i] = ((float)(i % 10) - 5.0f) * 0.01f;
    Fh3W w;
    w.type = FH3_QUANT_Q4_K;
    w.in = in;
    w.out = out;
    w.data = wd;
    const double gflop = 2.0 * (double)in * (double)out * (double)n_tok / 1e9;

    for (int reg = 0; reg < 2; reg++) {
        if (reg) CHECK(fh3_hip_register_weights(wd, wbytes, NULL) == FH3_OK);
        double t0 = now_s();
        fh3_matmul(&w, x, y, n_tok, bias);
        const double warm = now_s() - t0;
        double best = 1e30, total = 0.0;
        for (int it = 0; it < iters; it++) {
            t0 = now_s();
            fh3_matmul(&w, x, y, n_tok, bias);
            const double dt = now_s() - t0;
            total += dt;
            if (dt < best) best = dt;
        }
        printf("bench_matmul in=%lld out=%lld n_tok=%d %s: warm-up %.4f s, best %.4f s (%.1f GFLOP/s), "
               "mean %.4f s (%.1f GFLOP/s)\n", (long long)in, (long long)out, n_tok,
               reg ? "weights registered" : "host weights", warm, best, gflop / best, total / iters,
               gflop * iters / total);
    }
    CHECK(fh3_hip_unregister_weights(wd) == FH3_OK);

    /* every row holds the same super-block: y[t][o] - bias[o] is one value per token */
    float blk[256];
    fh3_dequant(FH3_QUANT_Q4_K, wd, blk, 256);
    double *want = (double *)malloc((size_t)n_tok * sizeof(double));
    float *got = (float *)malloc((size_t)n_tok * sizeof(float));
    CHECK(want && got);
    for (int t = 0; t < n_tok; t++) {
        double s = 0.0;
        for (int64_t k = 0; k < in; k++) s += (double)x[(size_t)t * in + k] * (double)blk[k % 256];
        want[t] = s;
        got[t] = y[(size_t)t * out] - bias[0];
        for (int64_t o = 1; o < out; o++) {
            const float v = y[(size_t)t * out + o] - bias[o];
            CHECK(fabs((double)v - (double)got[t]) <= 1e-5 * (fabs(want[t]) + 1e-3));
        }
    }
    const double err = rel_l2(got, want, (size_t)n_tok);
    CHECK(err <= 2e-3);
    printf("PASS bench_matmul output: rows agree, rel_l2 %.3e against the fp64 sum\n", err);
    free(wd), free(x), free(bias), free(y), free(want), free(got);
    return 0;
}

/* IEEE half -> double (finite values only: the weights below are finite). */
static double half_to_double(uint16_t h) {
    const int e = (h >> 10) & 31, m = h & 1023;
    const double v = e ? ldexp(1.0 + m / 1024.0, e - 15) : ldexp(m / 1024.0, -14);
    return (h & 0x8000) ? -v : v;
}

/* double -> IEEE half, round to nearest, for |v| well inside the normal range. */
static uint16_t double_to_half(double v) {
    const uint16_t s = v < 0 ? 0x8000 : 0;
    v = fabs(v);
    if (v < ldexp(1.0, -14)) return s | (uint16_t)lrint(v * ldexp(1.0, 24));
    int e;
    const double f = frexp(v, &e); /* v = f * 2^e, f in [0.5, 1) */
    long mant = lrint((f * 2.0 - 1.0) * 1024.0);
    if (mant == 1024) mant = 0, e++;
    return s | (uint16_t)((e - 1 + 15) << 10) | (uint16_t)mant;
}

static uint32_t lcg_state = 12345u;
static double lcg_normal(void) { /* sum of 12 uniforms - 6 */
    double s = 0.0;
    for (int i = 0; i < 12; i++) {
        lcg_state = lcg_state * 1664525u + 1013904223u;
        s += (double)(lcg_state >> 8) / 16777216.0;
    }
    return s - 6.0;
}

static int run_patch(int T, int A, int V) {
    const int64_t hidden = 5376;
    const size_t rows = (size_t)(T + A + V);
    float *h = (float *)malloc(rows * (size_t)hidden * sizeof(float));
    CHECK(h != NULL);
    for (size_t i = 0; i < rows * (size_t)hidden; i++) h[i] = NAN;
    for (size_t i = 0; i < (size_t)T * (size_t)hidden; i++) h[i] = (float)lcg_normal();
    const int ins[2] = {32, 96}, toks[2] = {A, V}, r0s[2] = {T, T + A};
    uint16_t *wb[2];
    float *xs[2], *bs[2];
    for (int p = 0; p < 2; p++) {
        const int in = ins[p], n = toks[p];
        wb[p] = (uint16_t *)malloc((size_t)hidden * (size_t)in * sizeof(uint16_t));
        xs[p] = (float *)malloc((size_t)n * (size_t)in * sizeof(float));
        bs[p] = (float *)malloc((size_t)hidden * sizeof(float));
        CHECK(wb[p] && xs[p] && bs[p]);
        for (size_t i = 0; i < (size_t)hidden * (size_t)in; i++) wb[p][i] = double_to_half(0.05 * lcg_normal());
        for (size_t i = 0; i < (size_t)n * (size_t)in; i++) xs[p][i] = (float)lcg_normal();
        for (int64_t i = 0; i < hidden; i++) bs[p][i] = (float)(0.1 * lcg_normal());
    }
    float *text = (float *)malloc((size_t)T * (size_t)hidden * sizeof(float));
    CHECK(text != NULL);
    memcpy(text, h, (size_t)T * (size_t)hidden * sizeof(float));
    /* src/model/fh3_dit.c:352-353 */
    for (int p = 0; p < 2; p++) {
        Fh3W w;
        w.type = FH3_QUANT_F16;
        w.in = ins[p];
        w.out = hidden;
        w.data = (const uint8_t *)wb[p];
        fh3_matmul(&w, xs[p], h + (size_t)r0s[p] * (size_t)hidden, toks[p], bs[p]);
    }
    CHECK(memcmp(text, h, (size_t)T * (size_t)hidden * sizeof(float)) == 0);
    for (int p = 0; p < 2; p++) {
        const int in = ins[p], n = toks[p];
        const size_t cnt = (size_t)n * (size_t)hidden;
        double *ref = (double *)malloc(cnt * sizeof(double));
        CHECK(ref != NULL);
        for (int t = 0; t < n; t++)
            for (int64_t o = 0; o < hidden; o++) {
                double s = 0.0;
                for (int k = 0; k < in; k++)
                    s += (double)xs[p][(size_t)t * in + k] * half_to_double(wb[p][(size_t)o * in + k]);
                ref[(size_t)t * hidden + o] = s + (double)bs[p][o];
            }
        const float *got = h + (size_t)r0s[p] * (size_t)hidden;
        for (size_t i = 0; i < cnt; i++) CHECK(isfinite(got[i]));
        const double err = rel_l2(got, ref, cnt);
        CHECK(err <= 2e-3);
        printf("PASS patch projection in=%d tokens=%d out=%lld: rel_l2 %.3e against the fp64 product\n", in, n,
               (long long)hidden, err);
        free(ref);
    }
    for (int p = 0; p < 2; p++) free(wb[p]), free(xs[p]), free(bs[p]);
    free(h), free(text);
    return 0;
}

static int run_trunk(const char *path) {
    Fh3Trunk tr; /* by value, as the reference CLI holds it */
    CHECK(fh3_trunk_open(path, 0, &tr) == FH3_OK);
    CHECK(tr.num_layers > 0 && tr.npin == 0 && tr.ring_buf[0] && tr.ring_buf[1]);
    for (int pass = 0; pass < 2; pass++)
        for (int L = 0; L < tr.num_layers; L++) {
            if (L + 1 < tr.num_layers) fh3_trunk_prefetch(&tr, L + 1);
            const uint8_t *p = fh3_trunk_acquire(&tr, L);
            CHECK(p != NULL);
            const Fh3LayerView v = fh3_trunk_layer(&tr, L, p);
            CHECK(v.qkv.data == p + tr.pack.layers[L].tensors[0].offset_in_layer);
            CHECK(v.qkv.in == tr.pack.layers[L].tensors[0].in_dim);
        }
    const Fh3TrunkStats st = fh3_trunk_stats(&tr);
    CHECK(st.hits + st.misses == 2u * (uint64_t)tr.num_layers);
    printf("PASS trunk by value: %d layers, %llu hits, %llu misses, %llu bytes read\n", tr.num_layers,
           (unsigned long long)st.hits, (unsigned long long)st.misses, (unsigned long long)st.bytes_read);
    CHECK(fh3_trunk_attach_device(&tr, 0, NULL) == FH3_OK);
    for (int L = 0; L < tr.num_layers; L++) {
        const uint8_t *d = fh3_trunk_acquire_dev(&tr, L);
        CHECK(d != NULL);
        if (L + 1 < tr.num_layers) fh3_trunk_prefetch_dev(&tr, L + 1);
        const size_t n = (size_t)tr.pack.layers[L].size_bytes;
        uint8_t *back = (uint8_t *)malloc(n);
        const uint8_t *h = fh3_trunk_acquire(&tr, L);
        CHECK(back && h);
        CHECK(fh3_hip_memcpy_dtoh(back, d, n) == FH3_OK);
        CHECK(memcmp(back, h, n) == 0);
        free(back);
    }
    const Fh3TrunkDevStats ds = fh3_trunk_dev_stats(&tr);
    CHECK(ds.uploads == (uint64_t)tr.num_layers);
    printf("PASS trunk device slots on the same struct: %llu uploads, bytes identical\n",
           (unsigned long long)ds.uploads);
    fh3_trunk_close(&tr);
    return 0;
}

int main(int argc, char **argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s matmul_ref <file> | bench [n_tok] [iters] | patch [T] [A] [V] | trunk <pack>\n",
                argv[0]);
        return 2;
    }
    CHECK(fh3_hip_init(0) == FH3_OK);
    int rc = 2;
    if (!strcmp(argv[1], "matmul_ref") && argc >= 3)
        rc = run_matmul_ref(argv[2]);
    else if (!strcmp(argv[1], "bench"))
        rc = run_bench(argc >= 3 ? atoi(argv[2]) : 1024, argc >= 4 ? atoi(argv[3]) : 3);
    else if (!strcmp(argv[1], "patch"))
        rc = run_patch(argc >= 3 ? atoi(argv[2]) : 6, argc >= 4 ? atoi(argv[3]) : 130,
                       argc >= 5 ? atoi(argv[4]) : 2880);
    else if (!strcmp(argv[1], "trunk") && argc >= 3)
        rc = run_trunk(argv[2]);
    fh3_hip_shutdown();
    return rc;
}
