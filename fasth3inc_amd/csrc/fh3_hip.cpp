// fh3_hip.cpp -- the thin C-ABI layer of libfh3hip.so: device state, memory
// helpers, the device-resident matmul/dequant entry points (fh3_hip.h) and the
// reference-signature host wrappers fh3_matmul / fh3_dequant (fh3.h).
//
// There is deliberately no CPU compute path here: if the GPU cannot be used
// the call fails with a message instead of computing on the host.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "fh3/fh3.h"
#include "fh3/fh3_hip.h"
#include "fh3_kernels.h"
#include "fh3_hip_internal.h"

namespace {

struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
};

struct State {
    bool init = false;
    int device = -1;
    hipStream_t stream = nullptr;
    DevBuf ws;                      // x16 fragments + per-row scales
    DevBuf ws2;                     // x16 made from a prepared fp32 copy (other weight types)
    DevBuf w16;                     // fp16 rows of a weight of another type
    DevBuf part;                    // split-K partial sums of the middle-M kernel
    DevBuf attn;                    // fp16 attention operands (Qp, Kp, Vt)
    DevBuf vsa_ws;                  // VSA operands, tile statistics, scores and tile lists
    DevBuf vsa_geo;                 // VSA tile geometry of the last sequence shape
    int vsa_key[8] = {-1, -1, -1, -1, -1, -1, -1, -1};
    struct Reg {
        const uint8_t *host;
        size_t bytes;
        void *dev;
    };
    std::vector<Reg> regs;          // registered host weight ranges and their device copies
    int vsa_T = 0, vsa_P = 0;
    DevBuf st_w, st_x, st_y, st_b;  // staging for the host-pointer wrappers
    int path = FH3_HIP_PATH_AUTO;
    // Workspace buffers replaced while captured graphs exist stay allocated
    // (graphs hold their addresses) until the last graph is destroyed; after
    // a capture begun outside fh3_hip_graph_begin (a caller's own graph, whose
    // lifetime the library cannot see) they stay until fh3_hip_shutdown.
    int live_graphs = 0;
    bool foreign_capture = false;
    std::vector<void *> retired;
    std::recursive_mutex mu;
};

State g;
thread_local char g_err[512] = "";
// Set on a thread between fh3_hip_graph_begin and fh3_hip_graph_end.
thread_local bool t_own_capture = false;
// fh3_hip_free calls made on that thread meanwhile: a hipFree there would end
// the (thread-local) capture with an error, so they wait for
// fh3_hip_graph_end.
thread_local std::vector<void *> t_deferred_free;
// Device address of the fixed scratch array of fh3_kernels.hip, per device
// (bound once per device by fh3_hip_init).
void *g_scratch[64];

int set_err(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return set_err(e == hipErrorOutOfMemory ? FH3_E_NOMEM : FH3_ERR, "%s: %s", what, hipGetErrorString(e));
}

#define FH3_HIPCALL(expr)                                 \
    do {                                                  \
        hipError_t e_ = (expr);                           \
        if (e_ != hipSuccess) return hip_fail(e_, #expr); \
    } while (0)

int ensure_init() {
    if (g.init) return FH3_OK;
    const char *env = getenv("FH3_HIP_DEVICE");
    return fh3_hip_init(env ? atoi(env) : 0);
}

bool capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return st && hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// Give up b's allocation: freed once the device is idle (enqueued kernels may
// still read it), or kept until fh3_hip_graph_destroy has destroyed the last
// graph when captured graphs exist (their kernels hold its address).
int release(DevBuf &b) {
    if (b.p) {
        if (g.live_graphs > 0 || g.foreign_capture) {
            g.retired.push_back(b.p);
        } else {
            FH3_HIPCALL(hipDeviceSynchronize());
            FH3_HIPCALL(hipFree(b.p));
        }
    }
    b.p = nullptr;
    b.cap = 0;
    return FH3_OK;
}

// Grow-only device buffer.  A grow allocates, so it is refused while `st` is
// being captured into a graph: the call must have run once eagerly first.
int grow(DevBuf &b, size_t need, hipStream_t st) {
    const bool cap = capturing(st);
    // a graph the library does not own may now hold this buffer's address
    if (cap && !t_own_capture) g.foreign_capture = true;
    if (b.cap >= need) return FH3_OK;
    if (cap)
        return set_err(FH3_E_INVALID,
                       "the library workspace must grow to %zu bytes while the stream is captured into a graph; "
                       "run the call once eagerly before capturing it", need);
    int rc = release(b);
    if (rc != FH3_OK) return rc;
    FH3_HIPCALL(hipMalloc(&b.p, need));
    b.cap = need;
    return FH3_OK;
}

int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Longest row (in) any product takes: rows of up to fh3k_max_in() values that
// are whole super-blocks run the kernels that read Q4_K in place; other rows
// ("general rows": in % 256 != 0, or in > fh3k_max_in()) are decoded to fp16
// rows zero-padded to kpad(in) columns.
constexpr int64_t kMaxInGeneral = (int64_t)1 << 24;
bool general_rows(int64_t in) { return in % 256 != 0 || in > fh3k_max_in(); }
int64_t kpad(int64_t in) { return round_up(in, 256); }

// Kernel family of the fp16-row products (weights of another type than Q4_K,
// and general rows of any type): k_skinny16 up to 64 tokens on padded rows of
// at most fh3k_max_in() values, else k_gemm16.
int path16(int n_tok, int64_t in) {
    if (g.path == FH3_HIP_PATH_GEMM) return FH3_HIP_PATH_GEMM;
    return n_tok <= fh3k_skinny_max_tokens() && kpad(in) <= fh3k_max_in() ? FH3_HIP_PATH_SKINNY
                                                                            : FH3_HIP_PATH_GEMM;
}

// A forced path that cannot take the shape falls back to the automatic choice.
int choose_path(int n_tok, int64_t in) {
    if (general_rows(in)) return path16(n_tok, in);
    const bool g8 = in <= fh3k_max_in() && fh3k_gemv8_fits((int)in, n_tok);
    const bool sw = in <= fh3k_max_in() && fh3k_sweep_fits((int)in, n_tok);
    if (g.path == FH3_HIP_PATH_GEMV8 && g8) return FH3_HIP_PATH_GEMV8;
    if (g.path == FH3_HIP_PATH_SWEEP && sw) return FH3_HIP_PATH_SWEEP;
    if (g.path == FH3_HIP_PATH_SKINNY && n_tok <= fh3k_skinny_max_tokens()) return FH3_HIP_PATH_SKINNY;
    if (g.path == FH3_HIP_PATH_MIDM && n_tok <= fh3k_midm_max_tokens()) return FH3_HIP_PATH_MIDM;
    if (g.path == FH3_HIP_PATH_GEMM) return FH3_HIP_PATH_GEMM;
    if (g8) return FH3_HIP_PATH_GEMV8;
    // up to 16 tokens, and up to 64 on rows of at least 5120: the persistent
    // kernel that keeps the activations in registers, long rows in K slices
    // (measured 10-20 % faster than k_skinny at M = 16, K = 5120, 1.2-1.5x at
    // K = 25600; at 17..64 tokens 0-25 % faster than k_skinny and k_midm at
    // K = 5120, 1.1-1.4x over k_midm at K = 25600; at K = 4096 more than 16
    // tokens need a K split and the ordered sum, or (rows of at most 4096)
    // groups of 32 tokens with their own workgroups, and k_skinny, eight
    // wavefronts with the next super-block's activations loaded while one
    // computes, is 0-25 % faster at K = 1024-4096, N = 1024-4096)
    if (sw && (n_tok <= 16 || in >= 5120)) return FH3_HIP_PATH_SWEEP;
    // long rows (K >= 8192) with 17..64 tokens (when not taken above): the
    // split-K kernel reads the
    // activations once per 128 rows instead of once per 16 (measured 25-45 %
    // faster at K = 13824; slower than k_skinny at K <= 5120)
    if (n_tok > 16 && n_tok <= fh3k_midm_max_tokens() && in >= 8192) return FH3_HIP_PATH_MIDM;
    return n_tok <= fh3k_skinny_max_tokens() ? FH3_HIP_PATH_SKINNY : FH3_HIP_PATH_GEMM;
}

}  // namespace

// ---------------------------------------------------------------------------
// Internal helpers shared with the C trunk streamer (fh3_hip_internal.h)
// ---------------------------------------------------------------------------
extern "C" int fh3i_set_error(int code, const char *msg) { return set_err(code, "%s", msg); }

extern "C" int fh3i_host_alloc(void **p, size_t bytes) {
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    FH3_HIPCALL(hipHostMalloc(p, bytes, hipHostMallocDefault));
    return FH3_OK;
}

extern "C" int fh3i_host_free(void *p) {
    if (!p) return FH3_OK;
    FH3_HIPCALL(hipHostFree(p));
    return FH3_OK;
}

extern "C" int fh3i_stream_create(void **st) {
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    hipStream_t s = nullptr;
    FH3_HIPCALL(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *st = (void *)s;
    return FH3_OK;
}

extern "C" int fh3i_stream_destroy(void *st) {
    if (!st) return FH3_OK;
    FH3_HIPCALL(hipStreamDestroy((hipStream_t)st));
    return FH3_OK;
}

extern "C" int fh3i_stream_sync(void *st) {
    FH3_HIPCALL(hipStreamSynchronize(st ? (hipStream_t)st : g.stream));
    return FH3_OK;
}

extern "C" int fh3i_copy_async(void *dst, const void *src, size_t bytes, void *st) {
    FH3_HIPCALL(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, st ? (hipStream_t)st : g.stream));
    return FH3_OK;
}

extern "C" int fh3i_event_create(void **ev) {
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    hipEvent_t e = nullptr;
    FH3_HIPCALL(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    *ev = (void *)e;
    return FH3_OK;
}

extern "C" int fh3i_event_destroy(void *ev) {
    if (!ev) return FH3_OK;
    FH3_HIPCALL(hipEventDestroy((hipEvent_t)ev));
    return FH3_OK;
}

extern "C" int fh3i_event_record(void *ev, void *st) {
    FH3_HIPCALL(hipEventRecord((hipEvent_t)ev, st ? (hipStream_t)st : g.stream));
    return FH3_OK;
}

extern "C" int fh3i_stream_wait(void *st, void *ev) {
    FH3_HIPCALL(hipStreamWaitEvent(st ? (hipStream_t)st : g.stream, (hipEvent_t)ev, 0));
    return FH3_OK;
}

extern "C" int fh3i_event_sync(void *ev) {
    FH3_HIPCALL(hipEventSynchronize((hipEvent_t)ev));
    return FH3_OK;
}

// ---------------------------------------------------------------------------
// fh3_hip.h
// ---------------------------------------------------------------------------
extern "C" int fh3_hip_init(int device) {
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    if (g.init && g.device == device) return FH3_OK;
    if (g.init) return set_err(FH3_E_INVALID, "fh3_hip_init: already initialised on device %d", g.device);
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0)
        return set_err(FH3_ERR, "fh3_hip_init: no HIP device available (%s)",
                       e != hipSuccess ? hipGetErrorString(e) : "0 devices");
    if (device < 0 || device >= n) return set_err(FH3_E_INVALID, "fh3_hip_init: device %d of %d", device, n);
    FH3_HIPCALL(hipSetDevice(device));
    hipDeviceProp_t prop;
    FH3_HIPCALL(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return set_err(FH3_ERR, "fh3_hip_init: device %d is %s; this library is built for gfx950", device,
                       prop.gcnArchName);
    if (device >= (int)(sizeof g_scratch / sizeof g_scratch[0]))
        return set_err(FH3_E_INVALID, "fh3_hip_init: device %d beyond the %d this library tracks", device,
                       (int)(sizeof g_scratch / sizeof g_scratch[0]));
    if (!g_scratch[device]) {
        // the device's own copy of the fixed scratch array (this device is current)
        void *p = nullptr;
        FH3_HIPCALL(fh3k_scratch_bind(&p));
        g_scratch[device] = p;
    }
    FH3_HIPCALL(hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking));
    g.device = device;
    g.init = true;
    return FH3_OK;
}

extern "C" void fh3_hip_shutdown(void) {
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    if (!g.init) return;
    (void)hipDeviceSynchronize();
    DevBuf *bufs[] = {&g.ws, &g.ws2, &g.w16, &g.part, &g.attn, &g.vsa_ws, &g.vsa_geo,
                      &g.st_w, &g.st_x, &g.st_y, &g.st_b};
    for (DevBuf *b : bufs) {
        if (b->p) (void)hipFree(b->p);
        b->p = nullptr;
        b->cap = 0;
    }
    for (auto &r : g.regs) (void)hipFree(r.dev);
    g.regs.clear();
    for (void *p : g.retired) (void)hipFree(p);
    g.retired.clear();
    g.foreign_capture = false;
    g.live_graphs = 0;
    for (int &k : g.vsa_key) k = -1;  // the VSA geometry was freed with vsa_geo
    g.vsa_T = g.vsa_P = 0;
    (void)hipStreamDestroy(g.stream);
    g.stream = nullptr;
    g.init = false;
    g.device = -1;
}

extern "C" const char *fh3_hip_last_error(void) { return g_err; }

extern "C" void *fh3_hip_stream(void) { return g.init ? (void *)g.stream : nullptr; }

extern "C" int fh3_hip_malloc(void **dptr, size_t bytes) {
    if (!dptr) return set_err(FH3_E_INVALID, "fh3_hip_malloc: NULL out pointer");
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    FH3_HIPCALL(hipMalloc(dptr, bytes ? bytes : 1));
    return FH3_OK;
}

extern "C" int fh3_hip_free(void *dptr) {
    if (!dptr) return FH3_OK;
    if (t_own_capture) {
        t_deferred_free.push_back(dptr);
        return FH3_OK;
    }
    FH3_HIPCALL(hipFree(dptr));
    return FH3_OK;
}

extern "C" int fh3_hip_memcpy_htod(void *dst, const void *src, size_t bytes) {
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    FH3_HIPCALL(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return FH3_OK;
}

extern "C" int fh3_hip_memcpy_dtoh(void *dst, const void *src, size_t bytes) {
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    FH3_HIPCALL(hipStreamSynchronize(g.stream));
    FH3_HIPCALL(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return FH3_OK;
}

extern "C" int fh3_hip_memcpy_dtod(void *dst, const void *src, size_t bytes) {
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    FH3_HIPCALL(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    return FH3_OK;
}

extern "C" int fh3_hip_memset(void *dptr, int value, size_t bytes) {
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    FH3_HIPCALL(hipMemset(dptr, value, bytes));
    return FH3_OK;
}

extern "C" int fh3_hip_synchronize(void) {
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    FH3_HIPCALL(hipDeviceSynchronize());
    return FH3_OK;
}

extern "C" int fh3_hip_graph_begin(void *stream) {
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    FH3_HIPCALL(hipStreamBeginCapture(stream ? (hipStream_t)stream : g.stream, hipStreamCaptureModeThreadLocal));
    t_own_capture = true;
    return FH3_OK;
}

extern "C" int fh3_hip_graph_end(void *stream, void **graph_exec) {
    if (!graph_exec) return set_err(FH3_E_INVALID, "fh3_hip_graph_end: NULL out pointer");
    hipGraph_t graph = nullptr;
    t_own_capture = false;
    const hipError_t ec = hipStreamEndCapture(stream ? (hipStream_t)stream : g.stream, &graph);
    for (void *p : t_deferred_free) (void)hipFree(p);
    t_deferred_free.clear();
    if (ec != hipSuccess) return hip_fail(ec, "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    *graph_exec = (void *)exec;
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    g.live_graphs++;
    return FH3_OK;
}

extern "C" int fh3_hip_graph_launch(void *graph_exec, void *stream) {
    if (!graph_exec) return set_err(FH3_E_INVALID, "fh3_hip_graph_launch: NULL graph");
    FH3_HIPCALL(hipGraphLaunch((hipGraphExec_t)graph_exec, stream ? (hipStream_t)stream : g.stream));
    return FH3_OK;
}

extern "C" int fh3_hip_graph_destroy(void *graph_exec) {
    if (!graph_exec) return FH3_OK;
    FH3_HIPCALL(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    if (g.live_graphs > 0 && --g.live_graphs == 0 && !g.foreign_capture && !g.retired.empty()) {
        // no graph holds the replaced workspace buffers any more
        hipError_t e = hipDeviceSynchronize();
        for (void *p : g.retired) {
            const hipError_t f = hipFree(p);
            if (e == hipSuccess) e = f;
        }
        g.retired.clear();
        if (e != hipSuccess) return hip_fail(e, "fh3_hip_graph_destroy: freeing replaced workspace");
    }
    return FH3_OK;
}

extern "C" int fh3_hip_set_path(int path) {
    if (path < FH3_HIP_PATH_AUTO || path > FH3_HIP_PATH_SWEEP)
        return set_err(FH3_E_INVALID, "fh3_hip_set_path: bad path %d", path);
    g.path = path;
    return FH3_OK;
}

extern "C" int fh3_hip_skinny_max(void) { return fh3k_skinny_max_tokens(); }

extern "C" int fh3_hip_matmul_path(int n_tok, int64_t in) { return choose_path(n_tok, in); }

extern "C" int fh3_hip_dequant_dev(int type, const void *d_src, float *d_dst, int64_t rows, int64_t n,
                                   void *stream) {
    if (!d_src || !d_dst || rows <= 0 || n <= 0)
        return set_err(FH3_E_INVALID, "fh3_hip_dequant_dev: NULL pointer or non-positive size");
    const int bl = fh3k_dequant_block_len(type);
    if (bl == 0) return set_err(FH3_E_INVALID, "fh3_hip_dequant_dev: unsupported type %d", type);
    if (n % bl)
        return set_err(FH3_E_INVALID, "fh3_hip_dequant_dev: n=%lld is not a multiple of the block length %d",
                       (long long)n, bl);
    if (((uintptr_t)d_src & 15u) || ((uintptr_t)d_dst & 15u))
        return set_err(FH3_E_INVALID, "fh3_hip_dequant_dev: pointers must be 16-byte aligned");
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    hipStream_t st = stream ? (hipStream_t)stream : g.stream;
    FH3_HIPCALL(fh3k_dequant_f32(type, d_src, (int64_t)fh3_row_bytes(type, n), n, rows, d_dst, st));
    return FH3_OK;
}

static int check_weights(const Fh3W *w, const char *fn) {
    if (!w || !w->data || w->in <= 0 || w->out <= 0)
        return set_err(FH3_E_INVALID, "%s: NULL weights or non-positive size", fn);
    const int bl = fh3k_dequant_block_len(w->type);
    if (bl == 0) return set_err(FH3_E_INVALID, "%s: unsupported weight type %d", fn, w->type);
    // a row must be whole blocks of its type: the reference decodes whole
    // blocks only and leaves the rest of such a row undefined
    if (w->in % bl)
        return set_err(FH3_E_INVALID, "%s: in=%lld is not a multiple of the type's block length %d", fn,
                       (long long)w->in, bl);
    if (w->in > kMaxInGeneral || w->out > 0x7FFFFFFF)
        return set_err(FH3_E_INVALID, "%s: in=%lld out=%lld out of range (in <= %lld)", fn, (long long)w->in,
                       (long long)w->out, (long long)kMaxInGeneral);
    if ((uintptr_t)w->data & 15u) return set_err(FH3_E_INVALID, "%s: weights must be 16-byte aligned", fn);
    return FH3_OK;
}

// Prepared-activation layout: fragments of Mpad = round_up(n_tok, 256) rows,
// then Mpad fp32 inverse scales at a 256-byte aligned offset, then (up to 64
// tokens) the fp32 sums of each 32-value group, [n_tok][in / 32], at the next
// 256-byte boundary: the FH3_HIP_PATH_SWEEP kernel's offsets.
static int64_t prep_rows(int n_tok) { return round_up(n_tok, fh3k_gemm_row_pad()); }
static size_t prep_scale_offset(int n_tok, int64_t in) {
    return (size_t)round_up(prep_rows(n_tok) * kpad(in) * 2, 256);
}
static size_t prep_sum_offset(int n_tok, int64_t in) {
    return (size_t)round_up((int64_t)(prep_scale_offset(n_tok, in) + (size_t)prep_rows(n_tok) * sizeof(float)), 256);
}

extern "C" size_t fh3_hip_prepared_bytes(int n_tok, int64_t in) {
    if (n_tok <= 0 || in <= 0) return 0;
    const size_t sums = n_tok <= fh3k_sweep_max_tokens() && !general_rows(in)
                            ? (size_t)n_tok * (size_t)(in / 32) * sizeof(float)
                            : 0;
    return prep_sum_offset(n_tok, in) + sums;
}

// the prepared form's parts
static const float *prep_scales(const void *prep, int n_tok, int64_t in) {
    return (const float *)((const char *)prep + prep_scale_offset(n_tok, in));
}
static const float *prep_sums(const void *prep, int n_tok, int64_t in) {
    return (const float *)((const char *)prep + prep_sum_offset(n_tok, in));
}

// Where the preparation writes the group sums: for every fragment form of up
// to fh3k_sweep_max_tokens() tokens, whichever kernel the current path
// setting picks, so that a prepared buffer stays valid for k_sweep when the
// setting changes between preparation and product.
static float *prep_sums_out(void *prep, int n_tok, int64_t in) {
    return n_tok <= fh3k_sweep_max_tokens() && !general_rows(in) ? (float *)prep_sums(prep, n_tok, in) : nullptr;
}

static int prepare(const float *d_x, int n_tok, int64_t in, void *d_prep, int64_t rows, hipStream_t st) {
    if (general_rows(in)) {
        FH3_HIPCALL(fh3k_xprep_any(d_x, n_tok, (int)in, (int)rows, d_prep, (float *)prep_scales(d_prep, n_tok, in), st));
        return FH3_OK;
    }
    const int path = choose_path(n_tok, in);
    if (path == FH3_HIP_PATH_GEMV8) {
        // that kernel quantises fp32 activations itself: the prepared form is x
        FH3_HIPCALL(hipMemcpyAsync(d_prep, d_x, (size_t)n_tok * (size_t)in * sizeof(float),
                                   hipMemcpyDeviceToDevice, st));
        return FH3_OK;
    }
    float *xs_inv = (float *)prep_scales(d_prep, n_tok, in);
    FH3_HIPCALL(fh3k_xprep(d_x, n_tok, (int)in, (int)rows, d_prep, xs_inv, prep_sums_out(d_prep, n_tok, in), st));
    return FH3_OK;
}

// prepared rows the kernels of `path` read (the preparation zeroes the rows
// from n_tok up to this count; rows past it are never read)
static int64_t kernel_rows(int path, int n_tok) {
    return path == FH3_HIP_PATH_SKINNY || path == FH3_HIP_PATH_MIDM || path == FH3_HIP_PATH_SWEEP
               ? round_up(n_tok, 32)
               : fh3k_gemm_rows(n_tok);
}

extern "C" int fh3_hip_prepare_x_dev(const float *d_x, int n_tok, int64_t in, void *d_prep, void *stream) {
    if (!d_x || !d_prep || n_tok <= 0 || in <= 0 || in > kMaxInGeneral)
        return set_err(FH3_E_INVALID, "fh3_hip_prepare_x_dev: bad arguments");
    if (((uintptr_t)d_x & 15u) || ((uintptr_t)d_prep & 15u))
        return set_err(FH3_E_INVALID, "fh3_hip_prepare_x_dev: pointers must be 16-byte aligned");
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    return prepare(d_x, n_tok, in, d_prep, prep_rows(n_tok), stream ? (hipStream_t)stream : g.stream);
}

// Weights of another type than Q4_K, and general rows of any type: Q5_K and
// Q6_K rows of whole super-blocks are read in place, by k_skinny (Q6_K: the
// sweep where it applies, q_sweep) up to 64 tokens and by k_gemm above;
// otherwise fp16 rows of kpad(in) columns (the weight itself for F16 rows of
// whole super-blocks, else decoded, zero-padded, into the library's w16
// buffer), then k_skinny16 / k_gemm16.
static bool reads_in_place_q(const Fh3W *w, int n_tok) {
    if (general_rows(w->in)) return false;
    return path16(n_tok, w->in) == FH3_HIP_PATH_SKINNY ? fh3k_skinny_q_takes(w->type) != 0
                                                        : fh3k_gemm_q_takes(w->type) != 0;
}

static size_t w16_bytes(const Fh3W *w, int n_tok) {
    if (reads_in_place_q(w, n_tok) || (w->type == FH3_QUANT_F16 && !general_rows(w->in))) return 0;
    return (size_t)w->out * (size_t)kpad(w->in) * 2;
}

// Up to 64 tokens Q6_K takes the sweep where Q4_K would (up to 16 tokens, or
// 17-64 on rows of at least 5120 values), or when that path is forced; other
// small-M in-place products run k_skinny.
static bool q_sweep(const Fh3W *w, int n_tok) {
    if (!fh3k_sweep_q_takes(w->type) || !fh3k_sweep_fits((int)w->in, n_tok)) return false;
    if (g.path == FH3_HIP_PATH_SWEEP) return true;
    return g.path == FH3_HIP_PATH_AUTO && (n_tok <= 16 || w->in >= 5120);
}

// Partial sums of the in-place Q5_K / Q6_K products (0 when they do not split
// K).
static size_t part16_bytes(const Fh3W *w, int n_tok) {
    if (!reads_in_place_q(w, n_tok)) return 0;
    const int K = (int)w->in, N = (int)w->out;
    if (path16(n_tok, w->in) == FH3_HIP_PATH_SKINNY)
        return q_sweep(w, n_tok) ? fh3k_sweep_q_part_bytes(w->type, N, K, n_tok)
                                 : fh3k_skinny_q_part_bytes(N, K, n_tok);
    return fh3k_gemm_part_bytes(N, K, n_tok, FH3_EPI_NONE);
}

// Called with g.mu held (it may grow the library's buffers).
static int product16(const Fh3W *w, const void *x16, const float *xs_inv, int n_tok, const float *bias, float *d_y,
                     hipStream_t st) {
    const int K = (int)w->in, Kp = (int)kpad(w->in), N = (int)w->out;
    if (reads_in_place_q(w, n_tok)) {
        const int64_t rb = (int64_t)fh3_row_bytes(w->type, w->in);
        float *part = nullptr;
        if (const size_t pb = part16_bytes(w, n_tok)) {
            int rc = grow(g.part, pb, st);
            if (rc != FH3_OK) return rc;
            part = (float *)g.part.p;
        }
        if (path16(n_tok, w->in) == FH3_HIP_PATH_SKINNY && q_sweep(w, n_tok))
            FH3_HIPCALL(fh3k_sweep_q(w->type, w->data, rb, N, K, x16, xs_inv, bias, d_y, n_tok, part, st));
        else if (path16(n_tok, w->in) == FH3_HIP_PATH_SKINNY)
            FH3_HIPCALL(fh3k_skinny_q(w->type, w->data, rb, N, K, x16, xs_inv, bias, d_y, n_tok, part, st));
        else
            FH3_HIPCALL(fh3k_gemm_q(w->type, w->data, rb, N, K, x16, xs_inv, bias, d_y, n_tok, part, st));
        return FH3_OK;
    }
    const void *w16 = w->data;
    if (const size_t wb = w16_bytes(w, n_tok)) {
        int rc = grow(g.w16, wb, st);
        if (rc != FH3_OK) return rc;
        FH3_HIPCALL(fh3k_weights_f16(w->type, w->data, (int64_t)fh3_row_bytes(w->type, w->in), K, Kp, N, g.w16.p,
                                     st));
        w16 = g.w16.p;
    }
    if (path16(n_tok, w->in) == FH3_HIP_PATH_SKINNY)
        FH3_HIPCALL(fh3k_skinny16(w16, N, Kp, x16, xs_inv, bias, d_y, n_tok, st));
    else
        FH3_HIPCALL(fh3k_gemm16(w16, N, Kp, x16, xs_inv, bias, d_y, n_tok, st));
    return FH3_OK;
}

// Partial-sum bytes of the split-K kernels for a Q4_K product (0 when the
// chosen kernel does not split K).
static size_t part_bytes(const Fh3W *w, int n_tok, int epi) {
    const int K = (int)w->in, N = (int)w->out;
    const int path = choose_path(n_tok, w->in);
    if (path == FH3_HIP_PATH_MIDM) return fh3k_midm_part_bytes(N, K, n_tok);
    if (path == FH3_HIP_PATH_GEMM) return fh3k_gemm_part_bytes(N, K, n_tok, epi);
    if (path == FH3_HIP_PATH_SWEEP) return fh3k_sweep_part_bytes(N, K, n_tok);
    return 0;
}

// part_ext: partial sums in caller-provided device memory (at least
// part_bytes()), else in the library's grow-only buffer.
static int product(const Fh3W *w, const void *prep, int n_tok, const float *bias, float *d_y, hipStream_t st,
                   int epi = FH3_EPI_NONE, const float *aux = nullptr, float *part_ext = nullptr) {
    if (w->type != FH3_QUANT_Q4_K || general_rows(w->in)) {
        std::lock_guard<std::recursive_mutex> lk(g.mu);
        if (choose_path(n_tok, w->in) == FH3_HIP_PATH_GEMV8) {
            // the prepared form is then a copy of x: make the fragments here,
            // the rows the chosen kernel reads (as fh3_hip_matmul_dev does)
            int rc = grow(g.ws2, fh3_hip_prepared_bytes(n_tok, w->in), st);
            if (rc != FH3_OK) return rc;
            float *xs = (float *)prep_scales(g.ws2.p, n_tok, w->in);
            const int64_t rows = path16(n_tok, w->in) == FH3_HIP_PATH_SKINNY ? round_up(n_tok, 32) : prep_rows(n_tok);
            FH3_HIPCALL(fh3k_xprep((const float *)prep, n_tok, (int)w->in, (int)rows, g.ws2.p, xs, nullptr, st));
            return product16(w, g.ws2.p, xs, n_tok, bias, d_y, st);
        }
        return product16(w, prep, prep_scales(prep, n_tok, w->in), n_tok, bias, d_y, st);
    }
    const int K = (int)w->in, N = (int)w->out;
    const int64_t row_bytes = (int64_t)fh3_row_bytes(w->type, w->in);
    const float *xs_inv = prep_scales(prep, n_tok, w->in);
    const int path = choose_path(n_tok, w->in);
    if (path == FH3_HIP_PATH_GEMV8) {
        FH3_HIPCALL(fh3k_gemv8_epi(w->data, row_bytes, N, K, (const float *)prep, bias, d_y, n_tok, epi, aux, st));
    } else if (path == FH3_HIP_PATH_SKINNY) {
        FH3_HIPCALL(fh3k_skinny_epi(w->data, row_bytes, N, K, prep, xs_inv, bias, d_y, n_tok, epi, aux, st));
    } else {
        // the split-K kernels (the sweep on rows of more than 32 super-blocks,
        // middle M, and the GEMM with few tiles) need the partial-sum workspace
        const size_t pb = part_bytes(w, n_tok, epi);
        std::unique_lock<std::recursive_mutex> lk(g.mu, std::defer_lock);
        float *part = part_ext;
        if (pb && !part) {
            lk.lock();
            int rc = grow(g.part, pb, st);
            if (rc != FH3_OK) return rc;
            part = (float *)g.part.p;
        }
        if (path == FH3_HIP_PATH_SWEEP)
            FH3_HIPCALL(fh3k_sweep_epi(w->data, row_bytes, N, K, prep, xs_inv, prep_sums(prep, n_tok, w->in), bias,
                                       d_y, n_tok, epi, aux, part, st));
        else if (path == FH3_HIP_PATH_MIDM)
            FH3_HIPCALL(fh3k_midm_epi(w->data, row_bytes, N, K, prep, xs_inv, bias, d_y, n_tok, epi, aux, part, st));
        else
            FH3_HIPCALL(fh3k_gemm_epi(w->data, row_bytes, N, K, prep, xs_inv, bias, d_y, n_tok, epi, aux, part, st));
    }
    return FH3_OK;
}

// k_gemm addresses its weight matrix with 32-bit byte offsets (buffer
// resources): the Q4_K / Q5_K / Q6_K products it runs, above 64 tokens, need
// out * row_bytes < 2^32.  Refused before any work is enqueued.
static int check_gemm_span(const Fh3W *w, int n_tok, const char *fn) {
    if (general_rows(w->in)) return FH3_OK;
    const bool gemm = w->type == FH3_QUANT_Q4_K
                          ? choose_path(n_tok, w->in) == FH3_HIP_PATH_GEMM
                          : reads_in_place_q(w, n_tok) && path16(n_tok, w->in) != FH3_HIP_PATH_SKINNY;
    const uint64_t span = (uint64_t)w->out * (uint64_t)fh3_row_bytes(w->type, w->in);
    if (gemm && span >= (1ull << 32))
        return set_err(FH3_E_INVALID, "%s: n_tok=%d with out * row_bytes = %llu bytes of weights; products of more "
                                      "than 64 tokens take less than 2^32 bytes (32-bit row offsets)",
                       fn, n_tok, (unsigned long long)span);
    return FH3_OK;
}

extern "C" int fh3_hip_matmul_prepared_dev(const Fh3W *w, const void *d_prep, float *d_y, int n_tok,
                                           const float *d_bias_or_null, void *stream) {
    int rc = check_weights(w, "fh3_hip_matmul_prepared_dev");
    if (rc != FH3_OK) return rc;
    if (n_tok > 0 && (rc = check_gemm_span(w, n_tok, "fh3_hip_matmul_prepared_dev")) != FH3_OK) return rc;
    if (!d_prep || !d_y || n_tok <= 0)
        return set_err(FH3_E_INVALID, "fh3_hip_matmul_prepared_dev: NULL pointer or n_tok <= 0");
    if ((uintptr_t)d_prep & 15u)
        return set_err(FH3_E_INVALID, "fh3_hip_matmul_prepared_dev: prepared buffer must be 16-byte aligned");
    rc = ensure_init();
    if (rc != FH3_OK) return rc;
    return product(w, d_prep, n_tok, d_bias_or_null, d_y, stream ? (hipStream_t)stream : g.stream);
}

// Epilogue arguments: Q4_K weights only; SwiGLU needs out % 128 == 0 (val and
// gate halves of whole 64-row tiles); the gate-residual epilogue needs aux.
static int check_epi(const Fh3W *w, int epi, const float *aux, const char *fn) {
    if (epi == FH3_EPI_NONE) return FH3_OK;
    if (epi != FH3_EPI_GATE_RESIDUAL && epi != FH3_EPI_SWIGLU) return set_err(FH3_E_INVALID, "%s: bad epilogue %d", fn, epi);
    if (w->type != FH3_QUANT_Q4_K || general_rows(w->in))
        return set_err(FH3_E_INVALID, "%s: fused epilogues take Q4_K weights with in %% 256 == 0 and in <= %d", fn,
                       fh3k_max_in());
    if (epi == FH3_EPI_SWIGLU && w->out % 128)
        return set_err(FH3_E_INVALID, "%s: SwiGLU needs out %% 128 == 0 (out=%lld)", fn, (long long)w->out);
    if (epi == FH3_EPI_GATE_RESIDUAL && !aux) return set_err(FH3_E_INVALID, "%s: gate-residual needs the gate", fn);
    return FH3_OK;
}

static int matmul_dev(const Fh3W *w, const float *d_x, float *d_y, int n_tok, const float *d_bias_or_null,
                      void *stream, int epi, const float *aux, const char *fn) {
    int rc = check_weights(w, fn);
    if (rc != FH3_OK) return rc;
    if ((rc = check_epi(w, epi, aux, fn)) != FH3_OK) return rc;
    if (!d_x || !d_y || n_tok <= 0)
        return set_err(FH3_E_INVALID, "%s: NULL pointer or n_tok <= 0", fn);
    if ((rc = check_gemm_span(w, n_tok, fn)) != FH3_OK) return rc;
    if ((uintptr_t)d_x & 15u) return set_err(FH3_E_INVALID, "%s: x must be 16-byte aligned", fn);
    rc = ensure_init();
    if (rc != FH3_OK) return rc;
    hipStream_t st = stream ? (hipStream_t)stream : g.stream;
    if (w->type != FH3_QUANT_Q4_K || general_rows(w->in)) {
        std::lock_guard<std::recursive_mutex> lk(g.mu);
        const int64_t rows = path16(n_tok, w->in) == FH3_HIP_PATH_SKINNY ? round_up(n_tok, 32) : prep_rows(n_tok);
        rc = grow(g.ws, fh3_hip_prepared_bytes(n_tok, w->in), st);
        if (rc != FH3_OK) return rc;
        float *xs = (float *)prep_scales(g.ws.p, n_tok, w->in);
        if (general_rows(w->in))
            FH3_HIPCALL(fh3k_xprep_any(d_x, n_tok, (int)w->in, (int)rows, g.ws.p, xs, st));
        else
            FH3_HIPCALL(fh3k_xprep(d_x, n_tok, (int)w->in, (int)rows, g.ws.p, xs, nullptr, st));
        return product16(w, g.ws.p, xs, n_tok, d_bias_or_null, d_y, st);
    }
    const int path = choose_path(n_tok, w->in);
    if (path == FH3_HIP_PATH_GEMV8) {  // no preparation and no workspace
        FH3_HIPCALL(fh3k_gemv8_epi(w->data, (int64_t)fh3_row_bytes(w->type, w->in), (int)w->out, (int)w->in, d_x,
                                   d_bias_or_null, d_y, n_tok, epi, aux, st));
        return FH3_OK;
    }
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    // the small- and middle-M kernels only read round_up(n_tok, 32) prepared rows
    const int64_t rows = kernel_rows(path, n_tok);
    rc = grow(g.ws, fh3_hip_prepared_bytes(n_tok, w->in), st);
    if (rc != FH3_OK) return rc;
    rc = prepare(d_x, n_tok, w->in, g.ws.p, rows, st);
    if (rc != FH3_OK) return rc;
    return product(w, g.ws.p, n_tok, d_bias_or_null, d_y, st, epi, aux);
}

extern "C" int fh3_hip_matmul_dev(const Fh3W *w, const float *d_x, float *d_y, int n_tok,
                                  const float *d_bias_or_null, void *stream) {
    return matmul_dev(w, d_x, d_y, n_tok, d_bias_or_null, stream, FH3_EPI_NONE, nullptr, "fh3_hip_matmul_dev");
}

extern "C" int fh3_hip_matmul_epi_dev(const Fh3W *w, const float *d_x, int n_tok, const float *d_bias_or_null,
                                      int epi, const float *d_aux, float *d_out, void *stream) {
    return matmul_dev(w, d_x, d_out, n_tok, d_bias_or_null, stream, epi, d_aux, "fh3_hip_matmul_epi_dev");
}

extern "C" int fh3_hip_matmul_prepared_epi_dev(const Fh3W *w, const void *d_prep, int n_tok,
                                               const float *d_bias_or_null, int epi, const float *d_aux,
                                               float *d_out, void *stream) {
    const char *fn = "fh3_hip_matmul_prepared_epi_dev";
    int rc = check_weights(w, fn);
    if (rc != FH3_OK) return rc;
    if ((rc = check_epi(w, epi, d_aux, fn)) != FH3_OK) return rc;
    if (!d_prep || !d_out || n_tok <= 0) return set_err(FH3_E_INVALID, "%s: NULL pointer or n_tok <= 0", fn);
    if ((rc = check_gemm_span(w, n_tok, fn)) != FH3_OK) return rc;
    if ((uintptr_t)d_prep & 15u) return set_err(FH3_E_INVALID, "%s: prepared buffer must be 16-byte aligned", fn);
    rc = ensure_init();
    if (rc != FH3_OK) return rc;
    return product(w, d_prep, n_tok, d_bias_or_null, d_out, stream ? (hipStream_t)stream : g.stream, epi, d_aux);
}

extern "C" size_t fh3_hip_matmul_workspace_bytes(const Fh3W *w, int n_tok, int epi, int prepared) {
    const int bl = w ? fh3k_dequant_block_len(w->type) : 0;
    if (!w || w->in <= 0 || w->out <= 0 || n_tok <= 0 || bl == 0 || w->in % bl || w->in > kMaxInGeneral)
        return 0;
    const size_t prep = fh3_hip_prepared_bytes(n_tok, w->in);
    if (w->type != FH3_QUANT_Q4_K || general_rows(w->in)) {
        const bool own_prep = !prepared || choose_path(n_tok, w->in) == FH3_HIP_PATH_GEMV8;
        return w16_bytes(w, n_tok) + part16_bytes(w, n_tok) + (own_prep ? prep : 0);
    }
    const bool gemv8 = choose_path(n_tok, w->in) == FH3_HIP_PATH_GEMV8;
    return (prepared || gemv8 ? 0 : prep) + part_bytes(w, n_tok, epi);
}

// The no-allocation product: fh3_hip_matmul_dev's kernels with their
// workspace (prepared activations, then partial sums at a 256-byte aligned
// offset) in the fixed scratch array bound by fh3_hip_init.
extern "C" int fh3_hip_matmul_noalloc_dev(const Fh3W *w, const float *d_x, float *d_y, int n_tok,
                                          const float *d_bias_or_null, void *stream) {
    const char *fn = "fh3_hip_matmul_noalloc_dev";
    int rc = check_weights(w, fn);
    if (rc != FH3_OK) return rc;
    if (w->type != FH3_QUANT_Q4_K) return set_err(FH3_E_INVALID, "%s: Q4_K weights only (type %d)", fn, w->type);
    if (general_rows(w->in))
        return set_err(FH3_E_INVALID, "%s: in=%lld; rows of more than %d values take fh3_hip_matmul_dev", fn,
                       (long long)w->in, fh3k_max_in());
    if (!d_x || !d_y || n_tok <= 0) return set_err(FH3_E_INVALID, "%s: NULL pointer or n_tok <= 0", fn);
    if ((uintptr_t)d_x & 15u) return set_err(FH3_E_INVALID, "%s: x must be 16-byte aligned", fn);
    if ((rc = check_gemm_span(w, n_tok, fn)) != FH3_OK) return rc;
    if (!g.init || !g_scratch[g.device])
        return set_err(FH3_E_INVALID, "%s: call fh3_hip_init first (it binds the scratch memory)", fn);
    hipStream_t st = stream ? (hipStream_t)stream : g.stream;
    const int path = choose_path(n_tok, w->in);
    if (path == FH3_HIP_PATH_GEMV8) {  // this kernel needs no workspace
        FH3_HIPCALL(fh3k_gemv8_epi(w->data, (int64_t)fh3_row_bytes(w->type, w->in), (int)w->out, (int)w->in, d_x,
                                   d_bias_or_null, d_y, n_tok, FH3_EPI_NONE, nullptr, st));
        return FH3_OK;
    }
    const size_t part_off = (size_t)round_up((int64_t)fh3_hip_prepared_bytes(n_tok, w->in), 256);
    const size_t need = part_off + part_bytes(w, n_tok, FH3_EPI_NONE);
    if (need > (size_t)FH3_HIP_NOALLOC_SCRATCH_BYTES)
        return set_err(FH3_E_INVALID, "%s: n_tok=%d in=%lld out=%lld needs %zu bytes of scratch; the fixed scratch "
                                      "holds %zu (use fh3_hip_matmul_dev)", fn, n_tok, (long long)w->in,
                       (long long)w->out, need, (size_t)FH3_HIP_NOALLOC_SCRATCH_BYTES);
    uint8_t *scr = (uint8_t *)g_scratch[g.device];
    const int64_t rows = kernel_rows(path, n_tok);
    rc = prepare(d_x, n_tok, w->in, scr, rows, st);
    if (rc != FH3_OK) return rc;
    return product(w, scr, n_tok, d_bias_or_null, d_y, st, FH3_EPI_NONE, nullptr, (float *)(scr + part_off));
}

extern "C" int fh3_hip_prepare_x_norm_dev(const float *d_x, int n_tok, int64_t in, const float *d_norm_w, float eps,
                                          const float *d_shift, const float *d_scale, void *d_prep, void *stream) {
    const char *fn = "fh3_hip_prepare_x_norm_dev";
    if (!d_x || !d_prep || !d_norm_w || n_tok <= 0 || in <= 0 || in % 256 || in > fh3k_max_in() ||
        (d_shift == nullptr) != (d_scale == nullptr))
        return set_err(FH3_E_INVALID, "%s: bad arguments", fn);
    if (((uintptr_t)d_x & 15u) || ((uintptr_t)d_prep & 15u) || ((uintptr_t)d_norm_w & 15u) ||
        ((uintptr_t)d_shift & 15u) || ((uintptr_t)d_scale & 15u))
        return set_err(FH3_E_INVALID, "%s: pointers must be 16-byte aligned", fn);
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    hipStream_t st = stream ? (hipStream_t)stream : g.stream;
    if (choose_path(n_tok, in) == FH3_HIP_PATH_GEMV8) {  // prepared form: the normalised fp32 rows
        FH3_HIPCALL(fh3k_rownorm_f32(d_x, n_tok, (int)in, (float *)d_prep, d_norm_w, eps, d_shift, d_scale, st));
        return FH3_OK;
    }
    float *xs_inv = (float *)prep_scales(d_prep, n_tok, in);
    float *xsum = prep_sums_out(d_prep, n_tok, in);
    FH3_HIPCALL(fh3k_xprep_norm(d_x, n_tok, (int)in, (int)prep_rows(n_tok), d_prep, xs_inv, d_norm_w, eps, d_shift,
                                d_scale, xsum, st));
    return FH3_OK;
}

extern "C" int fh3_hip_rownorm_dev(const float *d_x, int n_tok, int64_t in, const float *d_norm_w, float eps,
                                   const float *d_shift, const float *d_scale, float *d_y, void *stream) {
    const char *fn = "fh3_hip_rownorm_dev";
    if (!d_x || !d_y || !d_norm_w || n_tok <= 0 || in <= 0 || in % 4 || in > fh3k_max_in() ||
        (d_shift == nullptr) != (d_scale == nullptr))
        return set_err(FH3_E_INVALID, "%s: bad arguments", fn);
    if (((uintptr_t)d_x & 15u) || ((uintptr_t)d_y & 15u) || ((uintptr_t)d_norm_w & 15u) ||
        ((uintptr_t)d_shift & 15u) || ((uintptr_t)d_scale & 15u))
        return set_err(FH3_E_INVALID, "%s: pointers must be 16-byte aligned", fn);
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    FH3_HIPCALL(fh3k_rownorm_f32(d_x, n_tok, (int)in, d_y, d_norm_w, eps, d_shift, d_scale,
                                 stream ? (hipStream_t)stream : g.stream));
    return FH3_OK;
}

// ---------------------------------------------------------------------------
// Attention (fh3_attn.hip)
// ---------------------------------------------------------------------------
static int attention_dev(const float *q, const float *k, const float *v, int64_t ld, int n, int heads, int hd,
                         const float *qn_w, const float *kn_w, float eps, const float *cs, const float *sn, int rot,
                         float *d_o, void *stream, const char *fn) {
    if (!q || !k || !v || !d_o || n <= 0 || heads <= 0 || hd <= 0)
        return set_err(FH3_E_INVALID, "%s: NULL pointer or non-positive size", fn);
    if (!fh3k_attn_head_dim_ok(hd))
        return set_err(FH3_E_INVALID, "%s: head_dim %d is not supported (64 or 128)", fn, hd);
    if ((cs == nullptr) != (sn == nullptr) || (cs && (rot <= 0 || rot > hd || rot % 2)))
        return set_err(FH3_E_INVALID, "%s: rope needs cos and sin with an even rot_dim <= head_dim", fn);
    if ((uintptr_t)q & 15u || (uintptr_t)k & 15u || (uintptr_t)v & 15u || (uintptr_t)d_o & 15u ||
        (uintptr_t)cs & 15u || (uintptr_t)sn & 15u)
        return set_err(FH3_E_INVALID, "%s: q, k, v, o, cos and sin must be 16-byte aligned", fn);
    if ((int64_t)heads * hd > ((int64_t)1 << 30) || (int64_t)n > ((int64_t)1 << 30) / heads)
        return set_err(FH3_E_INVALID, "%s: n * heads too large", fn);
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    hipStream_t st = stream ? (hipStream_t)stream : g.stream;
    if ((rc = grow(g.attn, fh3k_attn_ws_bytes(n, heads, hd), st)) != FH3_OK) return rc;
    FH3_HIPCALL(fh3k_attention(q, k, v, ld, n, heads, hd, qn_w, kn_w, eps, cs, sn, cs ? rot : 0, g.attn.p, d_o,
                               (int64_t)heads * hd, st));
    return FH3_OK;
}

extern "C" int fh3_hip_attention_dev(const float *d_q, const float *d_k, const float *d_v, float *d_o, int n,
                                     int heads, int hd, void *stream) {
    return attention_dev(d_q, d_k, d_v, (int64_t)heads * hd, n, heads, hd, nullptr, nullptr, 0.f, nullptr, nullptr,
                         0, d_o, stream, "fh3_hip_attention_dev");
}

extern "C" int fh3_hip_attention_qkv_dev(const float *d_qkv, int n, int heads, int hd, const float *d_qnorm_w,
                                         const float *d_knorm_w, float eps, const float *d_cos, const float *d_sin,
                                         int rot_dim, float *d_o, void *stream) {
    const char *fn = "fh3_hip_attention_qkv_dev";
    if (!d_qkv) return set_err(FH3_E_INVALID, "%s: NULL qkv", fn);
    if ((d_qnorm_w == nullptr) != (d_knorm_w == nullptr))
        return set_err(FH3_E_INVALID, "%s: give both q and k norm weights or neither", fn);
    const int64_t inner = (int64_t)heads * hd;
    return attention_dev(d_qkv, d_qkv + inner, d_qkv + 2 * inner, 3 * inner, n, heads, hd, d_qnorm_w, d_knorm_w, eps,
                         d_cos, d_sin, rot_dim, d_o, stream, fn);
}

// ---------------------------------------------------------------------------
// Weight registration: a host range uploaded once, kept on the device and
// found by the host-pointer wrappers, which then copy only x in and y out
// ---------------------------------------------------------------------------
// Device address of [p, p + bytes) when it lies inside a registered range.
static const void *registered(const void *p, size_t bytes) {
    const uint8_t *q = (const uint8_t *)p;
    for (const auto &r : g.regs)
        if (q >= r.host && q + bytes <= r.host + r.bytes) return (const uint8_t *)r.dev + (q - r.host);
    return nullptr;
}

extern "C" int fh3_hip_register_weights(const void *host, size_t bytes, const void **d_out) {
    const char *fn = "fh3_hip_register_weights";
    if (!host || bytes == 0) return set_err(FH3_E_INVALID, "%s: NULL pointer or zero size", fn);
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    const uint8_t *h = (const uint8_t *)host;
    for (auto &r : g.regs) {
        if (r.host == h && r.bytes == bytes) {  // re-registration refreshes the device copy
            FH3_HIPCALL(hipDeviceSynchronize());
            FH3_HIPCALL(hipMemcpy(r.dev, host, bytes, hipMemcpyHostToDevice));
            if (d_out) *d_out = r.dev;
            return FH3_OK;
        }
        if (h < r.host + r.bytes && r.host < h + bytes)
            return set_err(FH3_E_INVALID, "%s: range overlaps a registered range", fn);
    }
    void *dev = nullptr;
    FH3_HIPCALL(hipMalloc(&dev, bytes));
    const hipError_t e = hipMemcpy(dev, host, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return hip_fail(e, "fh3_hip_register_weights upload");
    }
    g.regs.push_back({h, bytes, dev});
    if (d_out) *d_out = dev;
    return FH3_OK;
}

extern "C" int fh3_hip_unregister_weights(const void *host) {
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    for (size_t i = 0; i < g.regs.size(); i++)
        if (g.regs[i].host == (const uint8_t *)host) {
            FH3_HIPCALL(hipDeviceSynchronize());  // enqueued work may still read it
            FH3_HIPCALL(hipFree(g.regs[i].dev));
            g.regs.erase(g.regs.begin() + (long)i);
            return FH3_OK;
        }
    return set_err(FH3_E_INVALID, "fh3_hip_unregister_weights: %p is not registered", host);
}

extern "C" const void *fh3_hip_registered_ptr(const void *host, size_t bytes) {
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    return host ? registered(host, bytes) : nullptr;
}

// ---------------------------------------------------------------------------
// Video sparse attention
// ---------------------------------------------------------------------------
// Tile geometry of src/core/fh3_vsa.c:31-163: text tokens, then audio tokens,
// in runs of `tile`; then the video grid in 4x4x4 cubes (t-major, tokens of a
// cube in (t, h, w) order).  Counts that do not sum to n make every token
// video; a grid that does not match the video count becomes 1 x 1 x V.
static int vsa_geometry(const Fh3Seq *sq, int tile, std::vector<int> &tok, std::vector<int> &off, int *n_prefix) {
    const int n = sq->seq_len;
    int T = sq->num_text > 0 ? sq->num_text : 0, A = sq->num_audio > 0 ? sq->num_audio : 0;
    int V = sq->num_video > 0 ? sq->num_video : 0;
    if (T + A + V != n) T = 0, A = 0, V = n;
    int gt = sq->grid_t, gh = sq->grid_h, gw = sq->grid_w;
    if (gt <= 0 || gh <= 0 || gw <= 0 || (int64_t)gt * gh * gw != V) gt = 1, gh = 1, gw = V;
    tok.clear();
    off.assign(1, 0);
    const int runs[2][2] = {{0, T}, {T, A}};
    for (const auto &rn : runs)
        for (int s0 = 0; s0 < rn[1]; s0 += tile) {
            for (int e = s0; e < rn[1] && e < s0 + tile; e++) tok.push_back(rn[0] + e);
            off.push_back((int)tok.size());
        }
    *n_prefix = (int)off.size() - 1;
    if (V > 0)
        for (int t0 = 0; t0 < gt; t0 += 4)
            for (int h0 = 0; h0 < gh; h0 += 4)
                for (int w0 = 0; w0 < gw; w0 += 4) {
                    for (int t = t0; t < gt && t < t0 + 4; t++)
                        for (int h = h0; h < gh && h < h0 + 4; h++)
                            for (int w = w0; w < gw && w < w0 + 4; w++) tok.push_back(T + A + (t * gh + h) * gw + w);
                    off.push_back((int)tok.size());
                }
    return (int)off.size() - 1;
}

// Device copy of the geometry: inv[T] (1/count), cnt[T], gather[slots] (token
// of each 64-slot tile position, -1 empty), kept while the sequence shape
// does not change.
static int vsa_plan(const Fh3Seq *sq, int tile, hipStream_t st, const char *fn) {
    const int key[8] = {sq->seq_len, sq->num_text, sq->num_audio, sq->num_video, sq->grid_t, sq->grid_h, sq->grid_w,
                        tile};
    if (memcmp(key, g.vsa_key, sizeof key) == 0) return FH3_OK;
    if (capturing(st))
        return set_err(FH3_E_INVALID, "%s: a new sequence shape during graph capture; run the call once eagerly "
                                      "before capturing it", fn);
    std::vector<int> tok, off;
    int P = 0;
    const int T = vsa_geometry(sq, tile, tok, off, &P);
    if (T <= 0 || T > fh3k_vsa_max_tiles())
        return set_err(FH3_E_INVALID, "%s: %d tiles (at most %d on the device)", fn, T, fh3k_vsa_max_tiles());
    const int64_t slots = fh3k_attn_pad(64 * T);
    std::vector<int> host(2 * (size_t)T + (size_t)slots);
    int *h_inv = host.data(), *h_cnt = h_inv + T, *h_gat = h_cnt + T;
    for (int i = 0; i < T; i++) {
        const int c = off[i + 1] - off[i];
        const float inv = 1.0f / (float)c;
        memcpy(&h_inv[i], &inv, sizeof inv);
        h_cnt[i] = c;
    }
    for (int64_t sl = 0; sl < slots; sl++) {
        const int i = (int)(sl / 64), r = (int)(sl % 64);
        h_gat[sl] = (i < T && r < h_cnt[i]) ? tok[off[i] + r] : -1;
    }
    // captured graphs keep reading the geometry they were captured with: give
    // the new one its own buffer
    int rc = g.live_graphs > 0 || g.foreign_capture ? release(g.vsa_geo) : FH3_OK;
    if (rc == FH3_OK) rc = grow(g.vsa_geo, host.size() * sizeof(int), st);
    if (rc != FH3_OK) return rc;
    FH3_HIPCALL(hipDeviceSynchronize());  // earlier calls may still read the old geometry
    FH3_HIPCALL(hipMemcpy(g.vsa_geo.p, host.data(), host.size() * sizeof(int), hipMemcpyHostToDevice));
    memcpy(g.vsa_key, key, sizeof key);
    g.vsa_T = T;
    g.vsa_P = P;
    return FH3_OK;
}

static int vsa_dev(const Fh3VsaCfg *c, const float *q, const float *k, const float *v, int64_t ld, int64_t ldv,
                   const float *qn_w, const float *kn_w, float eps, const float *cs, const float *sn, int rot,
                   const float *gate, float *o, const Fh3Seq *sq, int heads, int hd, void *stream, const char *fn) {
    if (!q || !k || !v || !o || !sq || sq->seq_len <= 0 || heads <= 0 || hd <= 0)
        return set_err(FH3_E_INVALID, "%s: NULL pointer or non-positive size", fn);
    if (!fh3k_attn_head_dim_ok(hd)) return set_err(FH3_E_INVALID, "%s: head_dim %d is not supported (64 or 128)", fn, hd);
    const int tile = c && c->tile > 0 ? c->tile : 64;
    const float sparsity = c ? c->sparsity : 0.8f;
    if (tile > 64) return set_err(FH3_E_INVALID, "%s: tile %d above 64 is not supported on the device", fn, tile);
    if ((uintptr_t)q & 15u || (uintptr_t)k & 15u || (uintptr_t)v & 15u || (uintptr_t)o & 15u || (uintptr_t)gate & 15u)
        return set_err(FH3_E_INVALID, "%s: q, k, v, gate and o must be 16-byte aligned", fn);
    if ((int64_t)sq->seq_len * heads * hd > ((int64_t)1 << 31))
        return set_err(FH3_E_INVALID, "%s: n * heads * head_dim too large", fn);
    int rc = ensure_init();
    if (rc != FH3_OK) return rc;
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    hipStream_t st = stream ? (hipStream_t)stream : g.stream;
    if ((rc = vsa_plan(sq, tile, st, fn)) != FH3_OK) return rc;
    const int T = g.vsa_T, P = g.vsa_P, NV = T - P;
    int kv = 0;
    if (NV > 0) {  // src/core/fh3_vsa.c:165-172
        kv = (int)ceilf((1.0f - sparsity) * (float)NV);
        kv = kv < 1 ? 1 : (kv > NV ? NV : kv);
    }
    const int all = sparsity <= 0.0f || kv == NV;
    if ((rc = grow(g.vsa_ws, fh3k_vsa_ws_bytes(T, heads, hd), st)) != FH3_OK) return rc;
    const float *d_inv = (const float *)g.vsa_geo.p;
    const int *d_cnt = (const int *)(d_inv + T), *d_gat = d_cnt + T;
    const float scale = 1.0f / sqrtf((float)hd);
    FH3_HIPCALL(fh3k_vsa_attention(q, k, v, ld, ldv, qn_w, kn_w, eps, cs, sn, cs ? rot : 0, gate, o,
                                   (int64_t)heads * hd, heads, hd, d_inv, d_gat, d_cnt, T, P, kv, all, scale,
                                   g.vsa_ws.p, st));
    return FH3_OK;
}

extern "C" int fh3_hip_vsa_attention_dev(const Fh3VsaCfg *c, const float *d_q, const float *d_k, const float *d_v,
                                         const float *d_gate, float *d_o, const Fh3Seq *seq, int heads, int head_dim,
                                         void *stream) {
    const int64_t ld = (int64_t)heads * head_dim;
    return vsa_dev(c, d_q, d_k, d_v, ld, ld, nullptr, nullptr, 0.f, nullptr, nullptr, 0, d_gate, d_o, seq, heads,
                   head_dim, stream, "fh3_hip_vsa_attention_dev");
}

extern "C" int fh3_hip_vsa_attention_qkv_dev(const Fh3VsaCfg *c, const float *d_qkv, const float *d_qnorm_w,
                                             const float *d_knorm_w, float eps, const float *d_cos,
                                             const float *d_sin, int rot_dim, const float *d_gate, float *d_o,
                                             const Fh3Seq *seq, int heads, int head_dim, void *stream) {
    const char *fn = "fh3_hip_vsa_attention_qkv_dev";
    if (!d_qkv || !seq || seq->seq_len <= 0 || heads <= 0 || !fh3k_attn_head_dim_ok(head_dim))
        return set_err(FH3_E_INVALID, "%s: bad arguments", fn);
    if ((d_qnorm_w == nullptr) != (d_knorm_w == nullptr))
        return set_err(FH3_E_INVALID, "%s: give both q and k norm weights or neither", fn);
    if ((d_cos == nullptr) != (d_sin == nullptr) || (d_cos && (rot_dim <= 0 || rot_dim > head_dim || rot_dim % 2)))
        return set_err(FH3_E_INVALID, "%s: rope needs cos and sin with an even rot_dim <= head_dim", fn);
    if ((uintptr_t)d_qkv & 15u || (uintptr_t)d_cos & 15u || (uintptr_t)d_sin & 15u)
        return set_err(FH3_E_INVALID, "%s: qkv, cos and sin must be 16-byte aligned", fn);
    const int64_t inner = (int64_t)heads * head_dim;
    return vsa_dev(c, d_qkv, d_qkv + inner, d_qkv + 2 * inner, 3 * inner, 3 * inner, d_qnorm_w, d_knorm_w, eps, d_cos,
                   d_sin, rot_dim, d_gate, d_o, seq, heads, head_dim, stream, fn);
}

// ---------------------------------------------------------------------------
// fh3.h host-pointer wrappers
// ---------------------------------------------------------------------------
extern "C" size_t fh3_row_bytes(int type, int64_t n) {
    if (n <= 0) return 0;
    const int64_t b32 = (n + 31) / 32, b256 = (n + 255) / 256;
    switch (type) {
        case FH3_QUANT_F32: return (size_t)n * 4u;
        case FH3_QUANT_F16: return (size_t)n * 2u;
        case FH3_QUANT_BF16: return (size_t)n * 2u;
        case FH3_QUANT_Q4_0: return (size_t)b32 * 18u;
        case FH3_QUANT_Q4_1: return (size_t)b32 * 20u;
        case FH3_QUANT_Q5_0: return (size_t)b32 * 22u;
        case FH3_QUANT_Q5_1: return (size_t)b32 * 24u;
        case FH3_QUANT_Q8_0: return (size_t)b32 * 34u;
        case FH3_QUANT_Q8_1: return (size_t)b32 * 40u;
        case FH3_QUANT_Q2_K: return (size_t)b256 * 84u;
        case FH3_QUANT_Q3_K: return (size_t)b256 * 110u;
        case FH3_QUANT_Q4_K: return (size_t)b256 * 144u;
        case FH3_QUANT_Q5_K: return (size_t)b256 * 176u;
        case FH3_QUANT_Q6_K: return (size_t)b256 * 210u;
        case FH3_QUANT_Q8_K: return (size_t)b256 * 292u;
        default: return 0;
    }
}

static void report(const char *fn, int rc) {
    fprintf(stderr, "%s: GPU path failed (%d): %s\n", fn, rc, g_err);
}

extern "C" void fh3_dequant(int type, const void *src, float *dst, int64_t n) {
    if (!src || !dst || n <= 0) return;
    const int bl = fh3k_dequant_block_len(type);
    if (bl == 0) {
        set_err(FH3_E_INVALID, "fh3_dequant: unsupported type %d", type);
        fprintf(stderr, "fh3_dequant: unsupported type %d\n", type);
        return;
    }
    // whole blocks only, as the reference's decoders
    const int64_t cnt = (n / bl) * bl;
    if (cnt == 0) return;
    int rc = ensure_init();
    if (rc != FH3_OK) { report("fh3_dequant", rc); return; }
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    const size_t in_bytes = fh3_row_bytes(type, cnt), out_bytes = (size_t)cnt * sizeof(float);
    if ((rc = grow(g.st_w, in_bytes, g.stream)) != FH3_OK || (rc = grow(g.st_y, out_bytes, g.stream)) != FH3_OK) {
        report("fh3_dequant", rc);
        return;
    }
    const void *dsrc = registered(src, in_bytes);
    hipError_t e = dsrc ? hipSuccess : hipMemcpy(g.st_w.p, src, in_bytes, hipMemcpyHostToDevice);
    if (!dsrc) dsrc = g.st_w.p;
    if (e == hipSuccess) e = fh3k_dequant_f32(type, dsrc, (int64_t)in_bytes, cnt, 1, (float *)g.st_y.p, g.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g.stream);
    if (e == hipSuccess) e = hipMemcpy(dst, g.st_y.p, out_bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) report("fh3_dequant", hip_fail(e, "fh3_dequant"));
}

extern "C" void fh3_matmul(const Fh3W *w, const float *x, float *y, int n_tok, const float *bias_or_null) {
    if (!w || !x || !y || n_tok <= 0 || w->in <= 0 || w->out <= 0) return;
    int rc = ensure_init();
    if (rc != FH3_OK) { report("fh3_matmul", rc); return; }
    if (fh3k_dequant_block_len(w->type) == 0 || !w->data) {
        set_err(FH3_E_INVALID, "fh3_matmul: unsupported weight type %d", w->type);
        report("fh3_matmul", FH3_E_INVALID);
        return;
    }
    // refusals the device call would make, before the weights are staged
    if (w->in % fh3k_dequant_block_len(w->type) == 0 && (rc = check_gemm_span(w, n_tok, "fh3_matmul")) != FH3_OK) {
        report("fh3_matmul", rc);
        return;
    }
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    const size_t wb = fh3_row_bytes(w->type, w->in) * (size_t)w->out;
    const size_t xb = (size_t)n_tok * (size_t)w->in * sizeof(float);
    const size_t yb = (size_t)n_tok * (size_t)w->out * sizeof(float);
    const size_t bb = (size_t)w->out * sizeof(float);
    // a registered weight (fh3_hip_register_weights) is used in place
    const void *dw = registered(w->data, wb);
    if (dw && ((uintptr_t)dw & 15u)) dw = nullptr;
    if ((!dw && (rc = grow(g.st_w, wb, g.stream))) || (rc = grow(g.st_x, xb, g.stream)) || (rc = grow(g.st_y, yb, g.stream)) ||
        (bias_or_null && (rc = grow(g.st_b, bb, g.stream)))) {
        report("fh3_matmul", rc);
        return;
    }
    hipError_t e = dw ? hipSuccess : hipMemcpy(g.st_w.p, w->data, wb, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(g.st_x.p, x, xb, hipMemcpyHostToDevice);
    if (e == hipSuccess && bias_or_null) e = hipMemcpy(g.st_b.p, bias_or_null, bb, hipMemcpyHostToDevice);
    if (e != hipSuccess) { report("fh3_matmul", hip_fail(e, "fh3_matmul upload")); return; }
    Fh3W wd = *w;
    wd.data = (const uint8_t *)(dw ? dw : g.st_w.p);
    rc = fh3_hip_matmul_dev(&wd, (const float *)g.st_x.p, (float *)g.st_y.p, n_tok,
                            bias_or_null ? (const float *)g.st_b.p : nullptr, nullptr);
    if (rc != FH3_OK) { report("fh3_matmul", rc); return; }
    e = hipStreamSynchronize(g.stream);
    if (e == hipSuccess) e = hipMemcpy(y, g.st_y.p, yb, hipMemcpyDeviceToHost);
    if (e != hipSuccess) report("fh3_matmul", hip_fail(e, "fh3_matmul download"));
}

extern "C" void fh3_attention(const float *q, const float *k, const float *v, float *o, int n, int heads, int hd) {
    if (!q || !k || !v || !o || n <= 0 || heads <= 0 || hd <= 0) return;
    int rc = ensure_init();
    if (rc != FH3_OK) { report("fh3_attention", rc); return; }
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    const size_t b = (size_t)n * (size_t)heads * (size_t)hd * sizeof(float);
    if ((rc = grow(g.st_w, 3 * b, g.stream)) || (rc = grow(g.st_y, b, g.stream))) { report("fh3_attention", rc); return; }
    float *dq = (float *)g.st_w.p, *dk = dq + b / 4, *dv = dk + b / 4;
    hipError_t e = hipMemcpy(dq, q, b, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dk, k, b, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dv, v, b, hipMemcpyHostToDevice);
    if (e != hipSuccess) { report("fh3_attention", hip_fail(e, "fh3_attention upload")); return; }
    rc = fh3_hip_attention_dev(dq, dk, dv, (float *)g.st_y.p, n, heads, hd, nullptr);
    if (rc != FH3_OK) { report("fh3_attention", rc); return; }
    e = hipStreamSynchronize(g.stream);
    if (e == hipSuccess) e = hipMemcpy(o, g.st_y.p, b, hipMemcpyDeviceToHost);
    if (e != hipSuccess) report("fh3_attention", hip_fail(e, "fh3_attention download"));
}

extern "C" void fh3_vsa_attention(const Fh3VsaCfg *c, const float *q, const float *k, const float *v,
                                  const float *gate, float *o, const Fh3Seq *seq, int heads, int head_dim) {
    if (!q || !k || !v || !o || !seq || seq->seq_len <= 0 || heads <= 0 || head_dim <= 0) return;
    int rc = ensure_init();
    if (rc != FH3_OK) { report("fh3_vsa_attention", rc); return; }
    std::lock_guard<std::recursive_mutex> lk(g.mu);
    const size_t b = (size_t)seq->seq_len * (size_t)heads * (size_t)head_dim * sizeof(float);
    if ((rc = grow(g.st_w, (gate ? 4 : 3) * b, g.stream)) || (rc = grow(g.st_y, b, g.stream))) { report("fh3_vsa_attention", rc); return; }
    float *dq = (float *)g.st_w.p, *dk = dq + b / 4, *dv = dk + b / 4, *dg = gate ? dv + b / 4 : nullptr;
    hipError_t e = hipMemcpy(dq, q, b, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dk, k, b, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dv, v, b, hipMemcpyHostToDevice);
    if (e == hipSuccess && gate) e = hipMemcpy(dg, gate, b, hipMemcpyHostToDevice);
    if (e != hipSuccess) { report("fh3_vsa_attention", hip_fail(e, "fh3_vsa_attention upload")); return; }
    rc = fh3_hip_vsa_attention_dev(c, dq, dk, dv, dg, (float *)g.st_y.p, seq, heads, head_dim, nullptr);
    if (rc != FH3_OK) { report("fh3_vsa_attention", rc); return; }
    e = hipStreamSynchronize(g.stream);
    if (e == hipSuccess) e = hipMemcpy(o, g.st_y.p, b, hipMemcpyDeviceToHost);
    if (e != hipSuccess) report("fh3_vsa_attention", hip_fail(e, "fh3_vsa_attention download"));
}

extern "C" void fh3_matmul_scalar(const Fh3W *w, const float *x, float *y, int n_tok, const float *bias_or_null) {
    fh3_matmul(w, x, y, n_tok, bias_or_null);
}

extern "C" void fh3_matmul_avx2(const Fh3W *w, const float *x, float *y, int n_tok, const float *bias_or_null) {
    fh3_matmul(w, x, y, n_tok, bias_or_null);
}
