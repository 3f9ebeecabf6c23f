/*
 * fh3_trunk.c -- the layer streamer over an FH3P pack (C99, POSIX threads),
 * with its HBM extension.
 *
 * Host policy (reference src/io/fh3_trunk.c:135-510): a prefix of whole
 * layers is read once into host memory; every later layer is read on demand
 * into one of two ring slots by a worker thread, one layer in flight at a
 * time, the slot being the one not handed out by the last acquire.  A scan of
 * the trunk therefore costs (num_layers - npin) reads per pass however the
 * scans repeat, where an LRU of the same capacity would miss every time.
 *
 * Device policy (this file's addition): the same prefix/ring split again at
 * the HBM level, with uploads from page-locked host memory on a side stream.
 * See the comments of include/fh3/fh3_trunk.h for the event protocol.
 */
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#include "fh3/fh3_trunk.h"
#include "fh3/fh3_hip.h"
#include "fh3_hip_internal.h"

#define PAGE 4096u
#define FIXED_POINT_MAX_ITERS 1000

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static size_t page_up(uint64_t n) { return (size_t)((n + PAGE - 1) & ~(uint64_t)(PAGE - 1)); }

static size_t run_bytes(const Fh3Trunk *t, int L) { return (size_t)t->pack.layers[L].size_bytes; }

/* ------------------------------------------------------------------------- */
/* per-trunk state beyond the reference's struct                            */
/* ------------------------------------------------------------------------- */

/* Fh3Trunk has the reference's layout, so what this library adds lives here,
 * one record per open trunk, found by the trunk's address.  Created by
 * fh3_trunk_open, freed by fh3_trunk_close. */
typedef struct TrunkExt {
    const Fh3Trunk *t;
    struct TrunkExt *next;
    bool sync_init;               /* t->mutex and conditions initialised */
    int worker_errno;             /* errno of the last job's failed read, or 0 */
    bool host_pinned;             /* pinned_layers / ring_buf from hipHostMalloc */
    /* device extension (zero until fh3_trunk_attach_device) */
    bool device;
    int dpin;                     /* device-resident prefix layers */
    size_t dev_slot_size;
    void *compute_stream;         /* hipStream_t the matmuls run on */
    void *upload_stream;          /* hipStream_t of the slot uploads */
    uint8_t *dev_resident;        /* one allocation for the resident prefix */
    uint8_t **dev_layers;         /* [dpin] pointers into dev_resident */
    uint8_t *dev_slot[2];
    int dev_layer[2];             /* layer uploaded (or enqueued) into slot s, or -1 */
    bool dev_fresh[2];            /* upload not yet consumed by an acquire */
    int dev_active;               /* -1 before the first streamed acquire */
    void *ev_uploaded[2];         /* hipEvent_t */
    void *ev_slot_free[2];
    void *ev_host_read[2];
    bool slot_free_pending[2];    /* ev_slot_free[s] recorded by the prefetch that recycled slot s */
    int inject_fail;              /* test hook: 1 the next upload's copy fails, 2 its event record */
    Fh3TrunkDevStats dev_stats;
} TrunkExt;

static pthread_mutex_t g_ext_mu = PTHREAD_MUTEX_INITIALIZER;
static TrunkExt *g_ext;

static TrunkExt *ext_of(const Fh3Trunk *t) {
    pthread_mutex_lock(&g_ext_mu);
    TrunkExt *x = g_ext;
    while (x && x->t != t) x = x->next;
    pthread_mutex_unlock(&g_ext_mu);
    return x;
}

static TrunkExt *ext_new(const Fh3Trunk *t) {
    TrunkExt *x = (TrunkExt *)calloc(1, sizeof(TrunkExt));
    if (!x) return NULL;
    x->t = t;
    x->dev_layer[0] = x->dev_layer[1] = -1;
    x->dev_active = -1;
    pthread_mutex_lock(&g_ext_mu);
    x->next = g_ext;
    g_ext = x;
    pthread_mutex_unlock(&g_ext_mu);
    return x;
}

/* Unlink t's record (NULL when t has none: never opened, or closed). */
static TrunkExt *ext_take(const Fh3Trunk *t) {
    pthread_mutex_lock(&g_ext_mu);
    TrunkExt **pp = &g_ext;
    while (*pp && (*pp)->t != t) pp = &(*pp)->next;
    TrunkExt *x = *pp;
    if (x) *pp = x->next;
    pthread_mutex_unlock(&g_ext_mu);
    return x;
}

/* Read n bytes of the file at off (clamped to the file end) into dst.  The
 * O_DIRECT descriptor is used when dst, off and n are page aligned and dst is
 * ordinary memory; anything else goes through the buffered descriptor, and so
 * does every later read once a direct read fails (a filesystem without
 * O_DIRECT, or a destination the kernel cannot pin for DMA: page-locked
 * memory mapped by the GPU driver gives EFAULT).  Returns the bytes read, or
 * FH3_E_IO with *err set to errno. */
static int64_t read_run(Fh3Trunk *t, const TrunkExt *x, void *dst, size_t n, uint64_t off, int *err) {
    const uint64_t size = t->pack.file.size;
    if (off >= size) return 0;
    if (n > size - off) n = (size_t)(size - off);
    int fd = t->pack.file.fd;
    if (t->direct_file.is_direct && !x->host_pinned && (uintptr_t)dst % PAGE == 0 && off % PAGE == 0 &&
        n % PAGE == 0)
        fd = t->direct_file.fd;
    size_t got = 0;
    while (got < n) {
        ssize_t r = pread(fd, (uint8_t *)dst + got, n - got, (off_t)(off + got));
        if (r < 0) {
            if (errno == EINTR) continue;
            if (fd == t->direct_file.fd) {
                t->direct_file.is_direct = false;
                fd = t->pack.file.fd;
                continue;
            }
            if (err) *err = errno;
            return FH3_E_IO;
        }
        if (r == 0) break;
        got += (size_t)r;
    }
    return (int64_t)got;
}

/* Largest prefix [0, n) such that the prefix plus two slots as large as the
 * biggest layer after it fit in budget.  The slot size depends on n and n on
 * the slot size, so iterate from "slot = biggest layer" to a fixed point
 * (reference src/io/fh3_trunk.c:161-200; same iteration, so the same split). */
static void plan_prefix(const Fh3Pack *p, uint64_t budget, int *n_out, size_t *slot_out) {
    const int nl = p->num_layers;
    size_t biggest = 0;
    for (int i = 0; i < nl; i++)
        if (p->layers[i].size_bytes > biggest) biggest = (size_t)p->layers[i].size_bytes;
    biggest = page_up(biggest);
    size_t slot = biggest;
    int n = 0;
    for (int it = 0; it < FIXED_POINT_MAX_ITERS; it++) {
        const uint64_t avail = budget > 2ull * slot ? budget - 2ull * slot : 0;
        int k = 0;
        uint64_t used = 0;
        while (k < nl && used + p->layers[k].size_bytes <= avail) used += p->layers[k++].size_bytes;
        size_t need = 0;
        for (int i = k; i < nl; i++)
            if (p->layers[i].size_bytes > need) need = (size_t)p->layers[i].size_bytes;
        need = page_up(need);
        if (k == n && need == slot) break;
        n = k;
        slot = need;
    }
    *n_out = n;
    *slot_out = slot ? slot : biggest;
}

/* ------------------------------------------------------------------------- */
/* worker                                                                    */
/* ------------------------------------------------------------------------- */

static void *worker_main(void *arg) {
    TrunkExt *x = (TrunkExt *)arg;
    Fh3Trunk *t = (Fh3Trunk *)x->t;
    pthread_mutex_lock(&t->mutex);
    for (;;) {
        while (!t->worker_has_work && !t->worker_stop) pthread_cond_wait(&t->start_cond, &t->mutex);
        if (t->worker_stop) break;
        const int L = t->worker_req_layer, s = t->worker_req_slot;
        void *host_read = x->device ? x->ev_host_read[s] : NULL;
        pthread_mutex_unlock(&t->mutex);

        int64_t got = FH3_ERR;
        int err = 0;
        double io = 0.0;
        /* an upload enqueued earlier may still be reading host slot s */
        if (!host_read || fh3i_event_sync(host_read) == FH3_OK) {
            const double t0 = now_s();
            got = read_run(t, x, t->ring_buf[s], run_bytes(t, L), t->pack.layers[L].file_offset, &err);
            io = now_s() - t0;
        } else {
            err = -1; /* the wait for the previous upload failed */
        }

        pthread_mutex_lock(&t->mutex);
        t->worker_read_bytes = got;
        x->worker_errno = err;
        t->prefetch_io_time = io;
        t->worker_has_work = false;
        t->worker_done = true;
        pthread_cond_signal(&t->done_cond);
    }
    pthread_mutex_unlock(&t->mutex);
    return NULL;
}

/* Block until the job in flight is done; returns the seconds waited. */
static double wait_job(Fh3Trunk *t) {
    const double w0 = now_s();
    pthread_mutex_lock(&t->mutex);
    while (!t->worker_done) pthread_cond_wait(&t->done_cond, &t->mutex);
    pthread_mutex_unlock(&t->mutex);
    t->prefetch_in_flight = false;
    return now_s() - w0;
}

/* Record the finished job's slot as holding its layer, or as empty after a
 * short read; true when the read was whole. */
static bool settle_job(Fh3Trunk *t) {
    const bool whole = t->worker_read_bytes == (int64_t)run_bytes(t, t->prefetch_layer);
    t->ring_layer[t->prefetch_slot] = whole ? t->prefetch_layer : -1;
    return whole;
}

/* ------------------------------------------------------------------------- */
/* open / close                                                              */
/* ------------------------------------------------------------------------- */

static void free_host(const TrunkExt *x, void *p) {
    if (!p) return;
    if (x->host_pinned) fh3i_host_free(p);
    else free(p);
}

static void *alloc_page_aligned(size_t n) {
    void *p = NULL;
    return (n && posix_memalign(&p, PAGE, n) == 0) ? p : NULL;
}

static int open_fail(Fh3Trunk *t, int code) {
    fh3_trunk_close(t);
    return code;
}

int fh3_trunk_open(const char *path, uint64_t budget_bytes, Fh3Trunk *t) {
    if (!path || !t) return FH3_ERR;
    memset(t, 0, sizeof(*t));
    t->direct_file.fd = -1;
    int rc = fh3_pack_open(path, &t->pack);
    if (rc != FH3_OK) return rc;  /* the reader has released what it opened */
    TrunkExt *x = ext_new(t);
    if (!x) {
        fh3_pack_close(&t->pack);
        return FH3_E_NOMEM;
    }
    t->num_layers = t->pack.num_layers;
    t->budget_bytes = budget_bytes;
    t->ring_layer[0] = t->ring_layer[1] = -1;
    t->active_slot = t->prefetch_layer = t->prefetch_slot = -1;

    t->direct_file.fd = open(path, O_RDONLY | O_CLOEXEC | O_DIRECT);
    t->direct_file.is_direct = t->direct_file.fd >= 0;
    t->direct_file.size = t->pack.file.size;

    plan_prefix(&t->pack, budget_bytes, &t->npin, &t->slot_size);

    if (t->npin > 0) {
        t->pinned_layers = (uint8_t **)calloc((size_t)t->npin, sizeof(uint8_t *));
        if (!t->pinned_layers) return open_fail(t, FH3_E_NOMEM);
        for (int L = 0; L < t->npin; L++) {
            const size_t n = run_bytes(t, L);
            if (!(t->pinned_layers[L] = (uint8_t *)alloc_page_aligned(page_up(n)))) return open_fail(t, FH3_E_NOMEM);
            if (read_run(t, x, t->pinned_layers[L], n, t->pack.layers[L].file_offset, NULL) != (int64_t)n)
                return open_fail(t, FH3_E_IO);
        }
    }
    for (int s = 0; s < 2; s++)
        if (!(t->ring_buf[s] = (uint8_t *)alloc_page_aligned(t->slot_size))) return open_fail(t, FH3_E_NOMEM);

    pthread_mutex_init(&t->mutex, NULL);
    pthread_cond_init(&t->start_cond, NULL);
    pthread_cond_init(&t->done_cond, NULL);
    x->sync_init = true;
    if (pthread_create(&t->thread, NULL, worker_main, x) != 0) return open_fail(t, FH3_ERR);
    t->thread_created = true;
    return FH3_OK;
}

static void detach_device(TrunkExt *x) {
    /* kernels and uploads may still read the buffers freed below */
    if (x->upload_stream) fh3i_stream_sync(x->upload_stream);
    if (x->device || x->upload_stream) fh3i_stream_sync(x->compute_stream);
    for (int s = 0; s < 2; s++) {
        fh3_hip_free(x->dev_slot[s]);
        fh3i_event_destroy(x->ev_uploaded[s]);
        fh3i_event_destroy(x->ev_slot_free[s]);
        fh3i_event_destroy(x->ev_host_read[s]);
        x->dev_slot[s] = NULL;
        x->ev_uploaded[s] = x->ev_slot_free[s] = x->ev_host_read[s] = NULL;
        x->dev_layer[s] = -1;
        x->slot_free_pending[s] = false;
    }
    fh3_hip_free(x->dev_resident);
    x->dev_resident = NULL;
    free(x->dev_layers);
    x->dev_layers = NULL;
    fh3i_stream_destroy(x->upload_stream);
    x->upload_stream = NULL;
    x->device = false;
    x->dpin = 0;
}

void fh3_trunk_close(Fh3Trunk *t) {
    if (!t) return;
    TrunkExt *x = ext_take(t);
    if (!x) return;  /* not open */
    if (t->thread_created) {
        if (t->prefetch_in_flight) wait_job(t);
        pthread_mutex_lock(&t->mutex);
        t->worker_stop = true;
        pthread_cond_signal(&t->start_cond);
        pthread_mutex_unlock(&t->mutex);
        pthread_join(t->thread, NULL);
        t->thread_created = false;
    }
    if (x->sync_init) {
        pthread_mutex_destroy(&t->mutex);
        pthread_cond_destroy(&t->start_cond);
        pthread_cond_destroy(&t->done_cond);
    }
    detach_device(x);
    if (t->pinned_layers) {
        for (int i = 0; i < t->npin; i++) free_host(x, t->pinned_layers[i]);
        free(t->pinned_layers);
        t->pinned_layers = NULL;
    }
    t->npin = 0;
    for (int s = 0; s < 2; s++) {
        free_host(x, t->ring_buf[s]);
        t->ring_buf[s] = NULL;
    }
    if (t->direct_file.fd >= 0) close(t->direct_file.fd);
    t->direct_file.fd = -1;
    t->direct_file.is_direct = false;
    fh3_pack_close(&t->pack);
    free(x);
}

/* ------------------------------------------------------------------------- */
/* host prefetch / acquire                                                   */
/* ------------------------------------------------------------------------- */

void fh3_trunk_prefetch(Fh3Trunk *t, int L) {
    if (!t || L < 0 || L >= t->num_layers || L < t->npin) return;
    if (t->active_slot >= 0 && t->ring_layer[t->active_slot] == L) return;
    const int other = t->active_slot == 0 ? 1 : 0;
    if (t->active_slot >= 0 && t->ring_layer[other] == L && !t->prefetch_in_flight) return;
    if (t->prefetch_in_flight && t->prefetch_layer == L) return;
    if (t->prefetch_in_flight) {
        wait_job(t);
        settle_job(t);
    }
    /* the slot not handed out by the last acquire */
    const int idle = t->active_slot == 0 ? 1 : 0;
    t->ring_layer[idle] = -1;
    t->prefetch_layer = L;
    t->prefetch_slot = idle;
    t->prefetch_in_flight = true;
    t->prefetch_start_time = now_s();
    pthread_mutex_lock(&t->mutex);
    t->worker_req_layer = L;
    t->worker_req_slot = idle;
    t->worker_has_work = true;
    t->worker_done = false;
    pthread_cond_signal(&t->start_cond);
    pthread_mutex_unlock(&t->mutex);
}

const uint8_t *fh3_trunk_acquire(Fh3Trunk *t, int L) {
    if (!t || L < 0 || L >= t->num_layers) return NULL;
    if (L < t->npin) {
        t->stats.hits++;
        return t->pinned_layers[L];
    }
    if (t->active_slot >= 0 && t->ring_layer[t->active_slot] == L) {
        t->stats.hits++;
        return t->ring_buf[t->active_slot];
    }
    const int other = t->active_slot == 0 ? 1 : 0;
    if (t->ring_layer[other] == L) {
        t->active_slot = other;
        t->stats.hits++;
        return t->ring_buf[other];
    }
    /* a miss: read it now unless the worker already is */
    if (!(t->prefetch_in_flight && t->prefetch_layer == L)) fh3_trunk_prefetch(t, L);
    const double waited = wait_job(t);
    if (!settle_job(t)) return NULL;
    t->active_slot = t->prefetch_slot;
    t->stats.misses++;
    t->stats.bytes_read += run_bytes(t, L);
    t->stats.read_s += t->prefetch_io_time;
    t->stats.wait_s += waited;
    return t->ring_buf[t->active_slot];
}

Fh3TrunkStats fh3_trunk_stats(const Fh3Trunk *t) {
    Fh3TrunkStats z;
    memset(&z, 0, sizeof(z));
    return t ? t->stats : z;
}

Fh3LayerView fh3_trunk_layer(const Fh3Trunk *t, int L, const uint8_t *base) {
    Fh3LayerView z;
    memset(&z, 0, sizeof(z));
    return t ? fh3_pack_layer(&t->pack, L, base) : z;
}

const Fh3Pack *fh3_trunk_pack(const Fh3Trunk *t) { return t ? &t->pack : NULL; }

/* ------------------------------------------------------------------------- */
/* device extension                                                          */
/* ------------------------------------------------------------------------- */

/* Move the host prefix and ring slots to page-locked memory (all or nothing). */
static int pin_host_copies(Fh3Trunk *t, TrunkExt *x) {
    const int n = t->npin + 2;
    void **fresh = (void **)calloc((size_t)n, sizeof(void *));
    if (!fresh) return FH3_E_NOMEM;
    int rc = FH3_OK;
    for (int i = 0; i < n && rc == FH3_OK; i++) {
        const size_t bytes = i < t->npin ? page_up(run_bytes(t, i)) : t->slot_size;
        rc = fh3i_host_alloc(&fresh[i], bytes);
    }
    if (rc != FH3_OK) {
        for (int i = 0; i < n; i++) fh3i_host_free(fresh[i]);
        free(fresh);
        return rc;
    }
    for (int i = 0; i < n; i++) {
        uint8_t **slot = i < t->npin ? &t->pinned_layers[i] : &t->ring_buf[i - t->npin];
        memcpy(fresh[i], *slot, i < t->npin ? run_bytes(t, i) : t->slot_size);
        free(*slot);
        *slot = (uint8_t *)fresh[i];
    }
    free(fresh);
    x->host_pinned = true;
    return FH3_OK;
}

/* Copy the device-resident prefix into HBM, reading from disk what the host
 * does not hold. */
static int fill_resident(Fh3Trunk *t, TrunkExt *x) {
    uint64_t total = 0;
    for (int L = 0; L < x->dpin; L++) total += page_up(run_bytes(t, L));
    if (!total) return FH3_OK;
    x->dev_layers = (uint8_t **)calloc((size_t)x->dpin, sizeof(uint8_t *));
    if (!x->dev_layers) return FH3_E_NOMEM;
    int rc = fh3_hip_malloc((void **)&x->dev_resident, (size_t)total);
    if (rc != FH3_OK) return rc;
    uint8_t *bounce = NULL;
    uint64_t at = 0;
    for (int L = 0; L < x->dpin && rc == FH3_OK; L++) {
        const size_t n = run_bytes(t, L);
        const uint8_t *src = L < t->npin ? t->pinned_layers[L] : NULL;
        if (!src) {
            if (!bounce && !(bounce = (uint8_t *)alloc_page_aligned(t->slot_size))) {
                rc = FH3_E_NOMEM;
                break;
            }
            if (read_run(t, x, bounce, n, t->pack.layers[L].file_offset, NULL) != (int64_t)n) {
                rc = fh3i_set_error(FH3_E_IO, "fh3_trunk_attach_device: short read of a resident layer");
                break;
            }
            src = bounce;
        }
        x->dev_layers[L] = x->dev_resident + at;
        rc = fh3_hip_memcpy_htod(x->dev_layers[L], src, n);
        at += page_up(n);
    }
    free(bounce);
    x->dev_stats.resident_bytes = rc == FH3_OK ? total : 0;
    return rc;
}

int fh3_trunk_attach_device(Fh3Trunk *t, uint64_t dev_budget_bytes, void *compute_stream) {
    TrunkExt *x = t ? ext_of(t) : NULL;
    if (!x || !t->thread_created) return fh3i_set_error(FH3_E_INVALID, "fh3_trunk_attach_device: trunk not open");
    if (x->device) return fh3i_set_error(FH3_E_INVALID, "fh3_trunk_attach_device: already attached");
    if (t->prefetch_in_flight) {
        wait_job(t);
        settle_job(t);
    }
    int rc = x->host_pinned ? FH3_OK : pin_host_copies(t, x);
    if (rc != FH3_OK) return rc;

    x->compute_stream = compute_stream;
    plan_prefix(&t->pack, dev_budget_bytes, &x->dpin, &x->dev_slot_size);
    rc = fill_resident(t, x);
    if (rc == FH3_OK) rc = fh3i_stream_create(&x->upload_stream);
    for (int s = 0; s < 2 && rc == FH3_OK; s++) {
        if (x->dpin < t->num_layers) rc = fh3_hip_malloc((void **)&x->dev_slot[s], x->dev_slot_size);
        if (rc == FH3_OK) rc = fh3i_event_create(&x->ev_uploaded[s]);
        if (rc == FH3_OK) rc = fh3i_event_create(&x->ev_slot_free[s]);
        if (rc == FH3_OK) rc = fh3i_event_create(&x->ev_host_read[s]);
    }
    if (rc != FH3_OK) {
        detach_device(x);
        return rc;
    }
    pthread_mutex_lock(&t->mutex);
    x->device = true;
    pthread_mutex_unlock(&t->mutex);
    return FH3_OK;
}

/* Order slot s's next upload behind the compute work enqueued so far, the
 * last that may read it: the call that recycles a slot marks this point. */
static int mark_slot_free(TrunkExt *x, int s) {
    if (x->inject_fail == 2) {
        x->inject_fail = 0;
        return fh3i_set_error(FH3_ERR, "hipEventRecord: injected failure (fh3_trunk_inject_upload_failure)");
    }
    return fh3i_event_record(x->ev_slot_free[s], x->compute_stream);
}

/* Enqueue "device slot s <- src" behind the work that last read slot s: the
 * compute enqueued before the prefetch that recycled the slot when one did
 * (a disk layer's prefetch_dev), else the compute enqueued so far.
 * host_slot >= 0 names the host ring slot src lies in, so the worker will not
 * overwrite it before the copy ends. */
static int upload(const Fh3Trunk *t, TrunkExt *x, int s, int L, const uint8_t *src, int host_slot) {
    const size_t n = run_bytes(t, L);
    x->dev_layer[s] = -1;
    int rc = x->slot_free_pending[s] ? FH3_OK : mark_slot_free(x, s);
    x->slot_free_pending[s] = false;
    if (rc == FH3_OK) rc = fh3i_stream_wait(x->upload_stream, x->ev_slot_free[s]);
    if (rc == FH3_OK && x->inject_fail == 1) {
        x->inject_fail = 0;
        rc = fh3i_set_error(FH3_ERR, "hipMemcpyAsync: injected failure (fh3_trunk_inject_upload_failure)");
    }
    if (rc == FH3_OK) rc = fh3i_copy_async(x->dev_slot[s], src, n, x->upload_stream);
    if (rc == FH3_OK) rc = fh3i_event_record(x->ev_uploaded[s], x->upload_stream);
    if (rc == FH3_OK && host_slot >= 0) rc = fh3i_event_record(x->ev_host_read[host_slot], x->upload_stream);
    if (rc != FH3_OK) return rc;
    x->dev_layer[s] = L;
    x->dev_fresh[s] = true;
    x->dev_stats.uploads++;
    x->dev_stats.bytes_uploaded += n;
    return FH3_OK;
}

void fh3_trunk_prefetch_dev(Fh3Trunk *t, int L) {
    TrunkExt *x = t ? ext_of(t) : NULL;
    if (!x || !x->device || L < 0 || L >= t->num_layers || L < x->dpin) return;
    if (x->dev_active >= 0 && x->dev_layer[x->dev_active] == L) return;
    const int idle = x->dev_active == 0 ? 1 : 0;
    if (x->dev_layer[idle] == L) return;
    if (L < t->npin) {
        (void)upload(t, x, idle, L, t->pinned_layers[L], -1);
        return;
    }
    /* A disk layer: read ahead; the acquire uploads it.  This call recycles
     * the idle slot, so its upload needs only the compute enqueued so far
     * (the block that last read it), not the block the caller enqueues next:
     * the copy then overlaps that block. */
    if (!x->slot_free_pending[idle] && mark_slot_free(x, idle) == FH3_OK) {
        x->slot_free_pending[idle] = true;
        x->dev_layer[idle] = -1;
    }
    fh3_trunk_prefetch(t, L);
}

int fh3_trunk_inject_upload_failure(Fh3Trunk *t, int what) {
    TrunkExt *x = t ? ext_of(t) : NULL;
    if (!x || !x->device || what < 0 || what > 2)
        return fh3i_set_error(FH3_E_INVALID, "fh3_trunk_inject_upload_failure: trunk not attached or bad kind");
    x->inject_fail = what;
    return FH3_OK;
}

const uint8_t *fh3_trunk_acquire_dev(Fh3Trunk *t, int L) {
    TrunkExt *x = t ? ext_of(t) : NULL;
    if (!x || !x->device || L < 0 || L >= t->num_layers) return NULL;
    if (L < x->dpin) {
        x->dev_stats.hits++;
        return x->dev_layers[L];
    }
    int s = -1;
    if (x->dev_active >= 0 && x->dev_layer[x->dev_active] == L)
        s = x->dev_active;
    else if (x->dev_layer[x->dev_active == 0 ? 1 : 0] == L)
        s = x->dev_active == 0 ? 1 : 0;
    if (s < 0) {
        s = x->dev_active == 0 ? 1 : 0;
        const uint8_t *src = fh3_trunk_acquire(t, L); /* host prefix or a host ring slot */
        if (!src) {
            char msg[160];
            snprintf(msg, sizeof msg, "fh3_trunk_acquire_dev: layer %d: read %lld of %zu bytes (%s)", L,
                     (long long)t->worker_read_bytes, run_bytes(t, L),
                     x->worker_errno > 0 ? strerror(x->worker_errno)
                                         : x->worker_errno < 0 ? "waiting for an upload failed" : "short file");
            fh3i_set_error(FH3_E_IO, msg);
            return NULL;
        }
        if (upload(t, x, s, L, src, L < t->npin ? -1 : t->active_slot) != FH3_OK) return NULL;
    }
    if (fh3i_stream_wait(x->compute_stream, x->ev_uploaded[s]) != FH3_OK) return NULL;
    x->dev_active = s;
    if (x->dev_fresh[s]) {
        x->dev_fresh[s] = false;
        x->dev_stats.misses++;
    } else {
        x->dev_stats.hits++;
    }
    return x->dev_slot[s];
}

Fh3TrunkDevStats fh3_trunk_dev_stats(const Fh3Trunk *t) {
    Fh3TrunkDevStats z;
    memset(&z, 0, sizeof(z));
    const TrunkExt *x = t ? ext_of(t) : NULL;
    return x ? x->dev_stats : z;
}

size_t fh3_trunk_struct_bytes(void) { return sizeof(Fh3Trunk); }

int fh3_trunk_info(const Fh3Trunk *t, Fh3TrunkInfo *out) {
    const TrunkExt *x = t ? ext_of(t) : NULL;
    if (!x || !out) return FH3_ERR;
    memset(out, 0, sizeof(*out));
    out->num_layers = t->num_layers;
    out->npin = t->npin;
    out->slot_size = t->slot_size;
    out->dpin = x->device ? x->dpin : 0;
    out->dev_slot_size = x->dev_slot[0] ? x->dev_slot_size : 0;
    return FH3_OK;
}

/* ------------------------------------------------------------------------- */
/* memory plan (reference src/io/fh3_trunk.c:91-129)                         */
/* ------------------------------------------------------------------------- */

uint64_t fh3_plan_bytes(const Fh3Plan *p) {
    if (!p) return 0;
    const uint64_t parts = p->pinned_bytes + p->ring_bytes + p->activation_bytes + p->table_bytes;
    return parts ? parts : p->total_bytes ? p->total_bytes : p->budget_bytes;
}

uint64_t fh3_mem_available(void) {
    FILE *f = fopen("/proc/meminfo", "r");
    if (!f) return 0;
    char line[256];
    unsigned long long kb = 0;
    bool found = false;
    while (!found && fgets(line, sizeof line, f)) found = sscanf(line, "MemAvailable: %llu kB", &kb) == 1;
    fclose(f);
    return found ? (uint64_t)kb * 1024u : 0;
}

int fh3_plan_check(const Fh3Plan *p) {
    if (!p) return FH3_ERR;
    const double gib = 1024.0 * 1024.0 * 1024.0;
    const uint64_t need = fh3_plan_bytes(p);
    if (p->min_bytes && need < p->min_bytes) {
        fprintf(stderr, "fh3: error: plan of %.2f GB is below the %.2f GB minimum (short by %.2f GB)\n",
                need / gib, p->min_bytes / gib, (p->min_bytes - need) / gib);
        return FH3_E_NOMEM;
    }
    /* leave 5% of the available RAM to the rest of the system */
    const uint64_t limit = (uint64_t)(0.95 * (double)fh3_mem_available());
    if (limit && need > limit) {
        fprintf(stderr, "fh3: error: plan of %.2f GB exceeds 95%% of available RAM, %.2f GB (short by %.2f GB)\n",
                need / gib, limit / gib, (need - limit) / gib);
        return FH3_E_NOMEM;
    }
    return FH3_OK;
}
