/*
 * fh3_trunk.h -- the FH3P packed trunk and its layer streamer, with the
 * device extension that feeds the HIP matmul.
 *
 * Host side (same contract as the reference):
 *   - FH3P file layout and descriptors: reference src/io/fh3_pack.h:14-71;
 *     fh3_pack_open/close/layer replace src/io/fh3_pack.c:23-217.
 *   - Streamer: a pinned prefix of whole layers plus two ring slots filled by
 *     a worker thread with pread (O_DIRECT when the filesystem allows it);
 *     fh3_trunk_open/close/prefetch/acquire/stats replace
 *     src/io/fh3_trunk.c:135-510, with the same slot choice, hit/miss and
 *     error semantics (acquire returns NULL on a short read).
 *   - fh3_plan_bytes/fh3_plan_check replace src/io/fh3_trunk.c:91-129.
 * Device side (new, no counterpart in the CPU-only reference):
 *   fh3_trunk_attach_device gives the trunk a second, HBM-level copy of the
 *   same policy.  Under a device byte budget, a prefix of layers is made
 *   resident in HBM once (the same fixed point as the host prefix, with
 *   device slots in place of host slots); every later layer streams through
 *   two device slots.  The host copies that feed them (the pinned prefix and
 *   the two host ring slots) move to page-locked memory, so an upload is a
 *   hipMemcpyAsync on a side stream that overlaps the kernels of the
 *   previous layer.  Three events per slot order the work without host
 *   waits on the compute path:
 *     ev_slot_free[s]  compute work enqueued so far (recorded when device
 *                      slot s is recycled; the upload stream waits on it),
 *     ev_uploaded[s]   upload into device slot s done (the compute stream
 *                      waits on it in fh3_trunk_acquire_dev),
 *     ev_host_read[s]  last upload out of host ring slot s done (the read
 *                      worker waits on it before it overwrites that slot).
 *   Contract (as for the host slots): work that reads a device slot pointer
 *   must be enqueued before the call that recycles that slot, i.e. before
 *   the next acquire_dev/prefetch_dev of a layer not already in a slot.
 */
#ifndef FH3_TRUNK_H
#define FH3_TRUNK_H

#include <stddef.h>
#include <stdint.h>
#include <stdbool.h>
#include <pthread.h>

#include "fh3/fh3.h"

#ifdef __cplusplus
extern "C" {
#endif

#define FH3_PACK_MAGIC 0x50334846u /* 'FH3P' */
#define FH3_PACK_VERSION 1u
#define FH3_PACK_ALIGNMENT 4096u
#define FH3_PACK_TENSORS_PER_LAYER 9u
#define FH3_PACK_MAX_TENSORS_PER_LAYER 16u

#pragma pack(push, 1)
/* 168 bytes */
typedef struct Fh3PackTensorDesc {
    char name[64];
    uint32_t type;            /* Fh3QuantType */
    uint32_t n_dims;
    int64_t shape[4];
    uint64_t offset_in_layer; /* 32-byte aligned */
    uint64_t size_bytes;
    int64_t in_dim;
    int64_t out_dim;
    uint8_t reserved[32];
} Fh3PackTensorDesc;

/* 24-byte head + tensor descriptors; on disk a layer descriptor is
 * index_bytes / num_layers bytes (it may hold fewer than 16 tensors) */
typedef struct Fh3PackLayerDesc {
    uint64_t file_offset;     /* 4096-aligned */
    uint64_t size_bytes;      /* 4096-aligned */
    uint32_t n_tensors;
    uint32_t reserved;
    Fh3PackTensorDesc tensors[FH3_PACK_MAX_TENSORS_PER_LAYER];
} Fh3PackLayerDesc;

/* 128 bytes */
typedef struct Fh3PackHeader {
    uint32_t magic;
    uint32_t version;
    uint32_t num_layers;
    uint32_t layer_alignment; /* 4096 */
    uint64_t index_offset;
    uint64_t index_bytes;
    uint64_t data_offset;
    uint64_t total_bytes;
    uint8_t reserved[80];
} Fh3PackHeader;
#pragma pack(pop)

/* The structs below have the reference's exact layout (its POSIX build), so
 * that callers which hold them by value -- the reference CLI keeps an
 * Fh3Trunk on its stack (src/cli/fh3_cli.c:750,963) -- link against this
 * library unchanged:
 *   Fh3File  src/io/fh3_portable_io.h:220-224
 *   Fh3Pack  src/io/fh3_pack.h:91-101
 *   Fh3Trunk src/io/fh3_trunk.h:26-68
 * State the reference does not have (the device extension, page-locked host
 * copies, the worker's errno) lives in a separate record that the library
 * keys by the Fh3Trunk's address; Fh3Trunk itself only holds the reference's
 * fields. */
typedef struct Fh3File {
    int fd;
    uint64_t size;
    bool is_direct;
} Fh3File;

typedef struct Fh3Pack {
    Fh3File file;
    Fh3PackHeader header;
    int num_layers;
    Fh3PackLayerDesc *layers;
    const uint8_t *mapped_base;
    size_t mapped_size;
} Fh3Pack;

/* Read the header and layer index; map the file read-only when possible.
 * FH3_OK, FH3_E_IO, FH3_E_TRUNCATED, FH3_E_BAD_MAGIC, FH3_E_BAD_VERSION,
 * FH3_E_INVALID or FH3_E_NOMEM (reference src/io/fh3_pack.c:23-110). */
int fh3_pack_open(const char *path, Fh3Pack *p);
void fh3_pack_close(Fh3Pack *p);
/* Views of layer L's tensors (run order qkv, gate_compress, out, fc1, fc2,
 * norm1, norm2, q_norm, k_norm) at `base` (a host or device copy of the
 * layer run), or into the mapping when base is NULL (reference
 * src/io/fh3_pack.c:140-217). */
Fh3LayerView fh3_pack_layer(const Fh3Pack *p, int L, const uint8_t *base);

/* reference include/fh3/fh3.h:134-140 */
typedef struct Fh3TrunkStats {
    uint64_t hits;
    uint64_t misses;
    uint64_t bytes_read;
    double read_s;
    double wait_s;
} Fh3TrunkStats;

/* Device-side counters of the extension.  As on the host, the first acquire
 * of a layer that had to be uploaded for it (by acquire_dev itself or by an
 * earlier prefetch_dev) is a miss; an acquire of a layer resident in HBM or
 * already consumed from its slot is a hit. */
typedef struct Fh3TrunkDevStats {
    uint64_t hits;
    uint64_t misses;
    uint64_t uploads;
    uint64_t bytes_uploaded;
    uint64_t resident_bytes;  /* device-resident prefix kept in HBM */
} Fh3TrunkDevStats;

typedef struct Fh3Trunk {
    Fh3Pack pack;
    Fh3File direct_file;          /* O_DIRECT descriptor (is_direct), else fd -1 */
    int num_layers;
    uint64_t budget_bytes;
    int npin;                     /* pinned prefix layers */
    size_t slot_size;             /* 4096-aligned ring slot size */
    uint8_t **pinned_layers;      /* [npin] host copies */
    uint8_t *ring_buf[2];         /* host ring slots */
    int ring_layer[2];            /* layer resident in each slot, or -1 */
    int active_slot;              /* -1 before the first acquire */
    int prefetch_layer;
    int prefetch_slot;
    bool prefetch_in_flight;
    double prefetch_start_time;
    double prefetch_io_time;
    /* worker thread */
    pthread_t thread;
    pthread_mutex_t mutex;
    pthread_cond_t start_cond;
    pthread_cond_t done_cond;
    bool worker_has_work;
    bool worker_done;
    bool thread_created;
    bool worker_stop;
    int worker_req_layer;
    int worker_req_slot;
    int64_t worker_read_bytes;
    Fh3TrunkStats stats;
} Fh3Trunk;

int fh3_trunk_open(const char *path, uint64_t budget_bytes, Fh3Trunk *t);
void fh3_trunk_close(Fh3Trunk *t);
void fh3_trunk_prefetch(Fh3Trunk *t, int L);
const uint8_t *fh3_trunk_acquire(Fh3Trunk *t, int L);
Fh3TrunkStats fh3_trunk_stats(const Fh3Trunk *t);
Fh3LayerView fh3_trunk_layer(const Fh3Trunk *t, int L, const uint8_t *base);
const Fh3Pack *fh3_trunk_pack(const Fh3Trunk *t);

/* Attach the streamer to the GPU (see the file comment).  dev_budget_bytes
 * bounds the HBM held by the trunk (resident prefix + 2 device slots);
 * compute_stream NULL = the library's compute stream.  Call once, before the
 * first prefetch/acquire.  FH3_OK, FH3_E_INVALID, FH3_E_NOMEM or FH3_ERR
 * (fh3_hip_last_error says why). */
int fh3_trunk_attach_device(Fh3Trunk *t, uint64_t dev_budget_bytes, void *compute_stream);
/* Start bringing layer L into the idle device slot: a host-resident layer is
 * uploaded at once (asynchronously); a disk layer is read ahead by the worker
 * and uploaded by the acquire.  Either way this call recycles the idle slot:
 * the upload waits only for the compute enqueued before it, so with the loop
 * acquire_dev(L), prefetch_dev(L+1), block L's work, layer L+1's copy runs
 * while block L computes. */
void fh3_trunk_prefetch_dev(Fh3Trunk *t, int L);
/* Device pointer of layer L's run; work enqueued on the compute stream after
 * this call sees its bytes.  NULL on a short read or a HIP error (the message
 * in fh3_hip_last_error); a later acquire of the same layer tries again. */
const uint8_t *fh3_trunk_acquire_dev(Fh3Trunk *t, int L);
Fh3TrunkDevStats fh3_trunk_dev_stats(const Fh3Trunk *t);
/* Test hook, no counterpart in the reference: make the next slot upload fail
 * as a HIP error would, at its copy (what = 1) or at the event that orders it
 * behind the compute (what = 2); 0 clears.  For tests of the error path of
 * fh3_trunk_acquire_dev / fh3_trunk_prefetch_dev. */
int fh3_trunk_inject_upload_failure(Fh3Trunk *t, int what);

/* For bindings that cannot mirror the struct (it holds pthread objects):
 * its size, so they can allocate one, and the split chosen at open/attach.
 * No counterpart in the reference, whose callers read the fields directly. */
typedef struct Fh3TrunkInfo {
    int num_layers;
    int npin;
    uint64_t slot_size;
    int dpin;                 /* 0 until attached */
    uint64_t dev_slot_size;   /* 0 while every layer is resident or unattached */
} Fh3TrunkInfo;

size_t fh3_trunk_struct_bytes(void);
int fh3_trunk_info(const Fh3Trunk *t, Fh3TrunkInfo *out);

/* Memory plan (reference include/fh3/fh3.h:204-215). */
typedef struct Fh3Plan {
    uint64_t budget_bytes;
    uint64_t min_bytes;
    uint64_t pinned_bytes;
    uint64_t ring_bytes;
    uint64_t activation_bytes;
    uint64_t table_bytes;
    uint64_t total_bytes;
} Fh3Plan;

uint64_t fh3_plan_bytes(const Fh3Plan *p);
int fh3_plan_check(const Fh3Plan *p);
uint64_t fh3_mem_available(void);

#ifdef __cplusplus
}
#endif

#endif /* FH3_TRUNK_H */
