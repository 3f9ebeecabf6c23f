/*
 * fh3_pack.c -- reader of the FH3P packed trunk (C99, POSIX).
 *
 * File layout (reference src/io/fh3_pack.h:14-71, writer tools/pack_dit.py):
 *   [0, 128)                   Fh3PackHeader
 *   [index_offset, +index_bytes) num_layers descriptors of index_bytes /
 *                              num_layers bytes each: a 24-byte head
 *                              (file_offset, size_bytes, n_tensors, reserved)
 *                              followed by 168-byte tensor descriptors
 *   layer runs                 4096-aligned, tensors 32-aligned inside a run
 * Error codes follow reference src/io/fh3_pack.c:23-110.
 */
#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "fh3/fh3_trunk.h"

#define DESC_HEAD_BYTES 24u

/* Read exactly n bytes at off unless the file ends first; returns the byte
 * count read, or -1 on an I/O error. */
static int64_t read_at(int fd, void *buf, size_t n, uint64_t off) {
    size_t got = 0;
    while (got < n) {
        ssize_t r = pread(fd, (uint8_t *)buf + got, n - got, (off_t)(off + got));
        if (r < 0) {
            if (errno == EINTR) continue;
            return -1;
        }
        if (r == 0) break;
        got += (size_t)r;
    }
    return (int64_t)got;
}

static int pack_fail(Fh3Pack *p, int code) {
    fh3_pack_close(p);
    return code;
}

int fh3_pack_open(const char *path, Fh3Pack *p) {
    if (!path || !p) return FH3_ERR;
    memset(p, 0, sizeof(*p));
    p->file.fd = open(path, O_RDONLY | O_CLOEXEC);
    if (p->file.fd < 0) return FH3_E_IO;
    struct stat st;
    if (fstat(p->file.fd, &st) != 0) return pack_fail(p, FH3_E_IO);
    p->file.size = (uint64_t)st.st_size;
    if (p->file.size < sizeof(Fh3PackHeader)) return pack_fail(p, FH3_E_TRUNCATED);
    if (read_at(p->file.fd, &p->header, sizeof(p->header), 0) != (int64_t)sizeof(p->header))
        return pack_fail(p, FH3_E_IO);

    const Fh3PackHeader *h = &p->header;
    if (h->magic != FH3_PACK_MAGIC) return pack_fail(p, FH3_E_BAD_MAGIC);
    if (h->version != FH3_PACK_VERSION) return pack_fail(p, FH3_E_BAD_VERSION);
    if (h->layer_alignment != FH3_PACK_ALIGNMENT || h->num_layers == 0) return pack_fail(p, FH3_E_INVALID);
    const uint64_t stride = h->index_bytes / h->num_layers;
    if (stride < DESC_HEAD_BYTES || h->index_offset > p->file.size ||
        h->index_bytes > p->file.size - h->index_offset)
        return pack_fail(p, FH3_E_TRUNCATED);

    p->layers = (Fh3PackLayerDesc *)calloc(h->num_layers, sizeof(Fh3PackLayerDesc));
    if (!p->layers) return pack_fail(p, FH3_E_NOMEM);

    /* Descriptors on disk may be shorter (fewer tensors) or longer than the
     * in-memory struct; read what both hold. */
    const size_t take = stride < sizeof(Fh3PackLayerDesc) ? (size_t)stride : sizeof(Fh3PackLayerDesc);
    const uint32_t room = (uint32_t)((take - DESC_HEAD_BYTES) / sizeof(Fh3PackTensorDesc));
    for (uint32_t L = 0; L < h->num_layers; L++) {
        Fh3PackLayerDesc *ld = &p->layers[L];
        if (read_at(p->file.fd, ld, take, h->index_offset + (uint64_t)L * stride) != (int64_t)take)
            return pack_fail(p, FH3_E_IO);
        /* tensors beyond what the descriptor holds stay zero */
        uint32_t nt = ld->n_tensors < room ? ld->n_tensors : room;
        if (nt > FH3_PACK_MAX_TENSORS_PER_LAYER) nt = FH3_PACK_MAX_TENSORS_PER_LAYER;
        memset(&ld->tensors[nt], 0, (FH3_PACK_MAX_TENSORS_PER_LAYER - nt) * sizeof(Fh3PackTensorDesc));
    }
    p->num_layers = (int)h->num_layers;

    /* Map the file for callers that want views without a copy (optional). */
    void *m = mmap(NULL, (size_t)p->file.size, PROT_READ, MAP_SHARED, p->file.fd, 0);
    if (m != MAP_FAILED) {
        p->mapped_base = (const uint8_t *)m;
        p->mapped_size = (size_t)p->file.size;
    }
    return FH3_OK;
}

void fh3_pack_close(Fh3Pack *p) {
    if (!p) return;
    if (p->mapped_base) munmap((void *)p->mapped_base, p->mapped_size);
    p->mapped_base = NULL;
    p->mapped_size = 0;
    free(p->layers);
    p->layers = NULL;
    if (p->file.fd >= 0) close(p->file.fd);
    p->file.fd = -1;
    p->num_layers = 0;
}

static Fh3W view_of(const Fh3PackTensorDesc *d, const uint8_t *base) {
    Fh3W w;
    w.type = (int)d->type;
    w.in = d->in_dim;
    w.out = d->out_dim;
    w.data = base + d->offset_in_layer;
    return w;
}

Fh3LayerView fh3_pack_layer(const Fh3Pack *p, int L, const uint8_t *base) {
    Fh3LayerView v;
    memset(&v, 0, sizeof(v));
    if (!p || !p->layers || L < 0 || L >= p->num_layers) return v;
    const Fh3PackLayerDesc *ld = &p->layers[L];
    if (!base) {
        if (!p->mapped_base || ld->file_offset > p->mapped_size ||
            ld->size_bytes > p->mapped_size - ld->file_offset)
            return v;
        base = p->mapped_base + ld->file_offset;
    }
    /* Fh3LayerView lists its nine weights in the pack's run order. */
    Fh3W *slots[FH3_PACK_TENSORS_PER_LAYER] = {&v.qkv, &v.gate_compress, &v.out, &v.fc1, &v.fc2,
                                               &v.norm1, &v.norm2, &v.q_norm, &v.k_norm};
    for (unsigned i = 0; i < FH3_PACK_TENSORS_PER_LAYER; i++) *slots[i] = view_of(&ld->tensors[i], base);
    return v;
}
