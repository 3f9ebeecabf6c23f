/*
 * fh3_hip_internal.h -- small C-ABI over the HIP runtime used by the C99 host
 * code of libfh3hip.so (the trunk streamer), so that C files need no HIP
 * headers.  Streams and events are opaque pointers (hipStream_t / hipEvent_t);
 * a NULL stream means the library's compute stream.  Not part of the public
 * interface.
 */
#ifndef FH3_HIP_INTERNAL_H
#define FH3_HIP_INTERNAL_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

int fh3i_set_error(int code, const char *msg);
int fh3i_host_alloc(void **p, size_t bytes);   /* pinned, page aligned */
int fh3i_host_free(void *p);
int fh3i_stream_create(void **st);             /* default priority, non-blocking */
int fh3i_stream_destroy(void *st);
int fh3i_stream_sync(void *st);
int fh3i_copy_async(void *dst, const void *src, size_t bytes, void *st);
int fh3i_event_create(void **ev);
int fh3i_event_destroy(void *ev);
int fh3i_event_record(void *ev, void *st);
int fh3i_stream_wait(void *st, void *ev);
int fh3i_event_sync(void *ev);

#ifdef __cplusplus
}
#endif

#endif
