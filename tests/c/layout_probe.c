/*
 * layout_probe.c -- prints the size and field offsets of the structs that
 * callers hold by value (Fh3File, Fh3Pack, Fh3Trunk, Fh3TrunkStats,
 * Fh3PackLayerDesc, Fh3W, Fh3LayerView).  Compiled once against this
 * library's headers and once, with -DFH3_PROBE_REFERENCE, against the
 * reference's (include/fh3/fh3.h and src/io/fh3_trunk.h there); the two
 * outputs must be identical for the library to take the reference's structs
 * by pointer.
 */
#include <stddef.h>
#include <stdio.h>

#ifdef FH3_PROBE_REFERENCE
#include "fh3/fh3.h"
#include "io/fh3_trunk.h"
#else
#include "fh3/fh3.h"
#include "fh3/fh3_trunk.h"
#endif

#define SIZE(T) printf("sizeof %s %zu\n", #T, sizeof(T))
#define FIELD(T, f) printf("offsetof %s.%s %zu\n", #T, #f, offsetof(T, f))

int main(void) {
    SIZE(Fh3W);
    FIELD(Fh3W, type); FIELD(Fh3W, in); FIELD(Fh3W, out); FIELD(Fh3W, data);
    SIZE(Fh3LayerView);
    FIELD(Fh3LayerView, qkv); FIELD(Fh3LayerView, gate_compress); FIELD(Fh3LayerView, out);
    FIELD(Fh3LayerView, fc1); FIELD(Fh3LayerView, fc2); FIELD(Fh3LayerView, norm1);
    FIELD(Fh3LayerView, norm2); FIELD(Fh3LayerView, q_norm); FIELD(Fh3LayerView, k_norm);
    SIZE(Fh3TrunkStats);
    FIELD(Fh3TrunkStats, hits); FIELD(Fh3TrunkStats, misses); FIELD(Fh3TrunkStats, bytes_read);
    FIELD(Fh3TrunkStats, read_s); FIELD(Fh3TrunkStats, wait_s);
    SIZE(Fh3PackTensorDesc); SIZE(Fh3PackLayerDesc); SIZE(Fh3PackHeader);
    FIELD(Fh3PackLayerDesc, file_offset); FIELD(Fh3PackLayerDesc, size_bytes);
    FIELD(Fh3PackLayerDesc, n_tensors); FIELD(Fh3PackLayerDesc, tensors);
    SIZE(Fh3File);
    FIELD(Fh3File, fd); FIELD(Fh3File, size); FIELD(Fh3File, is_direct);
    SIZE(Fh3Pack);
    FIELD(Fh3Pack, file); FIELD(Fh3Pack, header); FIELD(Fh3Pack, num_layers); FIELD(Fh3Pack, layers);
    FIELD(Fh3Pack, mapped_base); FIELD(Fh3Pack, mapped_size);
    SIZE(Fh3Trunk);
    FIELD(Fh3Trunk, pack); FIELD(Fh3Trunk, direct_file); FIELD(Fh3Trunk, num_layers);
    FIELD(Fh3Trunk, budget_bytes); FIELD(Fh3Trunk, npin); FIELD(Fh3Trunk, slot_size);
    FIELD(Fh3Trunk, pinned_layers); FIELD(Fh3Trunk, ring_buf); FIELD(Fh3Trunk, ring_layer);
    FIELD(Fh3Trunk, active_slot); FIELD(Fh3Trunk, prefetch_layer); FIELD(Fh3Trunk, prefetch_slot);
    FIELD(Fh3Trunk, prefetch_in_flight); FIELD(Fh3Trunk, prefetch_start_time);
    FIELD(Fh3Trunk, prefetch_io_time); FIELD(Fh3Trunk, thread); FIELD(Fh3Trunk, mutex);
    FIELD(Fh3Trunk, start_cond); FIELD(Fh3Trunk, done_cond); FIELD(Fh3Trunk, worker_has_work);
    FIELD(Fh3Trunk, worker_done); FIELD(Fh3Trunk, thread_created); FIELD(Fh3Trunk, worker_stop);
    FIELD(Fh3Trunk, worker_req_layer); FIELD(Fh3Trunk, worker_req_slot);
    FIELD(Fh3Trunk, worker_read_bytes); FIELD(Fh3Trunk, stats);
    return 0;
}
