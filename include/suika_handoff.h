/*
 * suika_handoff.h -- same-GPU state hand-off between processes
 * (libsuika_reshard.so).
 *
 * A live migration replaces a job's training processes.  The processes of
 * the old plan and of the new plan run side by side, and on one GPU they
 * share its HBM.  An old rank packs its merged model and optimizer state
 * into a few device allocations of its own (sr_gather from the state tensors
 * into them), exports them, and passes the handles over its control channel.
 * A new rank opens the allocations of the old ranks it reads from and
 * gathers its new shards straight out of them.  The old rank frees them once
 * every new rank is done.  Together these are the pack -> per-peer buffer
 * -> unpack of the reshard, with the exchange replaced by an IPC mapping.
 *
 * Reference interface replaced (paths relative to the Suika repository):
 *   - Suika/utils.py:325-387  interactive_IPC_state_dict_send: one CUDA-IPC
 *       tensor per queue message, an acknowledgement each, the sender's
 *       tensor freed per acknowledgement
 *   - Suika/utils.py:389-406  interactive_IPC_state_dict_recv: every
 *       received tensor cloned into the receiver's memory
 *   (callers: Suika/migration.py:1430-1436, 1472-1478, 1618-1623, 1683-1688)
 *
 * Conventions
 *   - Every allocation is a separate hipMalloc on the current device, below
 *     SR_HANDOFF_MAX_BYTES: IPC mappings of larger allocations are avoided.
 *   - Handles are 64 opaque bytes (the HIP IPC memory handle) that another
 *     process of the same machine passes to sr_handoff_open on the same GPU.
 *   - Status codes are the sr_status values of suika_reshard.h;
 *     sr_last_error() describes the last failure.
 */
#ifndef SUIKA_HANDOFF_H
#define SUIKA_HANDOFF_H

#include <stdint.h>

#include "suika_reshard.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Largest hand-off allocation: 2 GiB - 1 MiB. */
#define SR_HANDOFF_MAX_BYTES ((uint64_t)2146435072)

typedef struct sr_ipc_handle {
  unsigned char bytes[64];
} sr_ipc_handle;

/*
 * Allocate `bytes` (1 .. SR_HANDOFF_MAX_BYTES) of device memory on the current
 * device and export it: *out_ptr is its address in this process, *out_handle
 * what another process opens.  Replaces the per-tensor CUDA-IPC export of
 * interactive_IPC_state_dict_send (Suika/utils.py:325-387).
 */
int sr_handoff_alloc(uint64_t bytes, void** out_ptr, sr_ipc_handle* out_handle);

/* Free an allocation of sr_handoff_alloc (after every opener has closed it). */
int sr_handoff_free(void* ptr);

/*
 * Map another process's hand-off allocation into this process (same GPU);
 * *out_ptr is its address here.  Replaces the receive side of
 * interactive_IPC_state_dict_recv (Suika/utils.py:389-406), without its
 * per-tensor clone: kernels read the mapped memory directly.
 */
int sr_handoff_open(const sr_ipc_handle* handle, void** out_ptr);

/* Unmap an allocation opened by sr_handoff_open. */
int sr_handoff_close(void* ptr);

#ifdef __cplusplus
}
#endif

#endif /* SUIKA_HANDOFF_H */
