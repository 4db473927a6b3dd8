// handoff.cpp -- same-GPU state hand-off between processes: exported device
// allocations for an old rank's packed state and their mapping in a new
// rank (C ABI in include/suika_handoff.h).  Host code only.
//
// Replaces Suika/utils.py:325-406 (interactive_IPC_state_dict_send / _recv),
// which moves the state one CUDA-IPC tensor per queue message and clones each
// on the receiving side.  Here the old rank packs its whole state into a few
// allocations with one gather launch, and a new rank maps them once and
// gathers its shards from them directly.

#include <hip/hip_runtime.h>

#include <cstring>

#include "suika_handoff.h"
#include "sr_internal.h"

using sr_internal::fail;

static_assert(sizeof(hipIpcMemHandle_t) == sizeof(sr_ipc_handle), "sr_ipc_handle holds a HIP IPC handle");

extern "C" {

int sr_handoff_alloc(uint64_t bytes, void** out_ptr, sr_ipc_handle* out_handle) {
  if (out_ptr == nullptr || out_handle == nullptr) return fail(SR_EINVAL, "sr_handoff_alloc: null argument");
  *out_ptr = nullptr;
  if (bytes == 0 || bytes > SR_HANDOFF_MAX_BYTES)
    return fail(SR_EINVAL, "sr_handoff_alloc: %llu bytes outside 1..%llu", (unsigned long long)bytes,
                (unsigned long long)SR_HANDOFF_MAX_BYTES);
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess)
    return fail(e == hipErrorOutOfMemory ? SR_ENOMEM : SR_EHIP, "sr_handoff_alloc: hipMalloc(%llu): %s",
                (unsigned long long)bytes, hipGetErrorString(e));
  hipIpcMemHandle_t h;
  e = hipIpcGetMemHandle(&h, p);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return fail(SR_EHIP, "sr_handoff_alloc: hipIpcGetMemHandle: %s", hipGetErrorString(e));
  }
  std::memcpy(out_handle->bytes, &h, sizeof h);
  *out_ptr = p;
  return SR_OK;
}

int sr_handoff_free(void* ptr) {
  if (ptr == nullptr) return fail(SR_EINVAL, "sr_handoff_free: null pointer");
  const hipError_t e = hipFree(ptr);
  if (e != hipSuccess) return fail(SR_EHIP, "sr_handoff_free: hipFree: %s", hipGetErrorString(e));
  return SR_OK;
}

int sr_handoff_open(const sr_ipc_handle* handle, void** out_ptr) {
  if (handle == nullptr || out_ptr == nullptr) return fail(SR_EINVAL, "sr_handoff_open: null argument");
  *out_ptr = nullptr;
  hipIpcMemHandle_t h;
  std::memcpy(&h, handle->bytes, sizeof h);
  void* p = nullptr;
  const hipError_t e = hipIpcOpenMemHandle(&p, h, hipIpcMemLazyEnablePeerAccess);
  if (e != hipSuccess) return fail(SR_EHIP, "sr_handoff_open: hipIpcOpenMemHandle: %s", hipGetErrorString(e));
  *out_ptr = p;
  return SR_OK;
}

int sr_handoff_close(void* ptr) {
  if (ptr == nullptr) return fail(SR_EINVAL, "sr_handoff_close: null pointer");
  const hipError_t e = hipIpcCloseMemHandle(ptr);
  if (e != hipSuccess) return fail(SR_EHIP, "sr_handoff_close: hipIpcCloseMemHandle: %s", hipGetErrorString(e));
  return SR_OK;
}

}  // extern "C"
