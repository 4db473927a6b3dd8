// sr_internal.h -- what the library's translation units share (not part of
// the C ABI): the thread-local error message behind sr_last_error() and a
// read-only view of a plan's host tables for the host-side staging code.
#ifndef SR_INTERNAL_H
#define SR_INTERNAL_H

#include <cstddef>
#include <cstdint>

#include "suika_reshard.h"

namespace sr_internal {

// Record a printf-style message for sr_last_error() and return `code`.
__attribute__((visibility("hidden"), format(printf, 2, 3)))
int fail(int code, const char* fmt, ...);

// The message of the last failure on this thread.
__attribute__((visibility("hidden"))) const char* last_error();

// Bytes per element of an sr_dtype (0 for an unknown code).
__attribute__((visibility("hidden"))) int dtype_size(int32_t dt);

// A plan's validated host tables, as sr_plan_create left them.
struct PlanView {
  const sr_tensor* src;
  size_t n_src;
  const sr_piece* pieces;
  size_t n_pieces;
  const uint64_t* piece_offset;   // byte offset in its peer buffer; UINT64_MAX for ZERO
  const uint64_t* peer_bytes;     // per peer
  int32_t n_peers;
  // the non-ZERO pieces of peer q, in piece order (so in ascending buffer
  // offset): peer_list[peer_begin[q] .. peer_begin[q + 1])
  const uint32_t* peer_begin;
  const uint32_t* peer_list;
};

__attribute__((visibility("hidden"))) PlanView plan_view(const sr_plan* plan);

}  // namespace sr_internal

#endif  // SR_INTERNAL_H
