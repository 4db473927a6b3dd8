// sr_internal.h -- what the library's translation units share (not part of
// the C ABI): the thread-local error message behind sr_last_error().
#ifndef SR_INTERNAL_H
#define SR_INTERNAL_H

namespace sr_internal {

// Record a printf-style message for sr_last_error() and return `code`.
__attribute__((visibility("hidden"), format(printf, 2, 3)))
int fail(int code, const char* fmt, ...);

// The message of the last failure on this thread.
__attribute__((visibility("hidden"))) const char* last_error();

}  // namespace sr_internal

#endif  // SR_INTERNAL_H
