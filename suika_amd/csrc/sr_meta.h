// sr_meta.h -- TensorMeta arithmetic shared by the scheduler and the lowering
// (not part of the C ABI).  Restates the accessors of the reference's
// TensorMeta (paths relative to the Suika repository):
//   Suika/migration.py:62-98   numel / volumn / actual_shape
//   Suika/migration.py:103-118 scale_to_tp (a View with another tp meta)
// and the vocab_pad extension (padded rows, the rows a shard holds).
#ifndef SR_META_H
#define SR_META_H

#include <algorithm>
#include <cstdint>

#include "sr_internal.h"
#include "suika_planner.h"
#include "suika_reshard.h"

namespace sr_internal {

// A TensorMeta: a table row, or a piece derived from one (another tp meta
// from scale_to_tp, or a row interval of a vocab_pad shard).
struct View {
  const sr_meta* m;
  int64_t tp_index;
  int64_t tp_deg;    // 0: not tensor-parallel
  int64_t row0;      // -1: no row interval
  int64_t row1;
  bool whole;        // the table row itself (scale_to_tp returned [self])
};

inline View view_of(const sr_meta& m) { return View{&m, m.tp_index, m.tp_deg, m.row0, m.row1, true}; }

inline int64_t deg_of(const View& v) { return v.tp_deg > 0 ? v.tp_deg : 1; }

inline bool mul(int64_t a, int64_t b, int64_t* out) { return !__builtin_mul_overflow(a, b, out); }

// Python's d % n for the split dim (n > 0).
inline int64_t norm_dim(int64_t d, int64_t n) { return ((d % n) + n) % n; }

// Padded vocabulary rows at the view's degree: a multiple of pad_multiple * deg.
inline bool padded_rows(const View& v, int64_t* out) {
  int64_t step;
  if (!mul(v.m->kind_args[0], deg_of(v), &step) || step <= 0) return false;
  const int64_t V = v.m->shape[0];
  return mul((V + step - 1) / step, step, out);
}

// Global rows of a vocab_pad shard that hold data (TensorMeta.valid_rows).
inline bool valid_rows(const View& v, int64_t* lo, int64_t* hi) {
  if (v.row0 >= 0) {
    *lo = v.row0;
    *hi = v.row1;
    return true;
  }
  int64_t padded;
  if (!padded_rows(v, &padded)) return false;
  const int64_t n = padded / deg_of(v);
  int64_t end;
  if (!mul(v.tp_index, n, lo) || __builtin_add_overflow(*lo, n, &end)) return false;
  *hi = std::max(*lo, std::min(end, v.m->shape[0]));
  return true;
}

// actual_shape (migration.py:92-98): the shard as stored.
inline bool actual_shape(const View& v, int64_t dims[SR_MAX_DIMS]) {
  const sr_meta& m = *v.m;
  for (int64_t d = 0; d < m.ndim; ++d) dims[d] = m.shape[d];
  if (v.row0 >= 0) {
    dims[0] = v.row1 - v.row0;
  } else if (v.tp_deg > 0) {
    if (m.kind == SR_KIND_VOCAB_PAD) {
      int64_t padded;
      if (!padded_rows(v, &padded)) return false;
      dims[0] = padded / v.tp_deg;
    } else {
      dims[norm_dim(m.slice_dim, m.ndim)] /= v.tp_deg;
    }
  }
  return true;
}

// numel (migration.py:62-64 and the extensions): chunk shards count
// prod(shape) / tp_deg, everything else its actual shape.
inline bool numel(const View& v, int64_t* out) {
  const sr_meta& m = *v.m;
  const bool plain_chunk = m.kind == SR_KIND_CHUNK && v.row0 < 0;
  int64_t dims[SR_MAX_DIMS];
  if (plain_chunk) {
    for (int64_t d = 0; d < m.ndim; ++d) dims[d] = m.shape[d];
  } else if (!actual_shape(v, dims)) {
    return false;
  }
  int64_t n = 1;
  for (int64_t d = 0; d < m.ndim; ++d)
    if (!mul(n, dims[d], &n)) return false;
  *out = plain_chunk ? n / deg_of(v) : n;
  return true;
}

inline bool volume(const View& v, int64_t* out) {
  int64_t n;
  return numel(v, &n) && mul(n, v.m->itemsize, out);
}

// A well-formed meta row (what TensorMeta's constructor guarantees), with a
// name id in [0, n_names) unless n_names < 0.
inline int check_meta(const sr_meta& m, int64_t n_names, const char* table, int64_t i) {
  if (m.name < 0 || (n_names >= 0 && m.name >= n_names))
    return fail(SR_EINVAL, "%s[%lld]: name id %lld outside [0, %lld)", table, (long long)i,
                (long long)m.name, (long long)n_names);
  if (m.ndim < 0 || m.ndim > SR_MAX_DIMS)
    return fail(SR_EINVAL, "#%lld: ndim %lld outside [0, %d]", (long long)m.name, (long long)m.ndim,
                SR_MAX_DIMS);
  if (m.itemsize < 1)
    return fail(SR_EINVAL, "#%lld: itemsize %lld", (long long)m.name, (long long)m.itemsize);
  for (int64_t d = 0; d < m.ndim; ++d)
    if (m.shape[d] < 0) return fail(SR_EINVAL, "#%lld: negative dim", (long long)m.name);
  if (m.kind < SR_KIND_CHUNK || m.kind > SR_KIND_QKV_HEADS)
    return fail(SR_EINVAL, "#%lld: unknown shard kind %lld", (long long)m.name, (long long)m.kind);
  if (m.tp_deg < 0 || m.tp_deg > SR_MAX_TP_DEG || (m.tp_deg > 0 && m.tp_index < 0))
    return fail(SR_EINVAL, "#%lld: tp meta (%lld, %lld, %lld) (degree at most %d)", (long long)m.name,
                (long long)m.slice_dim, (long long)m.tp_index, (long long)m.tp_deg, SR_MAX_TP_DEG);
  if (m.tp_deg > 0 && (m.ndim == 0 || m.slice_dim < -m.ndim || m.slice_dim >= m.ndim))
    return fail(SR_EINVAL, "#%lld: slice_dim %lld of a %lld-D tensor", (long long)m.name,
                (long long)m.slice_dim, (long long)m.ndim);
  if (m.kind == SR_KIND_VOCAB_PAD &&
      (m.tp_deg == 0 || (m.slice_dim != 0 && m.slice_dim != -m.ndim) || m.kind_args[0] < 1))
    return fail(SR_EINVAL, "#%lld: vocab_pad is a TP layout sharded along dim 0 with a "
                "positive pad multiple", (long long)m.name);
  if (m.kind == SR_KIND_QKV_HEADS) {
    // rows == (n_q + 2 n_kv) * head_dim, as TensorMeta's constructor asserts
    int64_t heads, rows;
    const int64_t n_q = m.kind_args[0], n_kv = m.kind_args[1], hd = m.kind_args[2];
    if (m.ndim < 1 || n_q < 1 || n_kv < 1 || hd < 1 || !mul(n_kv, 2, &heads) ||
        __builtin_add_overflow(heads, n_q, &heads) || !mul(heads, hd, &rows) || rows != m.shape[0])
      return fail(SR_EINVAL, "#%lld: qkv_heads rows %lld != (n_q + 2 n_kv) * head_dim", (long long)m.name,
                  (long long)(m.ndim ? m.shape[0] : 0));
  }
  if ((m.row0 < 0) != (m.row1 < 0) || (m.row0 >= 0 && m.row1 < m.row0))
    return fail(SR_EINVAL, "#%lld: row interval [%lld, %lld)", (long long)m.name, (long long)m.row0,
                (long long)m.row1);
  return SR_OK;
}

}  // namespace sr_internal

#endif  // SR_META_H
