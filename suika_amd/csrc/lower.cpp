// lower.cpp -- one destination rank's transfer ops as the engine's region
// moves (sr_lower, include/suika_planner.h).
//
// Reference behaviour reproduced (paths relative to the Suika repository):
//   Suika/migration.py:290-312  get_send_tensor: chunk(n, dim)[k].contiguous()
//                               and its shape / slice-dim checks (293-294)
//   Suika/migration.py:531-541  cat(pieces, dim=slice_dim) / clone()
//
// Every tensor is a row-major 2-D matrix [R, C]: split along dim 0 (or not
// split), R = shape[0] and C = prod(shape[1:]); split along the last dim,
// R = prod(shape[:-1]) and C = shape[-1].  A shard (or a piece of one) is a
// list of bands -- rectangles of the global matrix with their origin in the
// shard's local matrix -- plus, for vocab_pad, the box of padding rows.  The
// bands of a piece intersected with those of its source shard and of its
// destination shard are the region moves: for the chunk layout exactly
// chunk(n, dim)[k] on the sending side and cat in ascending piece order on
// the receiving side; for qkv_heads three bands per shard (its Q, K and V
// head blocks); for vocab_pad a row interval.

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <new>
#include <vector>

#include "sr_internal.h"
#include "sr_meta.h"
#include "suika_planner.h"
#include "suika_reshard.h"

namespace {

using namespace sr_internal;

struct Seg {
  int64_t g_row, g_col;   // origin in the global matrix
  int64_t l_row, l_col;   // origin in the shard's local matrix
  int64_t rows, cols;
};

struct Box {
  int64_t row, col, rows, cols;
};

struct Region {
  int64_t rows, cols, src_row, src_col, dst_row, dst_col;
};

struct Lowering : sr_lowering {
  std::vector<sr_tensor> src_v, dst_v;
  std::vector<sr_slot_key> src_key_v, dst_key_v, empty_v;
  std::vector<sr_piece> piece_v;
  std::vector<int64_t> peer_v;
};

long long ll(int64_t v) { return (long long)v; }

// 0: dim 0 is split; 1: the last dim is split; -1: not split.
int split_axis(const View& v, int* axis) {
  if (v.tp_deg == 0) {
    *axis = -1;
    return SR_OK;
  }
  const int64_t nd = v.m->ndim;
  const int64_t d = norm_dim(v.m->slice_dim, nd);
  if (d == 0) {
    *axis = 0;
  } else if (d == nd - 1) {
    *axis = 1;
  } else {
    return fail(SR_EINVAL, "#%lld: slice_dim %lld of a %lld-D tensor is neither the first nor the last dim",
                ll(v.m->name), ll(v.m->slice_dim), ll(nd));
  }
  return SR_OK;
}

// [R, C] of a shape in a view (a 0-D tensor is [1, 1]).
bool matrix(const int64_t* dims, int64_t nd, int view, int64_t* R, int64_t* C) {
  *R = 1;
  *C = 1;
  if (nd == 0) return true;
  for (int64_t d = 0; d < nd; ++d) {
    const bool to_rows = view == 1 ? d < nd - 1 : d == 0;
    if (!mul(to_rows ? *R : *C, dims[d], to_rows ? R : C)) return false;
  }
  return true;
}

int split(int64_t n, int64_t deg, const View& v, const char* what, int64_t* out) {
  if (n % deg != 0)
    return fail(SR_EINVAL, "#%lld %s: %lld is not divisible by tp degree %lld", ll(v.m->name), what, ll(n),
                ll(deg));
  *out = n / deg;
  return SR_OK;
}

// Bands of global data a shard (or piece) holds in `view`, and its pad boxes.
int segments(const View& v, int view, std::vector<Seg>* segs, std::vector<Box>* pads) {
  segs->clear();
  pads->clear();
  const sr_meta& m = *v.m;
  int64_t R, C;
  if (!matrix(m.shape, m.ndim, view, &R, &C)) return fail(SR_EINVAL, "#%lld: size overflows", ll(m.name));
  if (v.row0 >= 0) {   // a vocab piece: a row interval
    segs->push_back(Seg{v.row0, 0, 0, 0, v.row1 - v.row0, C});
    return SR_OK;
  }
  int axis;
  int rc = split_axis(v, &axis);
  if (rc != SR_OK) return rc;
  if (axis < 0) {
    segs->push_back(Seg{0, 0, 0, 0, R, C});
    return SR_OK;
  }
  if (axis != view) return fail(SR_EINVAL, "#%lld: split axis %d in view %d", ll(m.name), axis, view);
  const int64_t deg = v.tp_deg, idx = v.tp_index;
  if (idx < 0 || idx >= deg)
    return fail(SR_EINVAL, "#%lld: tp_index %lld outside degree %lld", ll(m.name), ll(idx), ll(deg));
  if (m.kind == SR_KIND_VOCAB_PAD) {
    int64_t padded, lo, hi;
    if (!padded_rows(v, &padded) || !valid_rows(v, &lo, &hi))
      return fail(SR_EINVAL, "#%lld: vocabulary rows overflow", ll(m.name));
    const int64_t n = padded / deg;
    if (hi > lo) segs->push_back(Seg{lo, 0, 0, 0, hi - lo, C});
    if (hi - lo < n) pads->push_back(Box{hi - lo, 0, n - (hi - lo), C});
    return SR_OK;
  }
  if (m.kind == SR_KIND_QKV_HEADS) {
    if (axis != 0) return fail(SR_EINVAL, "#%lld: qkv_heads splits rows", ll(m.name));
    const int64_t n_q = m.kind_args[0], n_kv = m.kind_args[1], hd = m.kind_args[2];
    int64_t q, kv;
    if ((rc = split(n_q, deg, v, "q heads", &q)) != SR_OK) return rc;
    if ((rc = split(n_kv, deg, v, "kv heads", &kv)) != SR_OK) return rc;
    q *= hd;
    kv *= hd;
    segs->push_back(Seg{idx * q, 0, 0, 0, q, C});
    segs->push_back(Seg{n_q * hd + idx * kv, 0, q, 0, kv, C});
    segs->push_back(Seg{(n_q + n_kv) * hd + idx * kv, 0, q + kv, 0, kv, C});
    return SR_OK;
  }
  int64_t n;
  if (axis == 0) {
    if ((rc = split(R, deg, v, "rows", &n)) != SR_OK) return rc;
    segs->push_back(Seg{idx * n, 0, 0, 0, n, C});
  } else {
    if ((rc = split(C, deg, v, "cols", &n)) != SR_OK) return rc;
    segs->push_back(Seg{0, idx * n, 0, 0, R, n});
  }
  return SR_OK;
}

bool intersect(const Seg& a, const Seg& b, int64_t* r0, int64_t* r1, int64_t* c0, int64_t* c1) {
  *r0 = std::max(a.g_row, b.g_row);
  *r1 = std::min(a.g_row + a.rows, b.g_row + b.rows);
  *c0 = std::max(a.g_col, b.g_col);
  *c1 = std::min(a.g_col + a.cols, b.g_col + b.cols);
  return *r1 > *r0 && *c1 > *c0;
}

struct Scratch {
  std::vector<Seg> piece, src, dst;
  std::vector<Box> pads;
};

// Name id -> dense group index, for at most `n` ids: open addressing in one
// allocation (a node-based map costs an allocation per name).
class IdTable {
 public:
  explicit IdTable(size_t n) {
    size_t cap = 16;
    while (cap < 2 * n) cap *= 2;
    slots_.assign(cap, Slot{0, -1});
    mask_ = cap - 1;
  }
  // the value stored for `id`, or `value` after storing it
  int64_t find_or_add(int64_t id, int64_t value) {
    uint64_t h = uint64_t(id) * 0x9E3779B97F4A7C15ull;
    for (size_t i = size_t(h >> 32) & mask_;; i = (i + 1) & mask_) {
      Slot& s = slots_[i];
      if (s.value < 0) {
        s = Slot{id, value};
        return value;
      }
      if (s.id == id) return s.value;
    }
  }

 private:
  struct Slot {
    int64_t id, value;   // value -1: empty
  };
  std::vector<Slot> slots_;
  size_t mask_;
};

// One tensor's ops: a range of op indices.
struct Span {
  const int64_t *b, *e;
  const int64_t* begin() const { return b; }
  const int64_t* end() const { return e; }
  int64_t operator[](size_t i) const { return b[i]; }
};

// Region moves of one op, source local -> destination local.
int lower_op(const sr_op& op, const sr_meta* metas, const View& shard, int view, Scratch& w,
             std::vector<Region>* out) {
  out->clear();
  const sr_meta& sm = metas[op.src_meta];
  const View src = view_of(sm);
  if (sm.kind != shard.m->kind)
    return fail(SR_EINVAL, "#%lld: shard kind %lld -> %lld", ll(op.name), ll(sm.kind), ll(shard.m->kind));
  bool same = sm.ndim == shard.m->ndim;
  for (int64_t d = 0; same && d < sm.ndim; ++d) same = sm.shape[d] == shard.m->shape[d];
  if (!same) return fail(SR_EINVAL, "#%lld: global shape differs between source and destination", ll(op.name));
  if (src.tp_deg > 0 && shard.tp_deg > 0) {
    int a, b, rc;
    if ((rc = split_axis(src, &a)) != SR_OK || (rc = split_axis(shard, &b)) != SR_OK) return rc;
    if (a != b)
      return fail(SR_EINVAL, "slice dim mismatch btw src %lld and dst %lld", ll(sm.slice_dim),
                  ll(shard.m->slice_dim));
  }
  const View piece = op.piece_tp_deg == 0
                         ? shard
                         : View{shard.m, op.piece_tp_index, op.piece_tp_deg, op.row0, op.row1, false};
  int rc;
  if ((rc = segments(piece, view, &w.piece, &w.pads)) != SR_OK) return rc;
  if ((rc = segments(src, view, &w.src, &w.pads)) != SR_OK) return rc;
  if ((rc = segments(shard, view, &w.dst, &w.pads)) != SR_OK) return rc;
  int64_t want = 0, got = 0;
  for (const Seg& pb : w.piece) {
    want += pb.rows * pb.cols;
    for (const Seg& s : w.src) {
      int64_t r0, r1, c0, c1;
      if (!intersect(pb, s, &r0, &r1, &c0, &c1)) continue;
      const Seg part{r0, c0, 0, 0, r1 - r0, c1 - c0};
      for (const Seg& d : w.dst) {
        int64_t jr0, jr1, jc0, jc1;
        if (!intersect(part, d, &jr0, &jr1, &jc0, &jc1)) continue;
        out->push_back(Region{jr1 - jr0, jc1 - jc0, s.l_row + jr0 - s.g_row, s.l_col + jc0 - s.g_col,
                              d.l_row + jr0 - d.g_row, d.l_col + jc0 - d.g_col});
        got += (jr1 - jr0) * (jc1 - jc0);
      }
    }
  }
  if (got != want)
    return fail(SR_EINVAL, "#%lld: source rank %lld holds %lld of the %lld elements of its piece", ll(op.name),
                ll(op.src_rank), ll(got), ll(want));
  return SR_OK;
}

sr_slot_key slot_key(int64_t op, int64_t field, int64_t recast, int64_t dtype, int64_t nd, const int64_t* dims) {
  sr_slot_key k;
  std::memset(&k, 0, sizeof(k));
  k.op = op;
  k.field = field;
  k.recast = recast;
  k.dtype = dtype;
  k.ndim = nd;
  for (int64_t d = 0; d < nd; ++d) k.shape[d] = dims[d];
  return k;
}

void shape_str(const int64_t* dims, int64_t nd, char* buf, size_t n) {
  size_t at = 0;
  at += snprintf(buf + at, n - at, "(");
  for (int64_t d = 0; d < nd && at < n; ++d) at += snprintf(buf + at, n - at, d ? ", %lld" : "%lld", ll(dims[d]));
  if (at < n) snprintf(buf + at, n - at, ")");
}

int lower(const sr_meta* metas, int64_t n_metas, const sr_op* ops, int64_t n_ops, const sr_src_spec* specs,
          int64_t n_fields, const int64_t* recast, Lowering* L) {
  if (n_metas < 0 || n_ops < 0 || n_fields < 0 || (n_metas && !metas) || (n_ops && !ops) ||
      (n_ops && n_fields && !specs) || (n_fields && !recast))
    return fail(SR_EINVAL, "sr_lower: null table or negative size");
  for (int64_t f = 0; f < n_fields; ++f)
    if (recast[f] != 0 && recast[f] != 1) return fail(SR_EINVAL, "sr_lower: recast[%lld] is not 0 or 1", ll(f));
  std::vector<char> checked(n_metas, 0);
  for (int64_t k = 0; k < n_ops; ++k) {
    const sr_op& op = ops[k];
    for (int64_t row : {op.src_meta, op.dst_shard}) {
      if (row < 0 || row >= n_metas)
        return fail(SR_EINVAL, "sr_lower: op %lld names meta row %lld of %lld", ll(k), ll(row), ll(n_metas));
      if (!checked[row]) {
        int rc = check_meta(metas[row], -1, "metas", row);
        if (rc != SR_OK) return rc;
        checked[row] = 1;
      }
    }
    if (op.dst_rank != ops[0].dst_rank)
      return fail(SR_EINVAL, "ops target several ranks (%lld and %lld)", ll(ops[0].dst_rank), ll(op.dst_rank));
    if (op.piece_tp_deg < 0 || op.piece_tp_deg > SR_MAX_TP_DEG || (op.piece_tp_deg > 0 && op.piece_tp_index < 0) ||
        (op.row0 < 0) != (op.row1 < 0) ||
        (op.row0 >= 0 && (op.row1 < op.row0 || op.piece_tp_deg == 0)))
      return fail(SR_EINVAL, "#%lld: malformed piece of op %lld", ll(op.name), ll(k));
    for (int64_t f = 0; f < n_fields; ++f) {
      const sr_src_spec& sp = specs[k * n_fields + f];
      if (sp.ndim < 0 || sp.ndim > SR_MAX_DIMS || sp.dtype < SR_DT_U8 || sp.dtype > SR_DT_I64)
        return fail(SR_EINVAL, "#%lld: malformed source spec of op %lld field %lld", ll(op.name), ll(k), ll(f));
    }
  }
  // peers: the source ranks, ascending
  for (int64_t k = 0; k < n_ops; ++k) L->peer_v.push_back(ops[k].src_rank);
  std::sort(L->peer_v.begin(), L->peer_v.end());
  L->peer_v.erase(std::unique(L->peer_v.begin(), L->peer_v.end()), L->peer_v.end());
  // tensors in order of first appearance, each with its ops in schedule
  // order: group g's ops are member[begin[g] .. begin[g + 1])
  std::vector<int64_t> group_of(static_cast<size_t>(n_ops)), begin, member(static_cast<size_t>(n_ops));
  {
    IdTable ids(static_cast<size_t>(n_ops));
    for (int64_t k = 0; k < n_ops; ++k) {
      const int64_t g = ids.find_or_add(ops[k].name, int64_t(begin.size()));
      if (g == int64_t(begin.size())) begin.push_back(0);
      group_of[k] = g;
      ++begin[g];
    }
    int64_t at = 0;
    for (int64_t& b : begin) {
      const int64_t n = b;
      b = at;
      at += n;
    }
    begin.push_back(at);
    std::vector<int64_t> fill(begin.begin(), begin.end() - 1);
    for (int64_t k = 0; k < n_ops; ++k) member[fill[group_of[k]]++] = k;
  }
  const int64_t n_groups = int64_t(begin.size()) - 1;
  int64_t n_recast = 0;
  for (int64_t f = 0; f < n_fields; ++f) n_recast += recast[f];
  L->dst_v.reserve(size_t(n_groups * (n_fields + n_recast)));
  L->dst_key_v.reserve(L->dst_v.capacity());
  L->src_v.reserve(size_t(n_ops * n_fields));
  L->src_key_v.reserve(L->src_v.capacity());
  L->piece_v.reserve(size_t(n_ops * n_fields));
  // a tensor's source slots by source rank (the ranks of one tensor's ops)
  std::vector<std::pair<int64_t, int32_t>> src_base;
  std::vector<int64_t> field_dtype(n_fields);
  std::vector<int32_t> dslot(n_fields), dslot2(n_fields);
  std::vector<Region> regions;
  Scratch w;
  char a[160], b[160];
  for (int64_t gi = 0; gi < n_groups; ++gi) {
    const Span g{member.data() + begin[gi], member.data() + begin[gi + 1]};
    const int64_t k0 = g[0];
    src_base.clear();
    const sr_meta& sh = metas[ops[k0].dst_shard];
    const View shard = view_of(sh);
    const int64_t name = ops[k0].name;
    // one 2-D view for the tensor: the split axis of any of its shards
    int view = -1, axis, rc;
    if ((rc = split_axis(shard, &axis)) != SR_OK) return rc;
    if (axis >= 0) view = axis;
    for (int64_t k : g) {
      if ((rc = split_axis(view_of(metas[ops[k].src_meta]), &axis)) != SR_OK) return rc;
      if (axis >= 0 && view >= 0 && axis != view)
        return fail(SR_EINVAL, "#%lld: shards split along different dims", ll(name));
      if (axis >= 0) view = axis;
    }
    if (view < 0) view = 0;
    // get_send_tensor's checks (migration.py:293-294); one dtype per field
    std::fill(field_dtype.begin(), field_dtype.end(), -1);
    for (int64_t k : g) {
      const sr_op& op = ops[k];
      const sr_meta& sm = metas[op.src_meta];
      int64_t want[SR_MAX_DIMS];
      if (!actual_shape(view_of(sm), want)) return fail(SR_EINVAL, "#%lld: size overflows", ll(name));
      for (int64_t f = 0; f < n_fields; ++f) {
        const sr_src_spec& sp = specs[k * n_fields + f];
        bool same = sp.ndim == sm.ndim;
        for (int64_t d = 0; same && d < sm.ndim; ++d) same = sp.shape[d] == want[d];
        if (!same) {
          shape_str(sp.shape, sp.ndim, a, sizeof a);
          shape_str(want, sm.ndim, b, sizeof b);
          return fail(SR_EINVAL, "get_send_tensor: param #%lld - src_tensor shape %s mismatch with src_meta %s",
                      ll(name), a, b);
        }
        if (field_dtype[f] < 0) field_dtype[f] = sp.dtype;
        if (field_dtype[f] != sp.dtype)
          return fail(SR_EINVAL, "#%lld field %lld: dtype differs between sources", ll(name), ll(f));
      }
      const bool piece_tp = op.piece_tp_deg > 0 || sh.tp_deg > 0;
      if (sm.tp_deg > 0 && piece_tp && sm.slice_dim != sh.slice_dim)
        return fail(SR_EINVAL, "get_send_tensor: param #%lld - slice dim mismatch btw src %lld and dst %lld",
                    ll(name), ll(sm.slice_dim), ll(sh.slice_dim));
    }
    int64_t dims[SR_MAX_DIMS], n_el = 1;
    if (!actual_shape(shard, dims)) return fail(SR_EINVAL, "#%lld: size overflows", ll(name));
    for (int64_t d = 0; d < sh.ndim; ++d)
      if (!mul(n_el, dims[d], &n_el)) return fail(SR_EINVAL, "#%lld: size overflows", ll(name));
    if (n_el == 0) {
      // nothing to move: an empty tensor per field, as clone() of an empty
      // piece gives in the reference (migration.py:538)
      for (int64_t f = 0; f < n_fields; ++f) {
        L->empty_v.push_back(slot_key(k0, f, 0, field_dtype[f], sh.ndim, dims));
        if (recast[f]) L->empty_v.push_back(slot_key(k0, f, 1, SR_DT_BF16, sh.ndim, dims));
      }
      continue;
    }
    int64_t dR, dC;
    if (!matrix(dims, sh.ndim, view, &dR, &dC)) return fail(SR_EINVAL, "#%lld: size overflows", ll(name));
    // destination slots of every field, then the pieces that fill them
    for (int64_t f = 0; f < n_fields; ++f) {
      dslot[f] = int32_t(L->dst_v.size());
      L->dst_v.push_back(sr_tensor{uint64_t(dR), uint64_t(dC), int32_t(field_dtype[f]), 0});
      L->dst_key_v.push_back(slot_key(k0, f, 0, field_dtype[f], sh.ndim, dims));
      dslot2[f] = -1;
      if (recast[f]) {
        if (field_dtype[f] != SR_DT_F32)
          return fail(SR_EINVAL, "#%lld field %lld: recast source must be float32", ll(name), ll(f));
        dslot2[f] = int32_t(L->dst_v.size());
        L->dst_v.push_back(sr_tensor{uint64_t(dR), uint64_t(dC), SR_DT_BF16, 0});
        L->dst_key_v.push_back(slot_key(k0, f, 1, SR_DT_BF16, sh.ndim, dims));
      }
    }
    for (int64_t k : g) {
      if (n_fields == 0) continue;
      const sr_op& op = ops[k];
      const int32_t peer = int32_t(std::lower_bound(L->peer_v.begin(), L->peer_v.end(), op.src_rank) -
                                   L->peer_v.begin());
      int32_t base = -1;
      for (const auto& rb : src_base)
        if (rb.first == op.src_rank) base = rb.second;
      if (base < 0) {
        base = int32_t(L->src_v.size());
        src_base.emplace_back(op.src_rank, base);
        const sr_src_spec& s0 = specs[k * n_fields];
        int64_t sR, sC;
        if (!matrix(s0.shape, s0.ndim, view, &sR, &sC)) return fail(SR_EINVAL, "#%lld: size overflows", ll(name));
        for (int64_t f = 0; f < n_fields; ++f) {
          const sr_src_spec& sp = specs[k * n_fields + f];
          L->src_v.push_back(sr_tensor{uint64_t(sR), uint64_t(sC), int32_t(sp.dtype), 0});
          L->src_key_v.push_back(slot_key(k, f, 0, sp.dtype, sp.ndim, sp.shape));
        }
      }
      if ((rc = lower_op(op, metas, shard, view, w, &regions)) != SR_OK) return rc;
      for (const Region& r : regions)
        for (int64_t f = 0; f < n_fields; ++f)
          L->piece_v.push_back(sr_piece{recast[f] ? SR_PIECE_RECAST : SR_PIECE_COPY, peer, base + int32_t(f),
                                        dslot[f], recast[f] ? dslot2[f] : -1, 0, uint64_t(r.rows),
                                        uint64_t(r.cols), uint64_t(r.src_row), uint64_t(r.src_col),
                                        uint64_t(r.dst_row), uint64_t(r.dst_col)});
    }
    // padding rows of a vocab_pad shard: zero fill, every slot of the tensor
    if ((rc = segments(shard, view, &w.dst, &w.pads)) != SR_OK) return rc;
    for (const Box& bx : w.pads)
      for (int64_t f = 0; f < n_fields; ++f)
        for (int32_t slot : {dslot[f], dslot2[f]})
          if (slot >= 0)
            L->piece_v.push_back(sr_piece{SR_PIECE_ZERO, 0, -1, slot, -1, 0, uint64_t(bx.rows), uint64_t(bx.cols),
                                          0, 0, uint64_t(bx.row), uint64_t(bx.col)});
  }
  if (L->src_v.size() > size_t(INT32_MAX) || L->dst_v.size() > size_t(INT32_MAX) ||
      L->piece_v.size() > size_t(INT32_MAX))
    return fail(SR_EINVAL, "sr_lower: more than 2^31 slots or pieces");
  return SR_OK;
}

}  // namespace

extern "C" {

int sr_lower(const sr_meta* metas, int64_t n_metas, const sr_op* ops, int64_t n_ops, const sr_src_spec* specs,
             int64_t n_fields, const int64_t* recast, sr_lowering** out) {
  if (!out) return fail(SR_EINVAL, "sr_lower: null output");
  *out = nullptr;
  Lowering* L = new (std::nothrow) Lowering();
  if (!L) return fail(SR_ENOMEM, "sr_lower: out of host memory");
  int rc;
  try {
    rc = lower(metas, n_metas, ops, n_ops, specs, n_fields, recast, L);
  } catch (const std::bad_alloc&) {
    rc = fail(SR_ENOMEM, "sr_lower: out of host memory");
  }
  if (rc != SR_OK) {
    delete L;
    return rc;
  }
  L->n_src = int64_t(L->src_v.size());
  L->n_dst = int64_t(L->dst_v.size());
  L->n_pieces = int64_t(L->piece_v.size());
  L->n_peers = int64_t(L->peer_v.size());
  L->n_empty = int64_t(L->empty_v.size());
  L->src = L->src_v.data();
  L->src_key = L->src_key_v.data();
  L->dst = L->dst_v.data();
  L->dst_key = L->dst_key_v.data();
  L->pieces = L->piece_v.data();
  L->peer_rank = L->peer_v.data();
  L->empty = L->empty_v.data();
  *out = L;
  return SR_OK;
}

void sr_lowering_destroy(sr_lowering* lowering) { delete static_cast<Lowering*>(lowering); }

}  // extern "C"
