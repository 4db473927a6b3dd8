// schedule.cpp -- native transfer scheduler (sr_schedule, include/suika_planner.h).
//
// Restates, over flat sr_meta tables, the greedy planner of Suika's state
// migration (paths relative to the Suika repository):
//   Suika/migration.py:322-381  schedule_param_transfer
//   Suika/migration.py:195-254  ParamLayout.is_owned / owners /
//                               is_tensor_tp_owned / is_tensor_tp_overlap
//   Suika/migration.py:62-118   TensorMeta.numel / volumn / actual_shape /
//                               scale_to_tp
// plus the two shard kinds the reference lacks: vocab_pad (a destination
// shard is cut into row intervals at every source shard boundary; ownership
// is row containment) and qkv_heads (nests across degrees like chunk).
//
// The schedule is a sequential greedy (each choice depends on the bytes
// already assigned), so it runs on the host; it is O(target pieces x owners)
// with every lookup indexed, against the reference's scan of all ranks per
// piece.  Load sums are doubles accumulated in the reference's order, so the
// choices -- ties included -- are the reference's.

#include <algorithm>
#include <cstdint>
#include <new>
#include <vector>

#include "sr_internal.h"
#include "sr_meta.h"
#include "suika_planner.h"
#include "suika_reshard.h"

namespace {

using namespace sr_internal;

// is_tensor_tp_owned (migration.py:246-254): may `src` (a layout row) send
// the piece `tgt`?  Returns 1 / 0, or a negative status.
int owned(const sr_meta& src_row, const View& tgt) {
  const View src = view_of(src_row);
  if (tgt.m->kind == SR_KIND_VOCAB_PAD) {
    if (src_row.kind != SR_KIND_VOCAB_PAD)
      return fail(SR_EINVAL, "shard kind mismatch for #%lld", (long long)tgt.m->name);
    int64_t lo, hi, slo, shi;
    if (!valid_rows(tgt, &lo, &hi) || !valid_rows(src, &slo, &shi))
      return fail(SR_EINVAL, "#%lld: vocabulary rows overflow", (long long)tgt.m->name);
    if (lo == hi) return 1;   // an empty piece (a shard of padding only)
    return slo <= lo && hi <= shi;
  }
  if (deg_of(src) > deg_of(tgt)) return 0;
  // is_tensor_tp_overlap (migration.py:220-244): a replicated side overlaps
  if (src.tp_deg == 0 || tgt.tp_deg == 0) return 1;
  if (src_row.slice_dim != tgt.m->slice_dim)
    return fail(SR_EINVAL, "slice dim mismatch %lld vs %lld", (long long)src_row.slice_dim,
                (long long)tgt.m->slice_dim);
  int64_t i1 = src.tp_index, d1 = src.tp_deg, i2 = tgt.tp_index, d2 = tgt.tp_deg;
  if (d1 > d2) {
    std::swap(i1, i2);
    std::swap(d1, d2);
  }
  return i2 / (d2 / d1) == i1;
}

// Contiguous blocks of equal `rank`; a rank may not come back later, and a
// name appears once per block.
int rank_blocks(const sr_meta* t, int64_t n, int64_t n_names, const char* table,
                std::vector<int64_t>* begin) {
  std::vector<int64_t> seen_in(n_names, -1);
  std::vector<int64_t> ranks;
  begin->clear();
  for (int64_t i = 0; i < n; ++i) {
    int rc = check_meta(t[i], n_names, table, i);
    if (rc != SR_OK) return rc;
    if (i == 0 || t[i].rank != t[i - 1].rank) {
      for (int64_t r : ranks)
        if (r == t[i].rank)
          return fail(SR_EINVAL, "%s: rank %lld is not one contiguous block", table,
                      (long long)t[i].rank);
      ranks.push_back(t[i].rank);
      begin->push_back(i);
    }
    int64_t& s = seen_in[t[i].name];
    if (s == (int64_t)begin->size())
      return fail(SR_EINVAL, "%s: #%lld twice on rank %lld", table, (long long)t[i].name,
                  (long long)t[i].rank);
    s = (int64_t)begin->size();
  }
  begin->push_back(n);
  return SR_OK;
}

int schedule(const sr_meta* src, int64_t n_src, int64_t R, const sr_meta* dst, int64_t n_dst,
             int64_t n_names, int64_t min_peers, sr_op* ops, int64_t cap, int64_t* n_ops) {
  if (n_src < 0 || R < 0 || n_dst < 0 || n_names < 0 || cap < 0 || !n_ops || (n_src && !src) ||
      (n_dst && !dst) || (cap && !ops))
    return fail(SR_EINVAL, "sr_schedule: null table or negative size");
  *n_ops = 0;
  std::vector<int64_t> sblk, dblk;
  int rc = rank_blocks(src, n_src, n_names, "source layout", &sblk);
  if (rc != SR_OK) return rc;
  rc = rank_blocks(dst, n_dst, n_names, "target layout", &dblk);
  if (rc != SR_OK) return rc;
  if (n_src == 0) return fail(SR_EINVAL, "empty source layout");
  // the load vector has one entry per source rank and is indexed by rank
  // value (migration.py:336, 365-369)
  for (size_t b = 0; b + 1 < sblk.size(); ++b) {
    const int64_t r = src[sblk[b]].rank;
    if (r < 0 || r >= R)
      return fail(SR_EINVAL, "source rank %lld outside the layout's %lld ranks", (long long)r,
                  (long long)R);
  }
  // every source row of a name, in rank-block order (the owners() order)
  std::vector<int64_t> name_begin(n_names + 1, 0), name_rows(n_src);
  for (int64_t i = 0; i < n_src; ++i) ++name_begin[src[i].name + 1];
  for (int64_t k = 0; k < n_names; ++k) name_begin[k + 1] += name_begin[k];
  {
    std::vector<int64_t> fill(name_begin.begin(), name_begin.end() - 1);
    for (int64_t i = 0; i < n_src; ++i) name_rows[fill[src[i].name]++] = i;
  }
  int64_t max_tp = 1;
  for (int64_t i = 0; i < n_src; ++i) max_tp = std::max(max_tp, deg_of(view_of(src[i])));

  std::vector<double> lat(R, 0.0);
  std::vector<char> est(R, 0);
  std::vector<View> pieces;
  std::vector<int64_t> owner_rows, cuts;
  int64_t count = 0;
  for (size_t b = 0; b + 1 < dblk.size(); ++b) {
    std::fill(est.begin(), est.end(), 0);
    int64_t n_est = 0;
    const int64_t dst_rank = dst[dblk[b]].rank;
    for (int64_t j = dblk[b]; j < dblk[b + 1]; ++j) {
      const sr_meta& dm = dst[j];
      const View shard = view_of(dm);
      const int64_t* rows_of = name_rows.data() + name_begin[dm.name];
      const int64_t n_rows = name_begin[dm.name + 1] - name_begin[dm.name];
      pieces.clear();
      if (dm.kind == SR_KIND_VOCAB_PAD && dm.tp_deg > 0) {
        // cut at every source shard boundary inside the shard's rows
        int64_t lo, hi;
        if (!valid_rows(shard, &lo, &hi))
          return fail(SR_EINVAL, "#%lld: vocabulary rows overflow", (long long)dm.name);
        if (lo == hi) {
          pieces.push_back(View{&dm, dm.tp_index, dm.tp_deg, lo, lo, false});
        } else {
          cuts.assign({lo, hi});
          for (int64_t q = 0; q < n_rows; ++q) {
            const sr_meta& s = src[rows_of[q]];
            if (s.kind != SR_KIND_VOCAB_PAD)
              return fail(SR_EINVAL, "shard kind mismatch for #%lld", (long long)dm.name);
            if (s.shape[0] != dm.shape[0])
              return fail(SR_EINVAL, "vocab size mismatch for #%lld: %lld vs %lld",
                          (long long)dm.name, (long long)s.shape[0], (long long)dm.shape[0]);
            int64_t slo, shi;
            if (!valid_rows(view_of(s), &slo, &shi))
              return fail(SR_EINVAL, "#%lld: vocabulary rows overflow", (long long)dm.name);
            for (int64_t e : {slo, shi})
              if (lo < e && e < hi) cuts.push_back(e);
          }
          std::sort(cuts.begin(), cuts.end());
          cuts.erase(std::unique(cuts.begin(), cuts.end()), cuts.end());
          for (size_t c = 0; c + 1 < cuts.size(); ++c)
            pieces.push_back(View{&dm, dm.tp_index, dm.tp_deg, cuts[c], cuts[c + 1], false});
        }
      } else if (dm.tp_deg > 0 && max_tp > dm.tp_deg) {
        // scale_to_tp (migration.py:103-118): ascending finer pieces
        if (max_tp % dm.tp_deg != 0)
          return fail(SR_EINVAL, "scale_to_tp: target degree %lld is not a multiple of %lld (#%lld)",
                      (long long)max_tp, (long long)dm.tp_deg, (long long)dm.name);
        const int64_t scale = max_tp / dm.tp_deg;   // <= SR_MAX_TP_DEG (checked degrees)
        for (int64_t i = 0; i < scale; ++i)
          pieces.push_back(View{&dm, scale * dm.tp_index + i, max_tp, -1, -1, false});
      } else {
        pieces.push_back(shard);
      }
      if (count + int64_t(pieces.size()) > SR_MAX_SCHEDULE)
        return fail(SR_EINVAL, "sr_schedule: more than %d pieces", SR_MAX_SCHEDULE);
      for (const View& p : pieces) {
        owner_rows.clear();
        bool self_owner = false;
        for (int64_t q = 0; q < n_rows; ++q) {
          const int o = owned(src[rows_of[q]], p);
          if (o < 0) return o;
          if (o) {
            owner_rows.push_back(rows_of[q]);
            self_owner |= src[rows_of[q]].rank == dst_rank;
          }
        }
        if (owner_rows.empty())
          return fail(SR_EINVAL, "illegal transfer, target param #%lld (tp %lld/%lld, rows "
                      "[%lld, %lld)) is not present in any source", (long long)dm.name,
                      (long long)p.tp_index, (long long)p.tp_deg, (long long)p.row0,
                      (long long)p.row1);
        int64_t vol;
        if (!volume(p, &vol)) return fail(SR_EINVAL, "#%lld: size overflows", (long long)dm.name);
        int64_t best = -1;
        if (self_owner) {
          for (int64_t k : owner_rows)
            if (src[k].rank == dst_rank) best = k;
        } else {
          // prefer connected owners once enough peers are connected
          bool use_est = false;
          if (n_est >= min_peers)
            for (int64_t k : owner_rows) use_est |= est[src[k].rank] != 0;
          double best_load = 0.0;
          for (int64_t k : owner_rows) {
            if (use_est && !est[src[k].rank]) continue;
            const double load = lat[src[k].rank] + (double)vol;
            if (best < 0 || load < best_load) {
              best = k;
              best_load = load;
            }
          }
        }
        const int64_t r = src[best].rank;
        if (!est[r]) {
          est[r] = 1;
          ++n_est;
        }
        if (count < cap) {
          sr_op& op = ops[count];
          op.name = dm.name;
          op.src_rank = r;
          op.dst_rank = dst_rank;
          op.src_meta = best;
          op.dst_shard = j;
          op.piece_tp_index = p.whole ? 0 : p.tp_index;
          op.piece_tp_deg = p.whole ? 0 : p.tp_deg;
          op.row0 = p.whole ? -1 : p.row0;
          op.row1 = p.whole ? -1 : p.row1;
        }
        ++count;
        lat[r] += (double)vol;
      }
    }
  }
  *n_ops = count;
  if (count > cap)
    return fail(SR_EINVAL, "sr_schedule: %lld ops do not fit in a table of %lld", (long long)count,
                (long long)cap);
  return SR_OK;
}

}  // namespace

extern "C" int sr_schedule(const sr_meta* src, int64_t n_src, int64_t n_src_ranks, const sr_meta* dst,
                           int64_t n_dst, int64_t n_names, int64_t minimum_est_peers, sr_op* ops,
                           int64_t cap, int64_t* n_ops) {
  try {
    return schedule(src, n_src, n_src_ranks, dst, n_dst, n_names, minimum_est_peers, ops, cap, n_ops);
  } catch (const std::bad_alloc&) {
    return fail(SR_ENOMEM, "sr_schedule: out of host memory");
  }
}
