/* A C11 caller of include/suika_reshard.h and include/suika_planner.h:
 * scheduling, plan creation, buffer layout and error reporting (host-only
 * calls, no GPU needed).  Prints one line per check; the test compares them. */
#include <stdio.h>
#include <string.h>

#include "suika_reshard.h"
#include "suika_planner.h"

/* one [4, 16] f32 row-parallel weight: rank `rank` holds column shard idx/deg */
static sr_meta weight(int64_t rank, int64_t idx, int64_t deg) {
  sr_meta m;
  memset(&m, 0, sizeof(m));
  m.rank = rank;
  m.name = 0;
  m.itemsize = 4;
  m.ndim = 2;
  m.shape[0] = 4;
  m.shape[1] = 16;
  m.slice_dim = -1;
  m.tp_index = idx;
  m.tp_deg = deg;
  m.kind = SR_KIND_CHUNK;
  m.row0 = m.row1 = -1;
  return m;
}

int main(void) {
  /* row-parallel merge: dst [4, 16] f32 = two [4, 8] column halves, two peers */
  sr_tensor src[2] = {{4, 8, SR_DT_F32, 0}, {4, 8, SR_DT_F32, 0}};
  sr_tensor dst[1] = {{4, 16, SR_DT_F32, 0}};
  sr_piece pcs[2] = {{SR_PIECE_COPY, 0, 0, 0, -1, 0, 4, 8, 0, 0, 0, 0},
                     {SR_PIECE_COPY, 1, 1, 0, -1, 0, 4, 8, 0, 0, 0, 8}};
  sr_plan* plan = NULL;
  int rc = sr_plan_create(src, 2, dst, 1, 2, pcs, 2, NULL, &plan);
  if (rc != SR_OK) {
    printf("create failed %d %s\n", rc, sr_last_error());
    return 1;
  }
  uint64_t b0 = 0, b1 = 0, off1 = 0;
  sr_plan_peer_bytes(plan, 0, &b0);
  sr_plan_peer_bytes(plan, 1, &b1);
  sr_plan_piece_offset(plan, 1, &off1);
  sr_plan_info info;
  memset(&info, 0, sizeof(info));
  sr_plan_info_get(plan, &info);
  printf("abi %d\n", sr_abi_version());
  printf("peer_bytes %llu %llu\n", (unsigned long long)b0, (unsigned long long)b1);
  printf("piece1_offset %llu\n", (unsigned long long)off1);
  printf("pieces %lld peers %lld pack_bytes_read %llu\n", (long long)info.n_pieces,
         (long long)info.n_peers, (unsigned long long)info.pack_bytes_read);
  sr_plan_destroy(plan);

  /* a hole in the destination is rejected with a message */
  sr_plan* bad = NULL;
  rc = sr_plan_create(src, 2, dst, 1, 2, pcs, 1, NULL, &bad);
  printf("hole %d %s\n", rc, bad == NULL ? "null" : "set");
  printf("message %s\n", strstr(sr_last_error(), "cover") ? "mentions coverage" : sr_last_error());

  /* the schedule of the same merge: TP2 -> TP1 on rank 0, one piece per source */
  sr_meta from[2] = {weight(0, 0, 2), weight(1, 1, 2)};
  sr_meta to[1] = {weight(0, 0, 1)};
  sr_op ops[4];
  int64_t n_ops = 0;
  rc = sr_schedule(from, 2, 2, to, 1, 1, 1, ops, 4, &n_ops);
  printf("schedule %d ops %lld\n", rc, (long long)n_ops);
  for (int64_t k = 0; k < n_ops; ++k)
    printf("op %lld -> %lld piece %lld/%lld\n", (long long)ops[k].src_rank, (long long)ops[k].dst_rank,
           (long long)ops[k].piece_tp_index, (long long)ops[k].piece_tp_deg);

  /* ... lowered to the engine's tables and planned, still without Python:
     one meta table (sources, then the target), the ops' shard rows shifted */
  sr_meta metas[3] = {from[0], from[1], to[0]};
  sr_src_spec specs[2];
  for (int64_t k = 0; k < n_ops; ++k) {
    ops[k].dst_shard += 2;
    memset(&specs[k], 0, sizeof(specs[k]));
    specs[k].dtype = SR_DT_F32;
    specs[k].ndim = 2;
    specs[k].shape[0] = 4;   /* each source shard: [4, 8] */
    specs[k].shape[1] = 8;
  }
  const int64_t no_recast[1] = {0};
  sr_lowering* low = NULL;
  rc = sr_lower(metas, 3, ops, n_ops, specs, 1, no_recast, &low);
  printf("lower %d src %lld dst %lld pieces %lld peers %lld\n", rc, (long long)low->n_src, (long long)low->n_dst,
         (long long)low->n_pieces, (long long)low->n_peers);
  for (int64_t k = 0; k < low->n_pieces; ++k)
    printf("piece peer %d src %d cols %llu dst_col %llu\n", low->pieces[k].peer, low->pieces[k].src,
           (unsigned long long)low->pieces[k].cols, (unsigned long long)low->pieces[k].dst_col);
  sr_plan* lowered = NULL;
  rc = sr_plan_create(low->src, (int32_t)low->n_src, low->dst, (int32_t)low->n_dst, (int32_t)low->n_peers,
                      low->pieces, (int32_t)low->n_pieces, NULL, &lowered);
  sr_plan_peer_bytes(lowered, 1, &b1);
  printf("planned %d peer1_bytes %llu\n", rc, (unsigned long long)b1);
  sr_plan_destroy(lowered);
  sr_lowering_destroy(low);
  return 0;
}
