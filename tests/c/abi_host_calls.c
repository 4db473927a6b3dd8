/* A C11 caller of include/suika_reshard.h: plan creation, buffer layout and
 * error reporting (host-only calls, no GPU needed).  Prints one line per
 * check; the test compares them. */
#include <stdio.h>
#include <string.h>

#include "suika_reshard.h"

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
  return 0;
}
