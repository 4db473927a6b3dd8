/* A C11 caller of the whole native path on the GPU, without Python:
 * layouts -> sr_schedule -> sr_lower -> sr_plan_create -> sr_gather and
 * sr_pack + sr_unpack on device memory from hipMalloc, checked byte for byte.
 *
 * The transfer is a row-parallel TP2 -> TP1 merge of one f32 weight
 * [ROWS, 2 * HALF] and a column-parallel TP2 -> TP1 merge of a bf16 bias-like
 * [2 * HALF] vector: source rank r holds column half r of the weight (a
 * strided destination region) and element half r of the vector.  Prints one
 * line per check; the test compares them. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "suika_planner.h"
#include "suika_reshard.h"

#define ROWS 1024
#define HALF 768

#define CHECK_HIP(x)                                                           \
  do {                                                                         \
    hipError_t e_ = (x);                                                       \
    if (e_ != hipSuccess) {                                                    \
      printf("hip error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      return 1;                                                                \
    }                                                                          \
  } while (0)

#define CHECK_SR(x)                                                            \
  do {                                                                         \
    int rc_ = (x);                                                             \
    if (rc_ != SR_OK) {                                                        \
      printf("sr error %d: %s at %s:%d\n", rc_, sr_last_error(), __FILE__, __LINE__); \
      return 1;                                                                \
    }                                                                          \
  } while (0)

static sr_meta meta(int64_t rank, int64_t name, int64_t itemsize, int64_t ndim, int64_t d0, int64_t d1,
                    int64_t slice_dim, int64_t idx, int64_t deg) {
  sr_meta m;
  memset(&m, 0, sizeof(m));
  m.rank = rank;
  m.name = name;
  m.itemsize = itemsize;
  m.ndim = ndim;
  m.shape[0] = d0;
  m.shape[1] = d1;
  m.slice_dim = slice_dim;
  m.tp_index = idx;
  m.tp_deg = deg;
  m.kind = SR_KIND_CHUNK;
  m.row0 = m.row1 = -1;
  return m;
}

int main(void) {
  /* layouts: name 0 = weight [ROWS, 2*HALF] f32 split along dim -1,
     name 1 = vector [2*HALF] bf16 split along dim 0 */
  sr_meta src[4] = {meta(0, 0, 4, 2, ROWS, 2 * HALF, -1, 0, 2), meta(0, 1, 2, 1, 2 * HALF, 0, 0, 0, 2),
                    meta(1, 0, 4, 2, ROWS, 2 * HALF, -1, 1, 2), meta(1, 1, 2, 1, 2 * HALF, 0, 0, 1, 2)};
  sr_meta dst[2] = {meta(0, 0, 4, 2, ROWS, 2 * HALF, -1, 0, 1), meta(0, 1, 2, 1, 2 * HALF, 0, 0, 0, 1)};
  sr_op ops[8];
  int64_t n_ops = 0;
  CHECK_SR(sr_schedule(src, 4, 2, dst, 2, 2, 1, ops, 8, &n_ops));
  printf("schedule ops %lld\n", (long long)n_ops);

  /* sr_lower wants one meta table: sources, then the target */
  sr_meta metas[6];
  memcpy(metas, src, sizeof(src));
  memcpy(metas + 4, dst, sizeof(dst));
  sr_src_spec specs[8];
  for (int64_t k = 0; k < n_ops; ++k) {
    ops[k].dst_shard += 4;
    const sr_meta* m = &src[ops[k].src_meta];
    memset(&specs[k], 0, sizeof(specs[k]));
    specs[k].dtype = m->name == 0 ? SR_DT_F32 : SR_DT_BF16;
    specs[k].ndim = m->ndim;
    specs[k].shape[0] = m->name == 0 ? ROWS : HALF;
    specs[k].shape[1] = m->name == 0 ? HALF : 0;
  }
  const int64_t no_recast[1] = {0};
  sr_lowering* low = NULL;
  CHECK_SR(sr_lower(metas, 6, ops, n_ops, specs, 1, no_recast, &low));
  printf("lowered src %lld dst %lld pieces %lld peers %lld\n", (long long)low->n_src, (long long)low->n_dst,
         (long long)low->n_pieces, (long long)low->n_peers);
  sr_plan* plan = NULL;
  CHECK_SR(sr_plan_create(low->src, (int32_t)low->n_src, low->dst, (int32_t)low->n_dst, (int32_t)low->n_peers,
                          low->pieces, (int32_t)low->n_pieces, NULL, &plan));

  /* host data: element values encode (rank, position) so a misplaced byte shows */
  size_t src_bytes[8], dst_bytes[8];
  void* h_src[8];
  void* d_src[8];
  for (int64_t s = 0; s < low->n_src; ++s) {
    const sr_slot_key* key = &low->src_key[s];
    const int64_t rank = ops[key->op].src_rank;
    const size_t n = (size_t)low->src[s].rows * low->src[s].cols;
    src_bytes[s] = n * (key->dtype == SR_DT_F32 ? 4 : 2);
    h_src[s] = malloc(src_bytes[s]);
    for (size_t i = 0; i < n; ++i) {
      if (key->dtype == SR_DT_F32) ((uint32_t*)h_src[s])[i] = (uint32_t)(rank * 100000000u + i);
      else ((uint16_t*)h_src[s])[i] = (uint16_t)(rank * 30000u + i);
    }
    CHECK_HIP(hipMalloc(&d_src[s], src_bytes[s]));
    CHECK_HIP(hipMemcpy(d_src[s], h_src[s], src_bytes[s], hipMemcpyHostToDevice));
  }
  void* d_dst[8];
  void* h_dst[8];
  for (int64_t t = 0; t < low->n_dst; ++t) {
    dst_bytes[t] = (size_t)low->dst[t].rows * low->dst[t].cols * (low->dst[t].dtype == SR_DT_F32 ? 4 : 2);
    CHECK_HIP(hipMalloc(&d_dst[t], dst_bytes[t]));
    h_dst[t] = malloc(dst_bytes[t]);
  }
  void* d_buf[8];
  for (int32_t q = 0; q < (int32_t)low->n_peers; ++q) {
    uint64_t b = 0;
    CHECK_SR(sr_plan_peer_bytes(plan, q, &b));
    CHECK_HIP(hipMalloc(&d_buf[q], b ? b : 1));
  }

  for (int route = 0; route < 2; ++route) {
    for (int64_t t = 0; t < low->n_dst; ++t) CHECK_HIP(hipMemset(d_dst[t], 0xA5, dst_bytes[t]));
    CHECK_HIP(hipDeviceSynchronize());
    if (route == 0) {
      CHECK_SR(sr_gather(plan, (const void* const*)d_src, (void* const*)d_dst, NULL));
    } else {
      CHECK_SR(sr_pack(plan, (const void* const*)d_src, (void* const*)d_buf, NULL));
      CHECK_SR(sr_unpack(plan, (const void* const*)d_buf, (void* const*)d_dst, NULL));
    }
    CHECK_HIP(hipDeviceSynchronize());
    /* expected: weight row r = [rank0 row r | rank1 row r]; vector = [rank0 | rank1] */
    long bad = 0;
    for (int64_t t = 0; t < low->n_dst; ++t) {
      CHECK_HIP(hipMemcpy(h_dst[t], d_dst[t], dst_bytes[t], hipMemcpyDeviceToHost));
      const sr_slot_key* key = &low->dst_key[t];
      if (key->dtype == SR_DT_F32) {
        const uint32_t* d = (const uint32_t*)h_dst[t];
        for (int64_t r = 0; r < ROWS; ++r)
          for (int64_t c = 0; c < 2 * HALF; ++c) {
            const uint32_t rank = (uint32_t)(c / HALF);
            const uint32_t want = rank * 100000000u + (uint32_t)(r * HALF + c % HALF);
            bad += d[r * 2 * HALF + c] != want;
          }
      } else {
        const uint16_t* d = (const uint16_t*)h_dst[t];
        for (int64_t i = 0; i < 2 * HALF; ++i) {
          const uint16_t want = (uint16_t)((i / HALF) * 30000u + (uint32_t)(i % HALF));
          bad += d[i] != want;
        }
      }
    }
    printf("%s mismatches %ld\n", route == 0 ? "gather" : "pack_unpack", bad);
  }

  sr_plan_destroy(plan);
  for (int64_t s = 0; s < low->n_src; ++s) {
    CHECK_HIP(hipFree(d_src[s]));
    free(h_src[s]);
  }
  for (int64_t t = 0; t < low->n_dst; ++t) {
    CHECK_HIP(hipFree(d_dst[t]));
    free(h_dst[t]);
  }
  for (int32_t q = 0; q < (int32_t)low->n_peers; ++q) CHECK_HIP(hipFree(d_buf[q]));
  sr_lowering_destroy(low);
  return 0;
}
