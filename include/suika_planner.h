/*
 * suika_planner.h -- native planner of libsuika_reshard.so: the transfer
 * schedule and its lowering to the engine's region moves.
 *
 * Host-only C ABI: no device memory, no HIP calls; usable without a GPU.
 * A C caller goes from two parameter layouts to the library's plan without
 * Python objects:
 *
 *   layouts (sr_meta tables) --sr_schedule--> transfer ops (sr_op table)
 *   one rank's ops --sr_lower--> slots + sr_piece table --sr_plan_create-->
 *   sr_gather / sr_pack + sr_unpack (include/suika_reshard.h)
 *
 * Reference interfaces replaced (paths relative to the Suika repository):
 *   - Suika/migration.py:29-131   TensorMeta          -> sr_meta (one row)
 *   - Suika/migration.py:161-254  ParamLayout         -> an sr_meta table,
 *       rank by rank; is_owned / owners / is_tensor_tp_owned /
 *       is_tensor_tp_overlap are evaluated inside sr_schedule
 *   - Suika/migration.py:257-312  TransferOp          -> sr_op (one row)
 *   - Suika/migration.py:322-381  schedule_param_transfer -> sr_schedule
 *   - Suika/migration.py:290-312, 531-541  TransferOp.get_send_tensor's
 *       chunk(n, dim)[k] and execute_param_transfer's cat(pieces, dim) per
 *       tensor and sub-field, as region moves                  -> sr_lower
 *
 * Status codes and sr_last_error() are those of suika_reshard.h.
 */
#ifndef SUIKA_PLANNER_H
#define SUIKA_PLANNER_H

#include <stdint.h>

#include "suika_reshard.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SR_MAX_DIMS 8
#define SR_MAX_TP_DEG 65536       /* largest tensor-parallel degree accepted */
#define SR_MAX_SCHEDULE (1 << 26) /* largest schedule sr_schedule produces */

/* Shard kinds: the reference's torch.chunk layout and two extensions. */
typedef enum sr_shard_kind {
  SR_KIND_CHUNK = 0,      /* chunk(tp_deg, slice_dim)[tp_index] */
  SR_KIND_VOCAB_PAD = 1,  /* rows of a table zero-padded to a multiple of
                             kind_args[0] * tp_deg, split along dim 0 */
  SR_KIND_QKV_HEADS = 2   /* fused [Q; K; V] split per projection at head
                             granularity; kind_args = (n_q, n_kv, head_dim) */
} sr_shard_kind;

/*
 * One TensorMeta of a layout: the global shape of a parameter and which
 * shard of it `rank` holds.  All fields are int64 so a table is a plain
 * [n, 21] int64 matrix.
 */
typedef struct sr_meta {
  int64_t rank;                  /* layout rank */
  int64_t name;                  /* caller's id of the tensor name, in [0, n_names) */
  int64_t itemsize;              /* bytes per element (the schedule balances bytes) */
  int64_t ndim;                  /* in [0, SR_MAX_DIMS] */
  int64_t shape[SR_MAX_DIMS];    /* global shape; vocab_pad: unpadded; unused dims 0 */
  int64_t slice_dim;             /* split dim (may be negative, Python style) */
  int64_t tp_index;
  int64_t tp_deg;                /* 0: not tensor-parallel (tp_meta None) */
  int64_t kind;                  /* sr_shard_kind */
  int64_t kind_args[3];          /* vocab_pad: (pad_multiple, 0, 0) */
  int64_t row0, row1;            /* a vocab piece's global rows [row0, row1); -1 otherwise */
} sr_meta;

/*
 * One scheduled piece: `src_rank` sends the part `piece` of parameter `name`
 * to `dst_rank`.  The piece is the destination shard cut at the largest
 * source TP degree (scale_to_tp, migration.py:103-118), or, for vocab_pad, a
 * row interval of the destination shard between source shard boundaries.
 */
typedef struct sr_op {
  int64_t name;
  int64_t src_rank;
  int64_t dst_rank;
  int64_t src_meta;              /* row of the source table: the source shard read */
  int64_t dst_shard;             /* row of the target table: the shard the piece lands in */
  int64_t piece_tp_index;        /* the piece's tp meta (slice_dim of the shard); */
  int64_t piece_tp_deg;          /*   deg 0: the piece is the whole destination shard */
  int64_t row0, row1;            /* vocab piece rows; -1 otherwise */
} sr_op;

/*
 * Greedy piece -> source assignment of schedule_param_transfer
 * (Suika/migration.py:322-381), on layouts given as tables.
 *
 * src[n_src] is the source layout and dst[n_dst] the target layout, each
 * grouped by rank (one contiguous block per rank, blocks in the layout's
 * rank order, a rank's tensors in its dict order).  The source layout has
 * n_src_ranks ranks (ranks holding no tensor included) and every source
 * rank is in [0, n_src_ranks): the reference sizes its load vector by the
 * rank count and indexes it by rank.  Pieces are
 * emitted in the reference's loop order: target rank block, tensor, piece.
 * Each goes to the destination rank itself when it owns the piece, else to
 * the owner with the smallest accumulated bytes (first in rank order on a
 * tie), restricted to already-connected owners once minimum_est_peers peers
 * are connected.
 *
 * Writes at most `cap` ops; *n_ops receives the schedule's length.  Returns
 * SR_EINVAL (nothing usable written) when cap is too small, when a piece
 * has no owner ("illegal transfer"), on malformed tables (a tp degree above
 * SR_MAX_TP_DEG among them), or when the schedule would exceed
 * SR_MAX_SCHEDULE pieces; the message names the tensor.
 */
int sr_schedule(const sr_meta* src, int64_t n_src, int64_t n_src_ranks,
                const sr_meta* dst, int64_t n_dst,
                int64_t n_names, int64_t minimum_est_peers,
                sr_op* ops, int64_t cap, int64_t* n_ops);

/* The tensor a source slot binds to: the caller's shard of one sub-field. */
typedef struct sr_src_spec {
  int64_t dtype;                 /* sr_dtype */
  int64_t ndim;
  int64_t shape[SR_MAX_DIMS];
} sr_src_spec;

/* What a tensor slot of a lowering holds. */
typedef struct sr_slot_key {
  int64_t op;                    /* an op of the tensor (the first one that uses it) */
  int64_t field;                 /* sub-field index in [0, n_fields) */
  int64_t recast;                /* 1: the bf16 copy rounded from `field` */
  int64_t dtype;                 /* sr_dtype */
  int64_t ndim;
  int64_t shape[SR_MAX_DIMS];    /* source: as given; destination: actual_shape of the shard */
} sr_slot_key;

/* Tables of one lowering, owned by the library until sr_lowering_destroy. */
typedef struct sr_lowering {
  int64_t n_src, n_dst, n_pieces, n_peers, n_empty;
  const sr_tensor* src;          /* [n_src] source slots, for sr_plan_create */
  const sr_slot_key* src_key;    /* [n_src] */
  const sr_tensor* dst;          /* [n_dst] destination slots */
  const sr_slot_key* dst_key;    /* [n_dst] */
  const sr_piece* pieces;        /* [n_pieces] */
  const int64_t* peer_rank;      /* [n_peers] source rank of each peer index, ascending */
  const sr_slot_key* empty;      /* [n_empty] zero-element destinations: no slot, no piece */
} sr_lowering;

/*
 * Lower one destination rank's ops to the engine's tables: for every tensor
 * (in order of first appearance) and sub-field, a destination slot of the
 * shard's 2-D view; for every op, source slots and one sr_piece per region x
 * sub-field -- the intersection of the piece with the source shard and the
 * destination shard, which for chunk layouts is chunk(n, dim)[k] on the
 * sending side and cat(pieces, dim) in ascending piece order on the
 * receiving side (Suika/migration.py:304-310, 536); ZERO pieces for the
 * padding rows of vocab_pad shards; RECAST pieces where recast[f] = 1 (an
 * f32 field also written as a bf16 copy, slot right after the field's).
 * Peers are the source ranks, ascending.
 *
 * metas[n_metas] holds every meta the ops name (op.src_meta and
 * op.dst_shard index it); specs[k * n_fields + f] is the source tensor of op
 * k, field f, and must have the op's source shard shape (get_send_tensor's
 * check, migration.py:293-294).  Returns SR_EINVAL with a message naming the
 * tensor (as "#<name id>") when the ops do not assemble their shards.
 */
int sr_lower(const sr_meta* metas, int64_t n_metas, const sr_op* ops, int64_t n_ops,
             const sr_src_spec* specs, int64_t n_fields, const int64_t* recast,
             sr_lowering** out);

/* Release the tables of sr_lower.  NULL is ignored. */
void sr_lowering_destroy(sr_lowering* lowering);

#ifdef __cplusplus
}
#endif

#endif /* SUIKA_PLANNER_H */
