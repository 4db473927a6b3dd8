/*
 * suika_reshard.h -- C ABI of the MI355X reshard engine (libsuika_reshard.so).
 *
 * The engine executes the data movement of Suika's live state migration:
 * every destination shard of every state field (param / master / exp_avg /
 * exp_avg_sq) is assembled from 2-D regions of source shards.  The work is
 * split in two stream-ordered phases so that an exchange (one message per
 * peer) can sit between them:
 *
 *   pack   : source shards  -> one contiguous send buffer per peer
 *   unpack : peer buffers   -> destination shards
 *            (+ fused fp32 -> bf16 round-to-nearest-even recast,
 *             + zero fill of padded vocabulary rows)
 *
 * When every source shard is resident on this GPU (a checkpoint reshard, or
 * the pieces a rank keeps for itself), sr_gather moves the same pieces from
 * source to destination in one pass, without buffers.
 *
 * Reference interfaces replaced (paths relative to the Suika repository):
 *   - Suika/migration.py:290-312  TransferOp.get_send_tensor
 *       chunk(n, dim)[k].contiguous() of a source shard          -> sr_pack
 *   - Suika/migration.py:426-492  execute_param_transfer send/recv loop
 *       one torch.distributed isend/irecv per tensor per field   -> per-peer
 *       buffers sized by sr_plan_peer_bytes (one message per peer)
 *   - Suika/migration.py:531-541  execute_param_transfer post-process
 *       torch.cat(pieces, dim=slice_dim) / clone()               -> sr_unpack
 *   - Suika/migration.py:322-381  schedule_param_transfer output (TransferOp
 *       list) lowered by the Python host to sr_piece records     -> sr_plan_create
 *
 * Conventions
 *   - Every tensor is a dense row-major 2-D view [rows, cols] of elements of
 *     elem_bytes bytes (a 1-D tensor of n elements is [n, 1]).
 *   - All device memory (sources, peer buffers, destinations) belongs to the
 *     caller.  The library owns only the plan and its descriptor tables.
 *   - Calls that take a hipStream_t are asynchronous and stream-ordered; the
 *     caller synchronizes.  A plan may be used from one host thread at a time.
 *     A phase's first call builds its device tables on a library stream of
 *     the device (they read none of the caller's data); the copy kernel on the
 *     caller's stream waits for them through an event.
 *   - Device pointers must be aligned to their element size; peer buffers
 *     to 16 bytes (torch allocations are 512-byte aligned).
 *   - Status codes: SR_OK (0) on success, a negative sr_status otherwise.
 *     sr_last_error() returns a thread-local message for the last failure.
 *     Invalid plans and pointers are rejected before any kernel launch.
 */
#ifndef SUIKA_RESHARD_H
#define SUIKA_RESHARD_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SR_ABI_VERSION 5

typedef enum sr_status {
  SR_OK = 0,
  SR_EINVAL = -1,    /* malformed argument (null, bad enum, bad size) */
  SR_EBOUNDS = -2,   /* region outside its tensor or buffer */
  SR_EALIGN = -3,    /* pointer not aligned to its element size */
  SR_EOVERLAP = -4,  /* destination regions overlap or leave holes; or, at a
                        call, objects one launch writes overlap each other or
                        an object it reads */
  SR_EHIP = -5,      /* HIP runtime error */
  SR_ENOMEM = -6,    /* host or device allocation failed */
  SR_EDTYPE = -7     /* dtype/element-size mismatch between src and dst */
} sr_status;

/* Element types.  Copies move bytes; only SR_PIECE_RECAST interprets them. */
typedef enum sr_dtype {
  SR_DT_U8 = 0,
  SR_DT_BF16 = 1,
  SR_DT_F16 = 2,
  SR_DT_F32 = 3,
  SR_DT_F64 = 4,
  SR_DT_I32 = 5,
  SR_DT_I64 = 6
} sr_dtype;

/* A tensor slot of the plan: dense row-major [rows, cols]. */
typedef struct sr_tensor {
  uint64_t rows;
  uint64_t cols;
  int32_t dtype;      /* sr_dtype */
  int32_t reserved;   /* must be 0 */
} sr_tensor;

typedef enum sr_piece_kind {
  SR_PIECE_COPY = 0,    /* src region -> buffer -> dst region (same dtype) */
  SR_PIECE_RECAST = 1,  /* f32 src region -> buffer -> f32 dst region (if dst >= 0)
                           and bf16 RNE(src) into dst2 region */
  SR_PIECE_ZERO = 2     /* zero fill of a dst region (no source, no buffer bytes) */
} sr_piece_kind;

/* One region move.  Region origins/extents are in elements of the tensors. */
typedef struct sr_piece {
  int32_t kind;        /* sr_piece_kind */
  int32_t peer;        /* buffer index in [0, n_peers); ignored for ZERO */
  int32_t src;         /* source tensor slot; -1 for ZERO */
  int32_t dst;         /* destination tensor slot; -1 allowed for RECAST (bf16 only) */
  int32_t dst2;        /* RECAST: bf16 destination slot; otherwise -1 */
  int32_t reserved;    /* must be 0 */
  uint64_t rows;       /* region extent */
  uint64_t cols;
  uint64_t src_row;    /* region origin in src */
  uint64_t src_col;
  uint64_t dst_row;    /* region origin in dst (and in dst2 for RECAST) */
  uint64_t dst_col;
} sr_piece;

/* Plan tuning; pass NULL to sr_plan_create for the defaults. */
typedef struct sr_plan_options {
  uint32_t tile_bytes;   /* bytes of source data per work tile; power of two in
                            [4096, 16 MiB]; 0 = default (16384).  A RECAST
                            piece that writes both the f32 and the bf16 copy
                            moves 2.5x its source bytes and is cut at half
                            this size */
  uint32_t max_blocks;   /* cap on workgroups per launch (grid-stride beyond;
                            rounded down to a multiple of 8 when the tile list
                            is XCD-interleaved); 0 = one workgroup per tile */
  uint32_t flags;        /* SR_OPT_* bits */
  uint32_t reserved;     /* must be 0 */
} sr_plan_options;

#define SR_OPT_TEMPORAL 0x1u      /* ordinary cached loads/stores instead of the
                                     default streaming (non-temporal) ones */
#define SR_OPT_SKIP_COVERAGE 0x2u /* skip the destination coverage check */
#define SR_OPT_PIECE_ORDER 0x4u   /* run pieces in plan order instead of ordered by
                                     the tensor address they start at */
#define SR_OPT_NO_XCD_INTERLEAVE 0x8u /* keep the tile list linear instead of
                                     interleaving it 8 ways (by default each XCD, fed
                                     round-robin, walks one contiguous eighth) */
#define SR_OPT_NO_ROW_GROUPS 0x10u /* keep each strided piece's tiles together instead
                                     of dealing out the tiles of side-by-side pieces
                                     (a dim -1 concatenation) row block by row block */
#define SR_OPT_GATHER_ONLY 0x20u  /* build only the gather phase (the buffer layout is still
                                     reported); sr_pack / sr_unpack then fail with SR_EINVAL */

typedef struct sr_plan sr_plan;

typedef struct sr_plan_info {
  int64_t n_pieces;
  int64_t n_peers;
  int64_t n_src;
  int64_t n_dst;
  int64_t pack_tiles;
  int64_t unpack_tiles;
  uint64_t pack_bytes_read;      /* algorithmic bytes of the pack phase */
  uint64_t pack_bytes_written;
  uint64_t unpack_bytes_read;    /* algorithmic bytes of the unpack phase */
  uint64_t unpack_bytes_written;
  uint64_t buffer_bytes;         /* sum over peers of sr_plan_peer_bytes */
  int64_t gather_tiles;
  uint64_t gather_bytes_read;    /* algorithmic bytes of sr_gather */
  uint64_t gather_bytes_written;
} sr_plan_info;

/* ABI version of the loaded library (SR_ABI_VERSION). */
int sr_abi_version(void);

/* Thread-local message describing the last non-zero status. */
const char* sr_last_error(void);

/* Host-only arithmetic self test (division constants, tiling); SR_OK if good. */
int sr_selftest(void);

/*
 * Validate the pieces against the tensor slots and build the plan: buffer
 * offsets per peer (256-byte aligned, in piece order), work tiles of both
 * phases.  Host only: no device memory is touched until the first
 * sr_pack / sr_unpack.  Destinations must be covered exactly once by the
 * pieces (copies, recasts and zero fills) unless SR_OPT_SKIP_COVERAGE.
 * Replaces the plan construction of Suika/migration.py:322-381 + 426-492.
 */
int sr_plan_create(const sr_tensor* src_tensors, int32_t n_src,
                   const sr_tensor* dst_tensors, int32_t n_dst,
                   int32_t n_peers,
                   const sr_piece* pieces, int32_t n_pieces,
                   const sr_plan_options* options,
                   sr_plan** out_plan);

/* Bytes the buffer of `peer` must hold. */
int sr_plan_peer_bytes(const sr_plan* plan, int32_t peer, uint64_t* out_bytes);

/* Byte offset of piece `piece` inside its peer buffer (UINT64_MAX for ZERO). */
int sr_plan_piece_offset(const sr_plan* plan, int32_t piece, uint64_t* out_offset);

int sr_plan_info_get(const sr_plan* plan, sr_plan_info* out_info);

/*
 * Pack: gather every non-ZERO piece's source region into its peer buffer.
 * src_ptrs[n_src] are device addresses of the source slots, peer_bufs[n_peers]
 * of the peer buffers (each >= sr_plan_peer_bytes).  Replaces
 * TransferOp.get_send_tensor (Suika/migration.py:290-312) for every op.
 */
int sr_pack(sr_plan* plan, const void* const* src_ptrs, void* const* peer_bufs,
            hipStream_t stream);

/*
 * Unpack: scatter buffer contents into the destination slots, recast f32 ->
 * bf16 (round-to-nearest-even, NaN -> 0x7FC0) for RECAST pieces, zero fill
 * ZERO pieces.  Replaces the cat/clone post-process of
 * Suika/migration.py:531-541.
 */
int sr_unpack(sr_plan* plan, const void* const* peer_bufs, void* const* dst_ptrs,
              hipStream_t stream);

/*
 * Gather: every piece straight from its source region to its destination
 * region(s), with the unpack's recast and zero fill, in one launch; reads P
 * and writes D bytes instead of the 3P + D of pack + unpack.  For sources
 * resident on this GPU: the fake-source (checkpoint) mode of
 * execute_param_transfer (Suika/migration.py:477-482) and its self transfers
 * (migration.py:448-459).
 */
int sr_gather(sr_plan* plan, const void* const* src_ptrs, void* const* dst_ptrs,
              hipStream_t stream);

/* Device bytes per GPU that sr_gather_noalloc keeps its tables in. */
#define SR_SCRATCH_BYTES (64u << 20)

/*
 * Gather without allocating.  No counterpart in the reference: this is for
 * callers that cannot allocate device memory -- tight serving loops and
 * harnesses that forbid hipMalloc.  Same plan, pointers and result as
 * sr_gather, but the phase's device tables (descriptors, pointer table,
 * items, tile prefix sums and tile list) are placed in a static array of
 * SR_SCRATCH_BYTES per GPU, part of the library's code object: every process
 * that loads the library's GPU code on a device (any entry point that
 * launches a kernel there) holds that array on the device until it exits.
 * The call makes no hipMalloc, hipHostMalloc or hipFree, creates no event or
 * stream, and leaves the plan's own device state untouched.  The first call
 * in a process that has launched nothing of the library yet loads its GPU
 * code object, which is when the array is placed.
 *   - The tables need 96 + 64 + 8 + 8 bytes per piece (descriptor, item, tile
 *     prefix, emit chunk), 8 per tensor slot and 24 per tile (tile = plan
 *     tile_bytes of source data; the Llama2-7B share needs 35 MB at 16 KiB).
 *     A plan that needs more than SR_SCRATCH_BYTES is rejected with SR_ENOMEM
 *     before any device work: create it with a larger tile_bytes, or split
 *     the transfer into several plans.
 *   - The descriptors and pointers are uploaded from pageable host memory at
 *     every call, which HIP performs synchronously: the call blocks the host
 *     until the work queued on `stream` before it has finished and the tables
 *     are on the device; the tile, bind and copy kernels then run
 *     asynchronously.  For the same reason the call cannot be recorded into a
 *     HIP graph: on a stream that is capturing it returns SR_EINVAL and does
 *     nothing.
 *   - Every call on one GPU uses that GPU's single scratch array, which keeps
 *     the last call's tables: calls on one stream are ordered, but calls that
 *     overlap on one GPU (different streams or threads) race.
 */
int sr_gather_noalloc(const sr_plan* plan, const void* const* src_ptrs, void* const* dst_ptrs,
                      hipStream_t stream);

/* ------------------------------------------------ host-resident state
 * The reference's fake-source (checkpoint) mode slices sources that live in
 * host memory and moves each piece with .to(device), and returns the new
 * state on the device it is asked for, "cpu" included
 * (Suika/migration.py:477-482, 1235-1244).  Here the pieces' bytes, and only
 * they, cross to the GPU in the peer-buffer layout; the GPU unpacks them
 * (sr_unpack); sr_download brings results back to host memory.  Both go
 * through rings of SR_STAGE_WINDOWS pinned windows of SR_STAGE_WINDOW_BYTES,
 * one per device and copy direction, allocated on first use and held until
 * the process exits, and copy between the caller's host memory and the
 * windows on a pool of host threads (sr_set_host_threads).  A ring serves one
 * call at a time: concurrent uploads (or downloads) on one device wait for
 * each other, while an upload and a download can run at once on two streams,
 * one per link direction. */
#define SR_STAGE_WINDOW_BYTES (16u << 20)
#define SR_STAGE_WINDOWS 4

/*
 * Stage: sr_pack for sources in host memory.  Writes into the device peer
 * buffers exactly the bytes sr_pack would write from the same source
 * contents, so that sr_unpack then completes the reshard.  Each source slot
 * a non-ZERO piece reads is classified by its address: in host memory
 * (pageable or pinned), host threads copy the piece's rows into the pinned
 * windows and each window goes to the device with host-to-device copies on
 * `stream`; in device memory, the piece is copied on the device on `stream`
 * (2-D copies).  Only piece bytes are read: a dim 0 piece is a row range of
 * its source, a dim -1 piece one run per row.  The bytes between payloads
 * (256-byte alignment) are left undefined; nothing reads them.
 * Returns once every host source byte has been read (host sources may then
 * change or be freed); the copies finish in stream order.  Replaces
 * get_send_tensor(src).to(device) of the fake-source mode
 * (Suika/migration.py:290-312, 477-482).
 */
int sr_stage_pack(sr_plan* plan, const void* const* src_ptrs, void* const* peer_bufs,
                  hipStream_t stream);

/*
 * The host half of sr_stage_pack, for callers that move the buffers
 * themselves (to a file, a socket, their own copy engine): every non-ZERO
 * piece's source region, read from host memory at src_ptrs, is copied by
 * host threads into host buffers peer_bufs in the peer-buffer layout
 * (sr_plan_peer_bytes, sr_plan_piece_offset); a NULL buffer skips its peer
 * and the slots only its pieces read.  No HIP call: no device, stream or
 * pinned memory is involved, and the call returns when the buffers are
 * written.  Same bytes as sr_pack from the same source contents.
 */
int sr_pack_host(const sr_plan* plan, const void* const* src_ptrs, void* const* peer_bufs);

/*
 * Copy `n` device regions into host memory: region i is bytes[i] bytes at
 * device address dev_ptrs[i], written to host address host_ptrs[i]
 * (pageable or pinned; regions may not overlap).  The device-to-host copies
 * run on `stream` after the work queued there (for example the sr_unpack
 * that wrote the regions), through the pinned windows, adjacent device
 * regions in one copy; host threads move each window to its destinations.
 * Host regions are advised for transparent huge pages (madvise
 * MADV_HUGEPAGE on their whole 2 MiB pages) before they are written: fresh
 * memory is then mapped 2 MiB per fault instead of 4 KiB.
 * Returns when every host byte is written.  Serves execute_param_transfer's
 * device="cpu" (Suika/migration.py:1235-1244), whose result the reference
 * returns in host memory.
 */
int sr_download(const void* const* dev_ptrs, void* const* host_ptrs, const uint64_t* bytes, int32_t n,
                hipStream_t stream);

/*
 * Host threads that sr_stage_pack and sr_download copy with, the calling
 * thread included: n in [1, 256], or 0 for the default, the CPUs in the
 * process's affinity mask up to 16.
 */
int sr_set_host_threads(int32_t n);

/* Totals since the library was loaded (every device, every thread). */
typedef struct sr_stage_counters {
  uint64_t host_bytes_up;     /* bytes sr_stage_pack copied host -> device (windows: piece
                                 bytes plus the alignment gaps between adjacent pieces) */
  uint64_t host_piece_bytes;  /* piece bytes among them */
  uint64_t device_piece_bytes;/* piece bytes sr_stage_pack copied on the device */
  uint64_t bytes_down;        /* bytes sr_download copied device -> host */
  uint64_t windows;           /* pinned windows filled or drained */
} sr_stage_counters;

int sr_stage_counters_get(sr_stage_counters* out);

/*
 * Pay this process's first-use costs of the library on the current device
 * now: load its GPU code (one empty launch), create the device's setup
 * stream and events, and make one host-to-device copy from pinned memory on
 * `stream` and on the setup stream (a process's first copies on a stream
 * set up the runtime's copy path).  Returns when that work, and whatever was
 * queued on `stream` before it, is done; the memory used goes to the
 * library's table cache.  Optional: every entry
 * point does the same on first use.  No counterpart in the reference: it
 * serves callers that start fresh processes for a live migration (the old
 * and new worlds' ranks), which can pay these costs -- tens of milliseconds
 * with many processes on one GPU -- while they wait for each other instead
 * of inside the transfer.
 */
int sr_prepare(hipStream_t stream);

/*
 * Release a plan and its device tables.  Waits for the plan's own launches
 * still in flight (it may follow an asynchronous call directly); does not
 * synchronize anything else.  NULL is ignored.  The table memory and events
 * are kept for reuse by later plans instead of being freed (hipFree
 * synchronizes the device): at most 256 MiB of device memory and 64 MiB of
 * pinned host memory per process, held until the process exits.
 */
void sr_plan_destroy(sr_plan* plan);

#ifdef __cplusplus
}
#endif

#endif /* SUIKA_RESHARD_H */
