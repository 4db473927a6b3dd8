// reshard.hip -- plan-driven pack / unpack engine for Suika state migration on
// MI355X (gfx950).  One source file: the C ABI declared in
// include/suika_reshard.h, the host-side plan builder, and the device kernels.
//
// Reference behaviour reproduced (paths relative to the Suika repository):
//   Suika/migration.py:290-312  get_send_tensor: chunk(n, dim)[k].contiguous()
//   Suika/migration.py:531-541  cat(pieces, dim=slice_dim) / clone()
// Both are pure byte movement.  The Python host lowers every TransferOp x
// sub-field into 2-D region moves (sr_piece); this file validates them, lays
// out the per-peer buffers and executes each phase -- pack (sources -> peer
// buffers), unpack (peer buffers -> destinations) or gather (sources ->
// destinations directly) -- as a single launch.
//
// Device design
//   * A phase is a list of items, one per piece.  An item is
//     a 2-D byte region: `rows` rows of `row_bytes` bytes at a source and a
//     destination stride.  Regions that are contiguous on both sides are
//     collapsed to one long row.
//   * Items are cut into tiles of `tile_bytes` (16 KiB) source bytes; one
//     workgroup (512 lanes = 8 wave64) processes one tile in a single pass,
//     and the grid is the tile count (or a grid-stride loop when capped).
//     Tiles balance the work whatever the tensor sizes (8 KB norms to GB
//     embeddings).
//   * The tile list follows the tensor address each item starts at and is
//     interleaved 8 ways: workgroups go to the 8 XCDs round-robin, so each XCD
//     walks one contiguous eighth of the work and the tiles in flight come
//     from 8 distant regions.  On the Llama2-7B share this takes the unpack
//     from 8.5 to 7.4 ms; a single window of consecutive tiles keeps the read
//     and write streams at a fixed distance and leaves HBM bandwidth idle.
//     Side-by-side strided items (the column bands of one dim -1 `cat`) deal
//     out their tiles row block by row block, so each destination row is
//     written by adjacent tiles.
//   * Lanes move 16-byte vectors (8/4/2/1 when a region is not 16-byte
//     aligned), two independent loads in flight before the stores.
//     Consecutive lanes touch consecutive 16-byte words of a row, so every
//     wave access is a coalesced 1 KB burst.  Loads and stores are
//     non-temporal by default: every byte is touched once.
//   * Strided regions (row-parallel dim -1 slices) map a tile-relative byte
//     position to (row, col) with a multiply-high division by the row width
//     (Granlund-Montgomery invariant-integer division), computed per item
//     on the host.
//   * The unpack RECAST item reads f32 once and writes the f32 copy and the
//     bf16 round-to-nearest-even copy in the same pass.
//   * The copy kernels use no LDS: every region row is >= 768 bytes at the
//     configured shapes, so a direct coalesced copy already issues full-width
//     bursts; a transpose is never needed because no piece changes the
//     element order within a row.
//
// Host design
//   * sr_plan_create is host only and O(pieces): validation, coverage, the
//     buffer layout the API reports, and one pointer-independent descriptor
//     per item.  The CPU test-suite exercises it without a GPU.
//   * The O(tiles) work runs on the GPU at first use of a phase: prefix sums
//     (wave64 shuffle scans, wave totals through LDS) give each peer's
//     256-byte aligned buffer offsets and each item's first tile, and an emit
//     kernel writes the tile table in its XCD-interleaved order.  The
//     Llama2-7B share has 1.44 M tiles per phase; building them on the host
//     took 0.12 s and a 35 MB upload per phase.
//   * Item tables hold absolute addresses.  When the caller's pointers
//     change, only the pointer table is uploaded and a bind kernel rebuilds
//     the items from the descriptors and the device-side buffer offsets.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "suika_reshard.h"
#include "sr_internal.h"

namespace sr_internal {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

const char* last_error() { return g_last_error.c_str(); }

int dtype_size(int32_t dt) {
  switch (dt) {
    case SR_DT_U8: return 1;
    case SR_DT_BF16: return 2;
    case SR_DT_F16: return 2;
    case SR_DT_F32: return 4;
    case SR_DT_F64: return 8;
    case SR_DT_I32: return 4;
    case SR_DT_I64: return 8;
    default: return 0;
  }
}

}  // namespace sr_internal

namespace {

#ifndef SR_BLOCK
#define SR_BLOCK 512
#endif
#ifndef SR_UNROLL
#define SR_UNROLL 2
#endif
constexpr int kBlock = SR_BLOCK;
constexpr int kUnroll = SR_UNROLL;
// Strided and recast paths carry two or three 64-bit offsets per vector;
// a smaller unroll keeps the kernel's register count (and so its occupancy)
// set by the contiguous copy path.
#ifndef SR_UNROLL_STRIDED
#define SR_UNROLL_STRIDED (SR_UNROLL < 4 ? SR_UNROLL : 4)
#endif
constexpr int kUnrollStrided = SR_UNROLL_STRIDED;
constexpr uint32_t kDefaultTileBytes = 16384;   // one 512-lane x 2 x 16 B pass
constexpr uint64_t kBufAlign = 256;
// Tile-list interleave width: the accelerator complex dies (XCDs) of an
// MI355X, which take workgroups round-robin.
#ifndef SR_INTERLEAVE_WAYS
#define SR_INTERLEAVE_WAYS 8
#endif
constexpr uint32_t kXcds = SR_INTERLEAVE_WAYS;
constexpr uint32_t kMaxGrid = 0xffffffffu / kBlock;    // grid work-items stay below 2^32
// A RECAST item that writes the f32 copy and the bf16 copy moves 2.5x its
// source bytes (a COPY item 2x); its tiles hold tile_bytes >> this many
// source bytes, so a workgroup's pass stays near a copy tile's traffic.
#ifndef SR_RECAST_TILE_SHIFT
#define SR_RECAST_TILE_SHIFT 1
#endif
constexpr uint32_t kRecastTileShift = SR_RECAST_TILE_SHIFT;
static_assert(kRecastTileShift <= 2, "RECAST tiles of at least tile_bytes / 4 (>= 1 KiB)");

// ---------------------------------------------------------------- errors

using sr_internal::fail;

#define SR_HIP_TRY(expr)                                                      \
  do {                                                                        \
    hipError_t e_ = (expr);                                                   \
    if (e_ != hipSuccess)                                                     \
      return fail(SR_EHIP, "%s failed: %s", #expr, hipGetErrorString(e_));    \
  } while (0)

using sr_internal::dtype_size;

// ------------------------------------------------ invariant integer division
// Granlund & Montgomery, "Division by invariant integers using
// multiplication" (PLDI 1994), Figure 4.1 with N = 32: for 1 <= d < 2^31 and
// any 32-bit n, q = (t + ((n - t) >> s1)) >> s2 with t = mulhi(m, n).

struct DivMagic {
  uint32_t m;
  uint32_t s1;
  uint32_t s2;
};

DivMagic div_magic(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;               // l = ceil(log2 d)
  const uint64_t num = (uint64_t(1) << 32) * ((uint64_t(1) << l) - d);
  DivMagic r;
  r.m = uint32_t(num / d + 1);
  r.s1 = l < 1 ? l : 1;
  r.s2 = l > 1 ? l - 1 : 0;
  return r;
}

__host__ __device__ inline uint32_t div_apply(uint32_t n, uint32_t m, uint32_t s1,
                                              uint32_t s2) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t t = __umulhi(m, n);
#else
  const uint32_t t = uint32_t((uint64_t(m) * n) >> 32);
#endif
  return (t + ((n - t) >> s1)) >> s2;
}

// ------------------------------------------------------- device structures

enum : uint32_t {
  kKindCopy = 0,
  kKindRecast = 1,
  kKindZero = 2,
};

// Item flags: bits 0-3 kind, 4-7 log2(vector bytes) (COPY/ZERO) or
// log2(elements per lane vector) (RECAST), bit 8: RECAST also writes f32.
struct alignas(16) DevItem {
  uint64_t src;           // absolute address of the region origin
  uint64_t dst;
  uint64_t dst2;          // bf16 target of RECAST
  uint64_t src_stride;    // bytes between rows
  uint64_t dst_stride;
  uint64_t dst2_stride;
  uint32_t row_bytes;     // source bytes per row; 0 = contiguous (one row)
  uint32_t magic;         // division by row_bytes
  uint32_t shifts;        // s1 | s2 << 8
  uint32_t flags;
};
static_assert(sizeof(DevItem) == 64, "DevItem layout");

struct alignas(8) DevTile {
  uint64_t start;    // contiguous: byte offset in the item; strided: first row
  uint32_t item;
  uint32_t nbytes;   // source bytes in this tile
  uint32_t c_base;   // strided: byte column of the tile start in its first row
  uint32_t pad;
};
static_assert(sizeof(DevTile) == 24, "DevTile layout");

// -------------------------------------------------------------- device code

template <int VB> struct VecOf;
template <> struct VecOf<16> { typedef unsigned int type __attribute__((ext_vector_type(4))); };
template <> struct VecOf<8> { typedef unsigned int type __attribute__((ext_vector_type(2))); };
template <> struct VecOf<4> { typedef unsigned int type; };
template <> struct VecOf<2> { typedef unsigned short type; };
template <> struct VecOf<1> { typedef unsigned char type; };

// Global-memory accessors.  Descriptor tables carry addresses as integers,
// so the global address space is stated here: the compiler then emits
// global_load/global_store (VMEM only) instead of flat instructions, which
// would also wait on the LDS counter.
#define SR_GLOBAL __attribute__((address_space(1)))

// Streaming (non-temporal) access applies to loads and stores separately
// (compile-time knobs, both on by default).
#ifndef SR_NT_LOADS
#define SR_NT_LOADS 1
#endif
#ifndef SR_NT_STORES
#define SR_NT_STORES 1
#endif

template <typename T, bool NT>
__device__ __forceinline__ T ld(uint64_t addr) {
  const SR_GLOBAL T* p = (const SR_GLOBAL T*)addr;
  if constexpr (NT && SR_NT_LOADS) return __builtin_nontemporal_load(p);
  else return *p;
}

template <typename T, bool NT>
__device__ __forceinline__ void st(uint64_t addr, T v) {
  SR_GLOBAL T* p = (SR_GLOBAL T*)addr;
  if constexpr (NT && SR_NT_STORES) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// Byte offsets, relative to the item's origins, of the source byte `b`
// (counted from the start of the tile): source side, destination side and
// bf16 side (half the destination column).  Contiguous items are one long
// row; strided items divide by the row width.
template <bool CONTIG>
struct TileMap {
  uint64_t start;
  uint32_t c_base, width, magic, s1, s2;
  uint64_t src_stride, dst_stride, dst2_stride;

  __device__ __forceinline__ TileMap(const DevItem& it, const DevTile& t)
      : start(t.start), c_base(t.c_base), width(it.row_bytes), magic(it.magic),
        s1(it.shifts & 0xffu), s2(it.shifts >> 8), src_stride(it.src_stride),
        dst_stride(it.dst_stride), dst2_stride(it.dst2_stride) {}

  __device__ __forceinline__ void at(uint32_t b, uint64_t& so, uint64_t& dof) const {
    if constexpr (CONTIG) {
      so = start + b;
      dof = so;
    } else {
      const uint32_t x = c_base + b;
      const uint32_t q = div_apply(x, magic, s1, s2);
      const uint64_t row = start + q;
      const uint32_t col = x - q * width;
      so = row * src_stride + col;
      dof = row * dst_stride + col;
    }
  }

  __device__ __forceinline__ void at(uint32_t b, uint64_t& so, uint64_t& dof, uint64_t& ho) const {
    if constexpr (CONTIG) {
      so = start + b;
      dof = so;
      ho = so >> 1;
    } else {
      const uint32_t x = c_base + b;
      const uint32_t q = div_apply(x, magic, s1, s2);
      const uint64_t row = start + q;
      const uint32_t col = x - q * width;
      so = row * src_stride + col;
      dof = row * dst_stride + col;
      ho = row * dst2_stride + (col >> 1);
    }
  }
};

// Copy one tile.  The main loop covers whole groups of kBlock * kUnroll
// vectors with no bounds test, so each lane issues its kUnroll loads back to
// back before the stores; the tail takes the remaining vectors one by one.
template <int VB, bool NT, bool CONTIG>
__device__ void copy_tile(const DevItem& it, const DevTile& t) {
  typedef typename VecOf<VB>::type V;
  constexpr int U = CONTIG ? kUnroll : kUnrollStrided;
  const TileMap<CONTIG> map(it, t);
  const uint32_t nvec = t.nbytes / VB;
  constexpr uint32_t kStep = kBlock * U;
  const uint32_t nfull = nvec / kStep * kStep;
  for (uint32_t base = 0; base < nfull; base += kStep) {
    V v[U];
    uint64_t doff[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      uint64_t soff;
      map.at((base + u * kBlock + threadIdx.x) * VB, soff, doff[u]);
      v[u] = ld<V, NT>(it.src + soff);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) st<V, NT>(it.dst + doff[u], v[u]);
  }
  for (uint32_t i = nfull + threadIdx.x; i < nvec; i += kBlock) {
    uint64_t soff, doff;
    map.at(i * VB, soff, doff);
    st<V, NT>(it.dst + doff, ld<V, NT>(it.src + soff));
  }
}

template <int VB, bool NT, bool CONTIG>
__device__ void zero_tile(const DevItem& it, const DevTile& t) {
  typedef typename VecOf<VB>::type V;
  const TileMap<CONTIG> map(it, t);
  const uint32_t nvec = t.nbytes / VB;
  const V z = V(0);
  for (uint32_t i = threadIdx.x; i < nvec; i += kBlock) {
    uint64_t soff, doff;
    map.at(i * VB, soff, doff);
    st<V, NT>(it.dst + doff, z);
  }
}

// float -> bfloat16, round to nearest, ties to even; NaN -> 0x7FC0.
// This is the standard integer rounding of the upper half-word: add
// 0x7FFF plus the lowest kept bit, then truncate.
__device__ __forceinline__ uint32_t bf16_rne(uint32_t u) {
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

template <int NE>
__device__ __forceinline__ typename VecOf<2 * NE>::type to_bf16(typename VecOf<4 * NE>::type v) {
  typename VecOf<2 * NE>::type h;
  if constexpr (NE == 4) {
    h.x = bf16_rne(v.x) | (bf16_rne(v.y) << 16);
    h.y = bf16_rne(v.z) | (bf16_rne(v.w) << 16);
  } else {
    h = (unsigned short)bf16_rne(v);
  }
  return h;
}

// f32 region -> f32 copy (when the item has one) + bf16 RNE copy.
template <int NE, bool NT, bool CONTIG>
__device__ void recast_tile(const DevItem& it, const DevTile& t) {
  constexpr int SB = 4 * NE;                 // source (f32) bytes per lane vector
  typedef typename VecOf<SB>::type VS;       // NE f32
  typedef typename VecOf<2 * NE>::type VH;   // NE bf16
  const TileMap<CONTIG> map(it, t);
  const uint32_t nvec = t.nbytes / SB;
  const bool has_dst = (it.flags >> 8) & 1u;
  constexpr int U = kUnrollStrided;
  constexpr uint32_t kStep = kBlock * U;
  const uint32_t nfull = nvec / kStep * kStep;
  for (uint32_t base = 0; base < nfull; base += kStep) {
    VS v[U];
    uint64_t doff[U], hoff[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      uint64_t soff;
      map.at((base + u * kBlock + threadIdx.x) * SB, soff, doff[u], hoff[u]);
      v[u] = ld<VS, NT>(it.src + soff);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (has_dst) st<VS, NT>(it.dst + doff[u], v[u]);
      st<VH, NT>(it.dst2 + hoff[u], to_bf16<NE>(v[u]));
    }
  }
  for (uint32_t i = nfull + threadIdx.x; i < nvec; i += kBlock) {
    uint64_t soff, doff, hoff;
    map.at(i * SB, soff, doff, hoff);
    const VS v = ld<VS, NT>(it.src + soff);
    if (has_dst) st<VS, NT>(it.dst + doff, v);
    st<VH, NT>(it.dst2 + hoff, to_bf16<NE>(v));
  }
}

template <bool NT, bool CONTIG>
__device__ __forceinline__ void exec_tile(const DevItem& it, const DevTile& t) {
  const uint32_t kind = it.flags & 0xfu;
  const uint32_t lv = (it.flags >> 4) & 0xfu;
  if (kind == kKindCopy) {
    switch (lv) {
      case 4: copy_tile<16, NT, CONTIG>(it, t); break;
      case 3: copy_tile<8, NT, CONTIG>(it, t); break;
      case 2: copy_tile<4, NT, CONTIG>(it, t); break;
      case 1: copy_tile<2, NT, CONTIG>(it, t); break;
      default: copy_tile<1, NT, CONTIG>(it, t); break;
    }
  } else if (kind == kKindRecast) {
    if (lv == 2) recast_tile<4, NT, CONTIG>(it, t);
    else recast_tile<1, NT, CONTIG>(it, t);
  } else {
    switch (lv) {
      case 4: zero_tile<16, NT, CONTIG>(it, t); break;
      case 3: zero_tile<8, NT, CONTIG>(it, t); break;
      case 2: zero_tile<4, NT, CONTIG>(it, t); break;
      case 1: zero_tile<2, NT, CONTIG>(it, t); break;
      default: zero_tile<1, NT, CONTIG>(it, t); break;
    }
  }
}

template <bool NT>
__device__ __forceinline__ void exec_tiles(const DevItem* __restrict__ items,
                                           const DevTile* __restrict__ tiles, uint32_t n_tiles) {
  for (uint32_t ti = blockIdx.x; ti < n_tiles; ti += gridDim.x) {
    const DevTile t = tiles[ti];
    const DevItem it = items[t.item];
    if (it.row_bytes == 0) exec_tile<NT, true>(it, t);
    else exec_tile<NT, false>(it, t);
  }
}

// Two entry points with one body, so profiles tell the phases apart.
template <bool NT>
__global__ __launch_bounds__(kBlock) void sr_pack_kernel(const DevItem* __restrict__ items,
                                                         const DevTile* __restrict__ tiles,
                                                         uint32_t n_tiles) {
  exec_tiles<NT>(items, tiles, n_tiles);
}

template <bool NT>
__global__ __launch_bounds__(kBlock) void sr_unpack_kernel(const DevItem* __restrict__ items,
                                                           const DevTile* __restrict__ tiles,
                                                           uint32_t n_tiles) {
  exec_tiles<NT>(items, tiles, n_tiles);
}

template <bool NT>
__global__ __launch_bounds__(kBlock) void sr_gather_kernel(const DevItem* __restrict__ items,
                                                           const DevTile* __restrict__ tiles,
                                                           uint32_t n_tiles) {
  exec_tiles<NT>(items, tiles, n_tiles);
}

// ------------------------------------------------- device-side plan binding
// The host keeps O(pieces) descriptors and the prefix sum of their tile
// counts; the per-tile table, the per-peer buffer offsets and the
// absolute-address item table are computed on the GPU from them:
//   sr_offsets_kernel   per peer: exclusive prefix sum of the 256-byte
//                       rounded payloads of its pieces, in piece order;
//   sr_tile_emit_kernel one workgroup per item writes its tiles, placed in
//                       the XCD-interleaved order, and on a phase's first
//                       launch binds the item as sr_bind_kernel does;
//   sr_bind_kernel      one lane per item: caller pointers + offsets ->
//                       DevItem (addresses, vector width); later launches
//                       with other pointers.

// Pointer-independent item descriptor (device resident, uploaded once).
enum : uint32_t {
  kRelSrcBuf = 1u << 16,   // source side is a peer buffer at the piece's offset
  kRelDstBuf = 1u << 17,   // destination side is a peer buffer at the piece's offset
  kRelTileShiftBit = 20,   // bits 20-23: the item's tiles are tile_bytes >> this
};

// log2 of an item's tile size in source bytes.
__host__ __device__ inline uint32_t item_tile_shift(uint32_t kind, uint32_t tile_shift) {
  return tile_shift - ((kind >> kRelTileShiftBit) & 0xfu);
}

struct alignas(8) DevRel {
  uint64_t src_off;        // byte offset of the region origin in its object
  uint64_t dst_off;
  uint64_t dst2_off;
  uint64_t src_stride;
  uint64_t dst_stride;
  uint64_t dst2_stride;
  uint64_t total;          // source bytes (destination bytes for ZERO)
  uint32_t row_bytes;      // 0 = contiguous
  uint32_t magic;
  uint32_t shifts;
  uint32_t kind;           // bits 0-7 kind, 8-15 element bytes, kRelSrcBuf / kRelDstBuf,
                           // bits 20-23 tile size reduction (kRelTileShiftBit)
  int32_t src_slot;        // index into the phase's pointer table, -1 = none
  int32_t dst_slot;
  int32_t dst2_slot;
  int32_t piece;           // piece whose buffer offset the buffer side uses
  uint32_t group_size;     // items whose tiles are dealt out row block by row block
  uint32_t group_index;    // this item's place in its group
};
static_assert(sizeof(DevRel) == 96, "DevRel layout");

// Exclusive prefix sum across a workgroup of NT lanes: an inclusive scan
// inside each wave64 by shuffles, then the wave totals through LDS.  Every
// lane of the workgroup must call it (it synchronises).  `total` receives
// the sum over the workgroup.
template <int NT>
__device__ uint64_t block_exclusive_scan(uint64_t v, uint64_t& total) {
  constexpr int kWaves = NT / 64;
  __shared__ uint64_t wave_sum[kWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint64_t x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint64_t y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) wave_sum[wave] = x;
  __syncthreads();
  uint64_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const uint64_t s = wave_sum[w];
    if (w < wave) before += s;
    all += s;
  }
  __syncthreads();   // wave_sum is reused by the next call
  total = all;
  return before + x - v;
}

constexpr int kSetupBlock = 256;
// Tiles one workgroup of the emit kernel writes at most (16 per lane): a
// large item's tiles are spread over several workgroups.
constexpr uint32_t kEmitTiles = 4096;
// Phases of at most this many tiles set up on the caller's stream even
// while earlier work still runs there: their setup takes a few microseconds
// of GPU time, less than a wait across streams costs the host.
constexpr uint64_t kInlineSetupTiles = 65536;

// An empty kernel: launching it loads the library's GPU code (sr_prepare).
__global__ void sr_prepare_kernel() {}

struct EmitChunk {
  uint32_t item;
  uint32_t chunk;   // the item's tiles [chunk * kEmitTiles, (chunk + 1) * kEmitTiles)
};
static_assert(sizeof(EmitChunk) == 8, "EmitChunk layout");

// One workgroup per peer.  peer_begin[p]..peer_begin[p+1] indexes
// peer_list, the peer's pieces in piece order.
__global__ __launch_bounds__(kSetupBlock) void sr_offsets_kernel(
    const uint32_t* __restrict__ peer_begin, const uint32_t* __restrict__ peer_list,
    const uint64_t* __restrict__ payload, uint64_t* __restrict__ offset) {
  const uint32_t b = peer_begin[blockIdx.x];
  const uint32_t e = peer_begin[blockIdx.x + 1];
  uint64_t carry = 0;
  for (uint32_t base = b; base < e; base += kSetupBlock) {
    const uint32_t i = base + threadIdx.x;
    const bool ok = i < e;
    const uint32_t k = ok ? peer_list[i] : 0u;
    const uint64_t v = ok ? (payload[k] + kBufAlign - 1) / kBufAlign * kBufAlign : 0;
    uint64_t total;
    const uint64_t ex = block_exclusive_scan<kSetupBlock>(v, total);
    if (ok) offset[k] = carry + ex;
    carry += total;
  }
}

// Largest power-of-two vector width (<= 16, >= esize) dividing every value
// OR-ed into `acc`.
__host__ __device__ inline uint32_t pick_vb(uint64_t acc, uint32_t esize) {
  uint32_t vb = 16;
  while (vb > esize && (acc & (vb - 1))) vb >>= 1;
  return vb;
}

__host__ __device__ inline uint32_t log2u(uint32_t v) {
  uint32_t l = 0;
  while ((1u << l) < v) ++l;
  return l;
}

// The item of descriptor `h`: its object addresses resolved from `ptrs`,
// the phase's pointer table (source objects, then destination objects),
// and `offset`, the per-piece buffer offsets from sr_offsets_kernel, and
// the widest vector access its addresses and sizes allow.
__device__ __forceinline__ DevItem bind_item(const DevRel& h, const uint64_t* __restrict__ ptrs,
                                             const uint64_t* __restrict__ offset) {
  const uint32_t kind = h.kind & 0xffu;
  const uint32_t esize = (h.kind >> 8) & 0xffu;
  const bool contiguous = h.row_bytes == 0;
  DevItem d;
  d.src = h.src_slot >= 0 ? ptrs[h.src_slot] + ((h.kind & kRelSrcBuf) ? offset[h.piece] : h.src_off) : 0;
  d.dst = h.dst_slot >= 0 ? ptrs[h.dst_slot] + ((h.kind & kRelDstBuf) ? offset[h.piece] : h.dst_off) : 0;
  d.dst2 = h.dst2_slot >= 0 ? ptrs[h.dst2_slot] + h.dst2_off : 0;
  d.src_stride = h.src_stride;
  d.dst_stride = h.dst_stride;
  d.dst2_stride = h.dst2_stride;
  d.row_bytes = h.row_bytes;
  d.magic = h.magic;
  d.shifts = h.shifts;
  uint32_t lv = 0;
  if (kind == kKindCopy) {
    uint64_t acc = d.src | d.dst;
    acc |= contiguous ? h.total : (uint64_t(h.row_bytes) | h.src_stride | h.dst_stride);
    lv = log2u(pick_vb(acc, esize));
  } else if (kind == kKindZero) {
    uint64_t acc = d.dst;
    acc |= contiguous ? h.total : (uint64_t(h.row_bytes) | h.dst_stride);
    lv = log2u(pick_vb(acc, esize));
  } else {
    // RECAST: 4 f32 per lane when the f32 sides are 16-byte and the bf16
    // side 8-byte aligned, otherwise one element per lane.
    const bool has_dst = h.dst_slot >= 0;
    bool wide = ((d.src | (has_dst ? d.dst : 0)) & 15) == 0 && (d.dst2 & 7) == 0;
    if (contiguous) {
      wide = wide && (h.total & 15) == 0;
    } else {
      wide = wide && (h.row_bytes & 15) == 0 && (h.src_stride & 15) == 0 &&
             (!has_dst || (h.dst_stride & 15) == 0) && (h.dst2_stride & 7) == 0;
    }
    lv = wide ? 2 : 0;
  }
  d.flags = kind | (lv << 4) | ((kind == kKindRecast && h.dst_slot >= 0) ? (1u << 8) : 0u);
  return d;
}

// Tile i of the item-ordered list goes to position pos(i).  With `ways`
// segments of seg = ceil(n/ways) tiles (q full segments and a last one of
// r tiles), tile j of segment s is dispatched at j*q + min(j, r) + s: the
// list is read column by column, so consecutive workgroups -- which the
// hardware deals to the 8 XCDs in turn -- take one tile from each segment.
__device__ __forceinline__ uint64_t xcd_position(uint64_t i, uint64_t seg, uint64_t q, uint64_t r) {
  const uint64_t s = i / seg;
  const uint64_t j = i - s * seg;
  return j * q + (j < r ? j : r) + s;
}

// One workgroup per emit chunk -- up to kEmitTiles consecutive tiles of one
// item (chunks[c] = {item, chunk index}; every item has at least one) --
// writes those tiles (tile_base[k] = tiles of items 0..k-1, computed with the
// descriptors on the host).  With `items` non-null, lane 0 of an item's
// first chunk also binds the item to the pointer table `ptrs` (and the
// buffer offsets `offset`), as sr_bind_kernel does: a phase's first launch
// builds both tables in one kernel.
__global__ __launch_bounds__(kSetupBlock) void sr_tile_emit_kernel(
    const DevRel* __restrict__ rel, const uint64_t* __restrict__ tile_base, const EmitChunk* __restrict__ chunks,
    uint32_t n_chunks, uint32_t tile_shift, uint64_t n_tiles, uint32_t ways, DevTile* __restrict__ tiles,
    const uint64_t* __restrict__ ptrs, const uint64_t* __restrict__ offset, DevItem* __restrict__ items) {
  uint64_t seg = 1, q = n_tiles, r = 0;
  if (ways > 1) {
    seg = (n_tiles + ways - 1) / ways;
    q = n_tiles / seg;
    r = n_tiles - q * seg;
  }
  for (uint32_t c = blockIdx.x; c < n_chunks; c += gridDim.x) {
    const uint32_t k = chunks[c].item;
    const uint64_t j0 = uint64_t(chunks[c].chunk) * kEmitTiles;
    const uint64_t total = rel[k].total;
    const uint32_t width = rel[k].row_bytes;
    const uint32_t sh = item_tile_shift(rel[k].kind, tile_shift);
    const uint64_t cnt = tile_base[k + 1] - tile_base[k];
    // Items of a group have equal tile counts; tile j of member m goes to
    // group_start + j*M + m, so the members' tiles over the same rows are
    // adjacent in the list.
    const uint64_t gm = rel[k].group_index;
    const uint64_t gsize = rel[k].group_size;
    const uint64_t b = tile_base[k] - gm * cnt + gm;
    if (items != nullptr && j0 == 0 && threadIdx.x == 0) items[k] = bind_item(rel[k], ptrs, offset);
    const uint64_t j1 = cnt < j0 + kEmitTiles ? cnt : j0 + kEmitTiles;
    for (uint64_t j = j0 + threadIdx.x; j < j1; j += kSetupBlock) {
      const uint64_t start = j << sh;
      const uint64_t left = total - start;
      DevTile t;
      t.item = k;
      t.nbytes = uint32_t(left < (uint64_t(1) << sh) ? left : (uint64_t(1) << sh));
      t.pad = 0;
      if (width == 0) {
        t.start = start;
        t.c_base = 0;
      } else {
        const uint64_t row = start / width;
        t.start = row;
        t.c_base = uint32_t(start - row * width);
      }
      const uint64_t i = b + j * gsize;
      tiles[ways > 1 ? xcd_position(i, seg, q, r) : i] = t;
    }
  }
}

__global__ __launch_bounds__(kSetupBlock) void sr_bind_kernel(const DevRel* __restrict__ rel,
                                                              uint32_t n,
                                                              const uint64_t* __restrict__ ptrs,
                                                              const uint64_t* __restrict__ offset,
                                                              DevItem* __restrict__ items) {
  const uint32_t k = blockIdx.x * kSetupBlock + threadIdx.x;
  if (k >= n) return;
  items[k] = bind_item(rel[k], ptrs, offset);
}

// ----------------------------------------------------------- host structures

// Pointer-independent description of one item of a phase.
struct HostItem {
  uint32_t kind;
  int32_t src_slot;       // pack: src tensor slot; unpack: peer index
  int32_t dst_slot;       // pack: peer index; unpack: dst slot (-1: none)
  int32_t dst2_slot;      // unpack RECAST: bf16 slot, else -1
  uint64_t src_off;       // byte offset of region origin in the source object
  uint64_t dst_off;
  uint64_t dst2_off;
  uint64_t src_stride;
  uint64_t dst_stride;
  uint64_t dst2_stride;
  uint64_t rows;
  uint64_t row_bytes;     // source bytes per row (dst bytes for ZERO)
  bool contiguous;        // collapsed to one row of rows*row_bytes bytes
  uint32_t esize;         // element bytes of the source (dst for ZERO)
  int32_t piece;          // the sr_piece this item moves
};

struct Phase {
  std::vector<HostItem> items;          // in piece order while the plan is built
  std::vector<DevRel> rel;              // items in dispatch (tile) order
  std::vector<uint64_t> tile_base;      // tiles of rel[0..k-1]; tile_base[n] = n_tiles
  std::vector<EmitChunk> emit_chunks;   // the emit kernel's work: every item's tiles in chunks
  uint64_t n_tiles = 0;
  uint32_t n_src_base = 0;              // pointer table: sources, then destinations
  uint32_t n_dst_base = 0;
  std::vector<uint64_t> obj_bytes;      // per pointer-table slot: object size
  std::vector<uint8_t> obj_use;         // per slot: 1 read, 2 written (0: unused)
  const char* src_name = "src_ptrs";    // caller-side names of the two tables
  const char* dst_name = "dst_ptrs";
  bool interleave = false;
  uint64_t bytes_read = 0;
  uint64_t bytes_written = 0;
  // device state, created on first use: one device allocation carved into
  // the tables, one pinned host buffer for their uploads
  bool ready = false;
  void* d_mem = nullptr;
  size_t d_cap = 0;                     // bytes of d_mem / h_staging as allocated
  size_t h_cap = 0;
  DevRel* d_rel = nullptr;              // uploaded: descriptors, tile prefix, pointer table
  uint64_t* d_tile_base = nullptr;
  uint64_t* d_ptrs = nullptr;
  DevItem* d_items = nullptr;           // built on the device
  DevTile* d_tiles = nullptr;
  unsigned char* h_staging = nullptr;   // pinned: the uploaded part, in the same layout
  uint64_t* h_ptrs = nullptr;           // the pointer-table part of h_staging
  std::vector<uint64_t> bound;          // pointer table of the last bind
  bool bound_valid = false;
  hipEvent_t ev_setup = nullptr;        // tile table, offsets and the first bind written
  hipEvent_t ev_staging = nullptr;      // a later bind done (its copy out of h_staging too)
  hipEvent_t ev_kernel = nullptr;       // last kernel reading d_items
  hipEvent_t ev_bound = nullptr;        // the latest bind: ev_setup or ev_staging (not owned)
};

}  // namespace

struct sr_plan {
  std::vector<sr_tensor> src;
  std::vector<sr_tensor> dst;
  std::vector<sr_piece> pieces;
  std::vector<uint64_t> piece_offset;   // buffer offset, UINT64_MAX for ZERO
  std::vector<uint64_t> peer_bytes;
  int32_t n_peers = 0;
  sr_plan_options opt{};
  Phase pack;
  Phase unpack;
  Phase gather;   // direct source -> destination, no buffers
  // alignment each gather pointer must satisfy: its element size; 0 = the
  // slot is not used by the gather
  std::vector<uint32_t> gather_src_align, gather_dst_align;
  int device = -1;
  // Buffer offsets recomputed on the device: per-peer piece lists (CSR).
  std::vector<uint32_t> peer_begin;
  std::vector<uint32_t> peer_list;
  std::vector<uint64_t> payload;        // per piece, 0 for ZERO
  bool offsets_ready = false;
  void* d_offmem = nullptr;             // carved: offsets, payloads, peer lists
  unsigned char* h_offmem = nullptr;    // pinned upload of payloads and peer lists
  size_t d_offcap = 0;
  size_t h_offcap = 0;
  uint64_t* d_offset = nullptr;
  uint32_t* d_peer_begin = nullptr;
  uint32_t* d_peer_list = nullptr;
  uint64_t* d_payload = nullptr;
  hipEvent_t ev_offsets = nullptr;
};

namespace sr_internal {
PlanView plan_view(const sr_plan* p) {
  return PlanView{p->src.data(), p->src.size(), p->pieces.data(), p->pieces.size(), p->piece_offset.data(),
                  p->peer_bytes.data(), p->n_peers, p->peer_begin.data(), p->peer_list.data()};
}
}  // namespace sr_internal

namespace {

int check_tensor(const sr_tensor& t, const char* what, int32_t idx) {
  if (t.reserved != 0) return fail(SR_EINVAL, "%s[%d]: reserved field must be 0", what, idx);
  const int es = dtype_size(t.dtype);
  if (es == 0) return fail(SR_EINVAL, "%s[%d]: unknown dtype %d", what, idx, t.dtype);
  if (t.rows == 0 || t.cols == 0)
    return fail(SR_EINVAL, "%s[%d]: empty tensor [%llu, %llu]", what, idx,
                (unsigned long long)t.rows, (unsigned long long)t.cols);
  const uint64_t lim = uint64_t(1) << 62;
  uint64_t n, bytes;
  if (__builtin_mul_overflow(t.rows, t.cols, &n) || __builtin_mul_overflow(n, uint64_t(es), &bytes) || bytes > lim)
    return fail(SR_EINVAL, "%s[%d]: tensor too large", what, idx);
  return SR_OK;
}

int check_region(const sr_tensor& t, uint64_t r0, uint64_t c0, uint64_t rows, uint64_t cols,
                 const char* what, int32_t piece) {
  if (r0 > t.rows || rows > t.rows - r0 || c0 > t.cols || cols > t.cols - c0)
    return fail(SR_EBOUNDS,
                "piece %d: %s region rows [%llu,+%llu) cols [%llu,+%llu) outside tensor [%llu, %llu]",
                piece, what, (unsigned long long)r0, (unsigned long long)rows,
                (unsigned long long)c0, (unsigned long long)cols, (unsigned long long)t.rows,
                (unsigned long long)t.cols);
  return SR_OK;
}

struct Box {
  uint64_t r0, r1, c0, c1;
  int32_t piece;
  int32_t slot;   // destination slot written
};

// Every destination slot must be written exactly once: boxes pairwise
// disjoint and their areas summing to the slot's area.  `boxes` holds the
// regions of all slots (any order; sorted here by slot, row, column).
int check_coverage(std::vector<Box>& boxes, const std::vector<sr_tensor>& dst) {
  std::sort(boxes.begin(), boxes.end(), [](const Box& x, const Box& y) {
    if (x.slot != y.slot) return x.slot < y.slot;
    return x.r0 != y.r0 ? x.r0 < y.r0 : x.c0 < y.c0;
  });
  size_t at = 0;
  for (size_t s = 0; s < dst.size(); ++s) {
    size_t end = at;
    while (end < boxes.size() && boxes[end].slot == int32_t(s)) ++end;
    unsigned __int128 area = 0;
    for (size_t i = at; i < end; ++i) {
      const Box& bi = boxes[i];
      area += (unsigned __int128)(bi.r1 - bi.r0) * (bi.c1 - bi.c0);
      for (size_t j = i + 1; j < end && boxes[j].r0 < bi.r1; ++j) {
        if (boxes[j].c0 < bi.c1 && bi.c0 < boxes[j].c1)
          return fail(SR_EOVERLAP, "dst[%zu]: pieces %d and %d write overlapping regions", s, bi.piece,
                      boxes[j].piece);
      }
    }
    const unsigned __int128 full = (unsigned __int128)dst[s].rows * dst[s].cols;
    if (area != full)
      return fail(SR_EOVERLAP, "dst[%zu]: pieces cover %llu of %llu elements", s,
                  (unsigned long long)area, (unsigned long long)full);
    at = end;
  }
  return SR_OK;
}

// Device descriptors of a phase, in `order`.  Pointer-table slots: sources
// first, then destinations (offset by n_src_base).  `buf_src` / `buf_dst`
// mark the side that is a peer buffer (its address is the buffer base plus
// the piece's offset, computed on the device).
//
// With `row_groups`, runs of consecutive strided items that sit side by side
// on the ordering side (the source for pack, the destination otherwise:
// same tensor, rows, row width and stride, each starting where the previous
// one's rows end) form a group whose tiles are dealt out row block by row
// block.  A destination row assembled from several pieces (a dim -1 `cat`)
// is then written by adjacent tiles instead of once per piece, far apart in
// time, so each DRAM page is opened once rather than once per piece.
// Tile size reduction of an item (log2): RECAST items writing both copies.
uint32_t tile_reduce(const HostItem& h) {
  return (h.kind == kKindRecast && h.dst_slot >= 0) ? kRecastTileShift : 0;
}

void build_rel(Phase& ph, const std::vector<uint32_t>& order, uint32_t tile_bytes, bool buf_src,
               bool buf_dst, bool group_by_src, bool row_groups) {
  ph.rel.clear();
  ph.rel.reserve(order.size());
  ph.tile_base.clear();
  ph.tile_base.reserve(order.size() + 1);
  ph.n_tiles = 0;
  for (uint32_t k : order) {
    ph.tile_base.push_back(ph.n_tiles);
    const HostItem& h = ph.items[k];
    DevRel r{};
    r.src_off = h.src_off;
    r.dst_off = h.dst_off;
    r.dst2_off = h.dst2_off;
    r.src_stride = h.src_stride;
    r.dst_stride = h.dst_stride;
    r.dst2_stride = h.dst2_stride;
    r.total = h.rows * h.row_bytes;
    if (h.contiguous) {
      r.row_bytes = 0;
    } else {
      r.row_bytes = uint32_t(h.row_bytes);
      const DivMagic m = div_magic(uint32_t(h.row_bytes));
      r.magic = m.m;
      r.shifts = m.s1 | (m.s2 << 8);
    }
    r.kind = h.kind | (h.esize << 8);
    if (buf_src && h.src_slot >= 0) r.kind |= kRelSrcBuf;
    if (buf_dst && h.dst_slot >= 0) r.kind |= kRelDstBuf;
    const uint32_t reduce = tile_reduce(h);
    r.kind |= reduce << kRelTileShiftBit;
    r.src_slot = h.src_slot;
    r.dst_slot = h.dst_slot >= 0 ? int32_t(ph.n_src_base) + h.dst_slot : -1;
    r.dst2_slot = h.dst2_slot >= 0 ? int32_t(ph.n_src_base) + h.dst2_slot : -1;
    ph.obj_use.resize(size_t(ph.n_src_base) + ph.n_dst_base, 0);
    if (r.src_slot >= 0) ph.obj_use[r.src_slot] |= 1;
    if (r.dst_slot >= 0) ph.obj_use[r.dst_slot] |= 2;
    if (r.dst2_slot >= 0) ph.obj_use[r.dst2_slot] |= 2;
    r.piece = h.piece;
    r.group_size = 1;
    r.group_index = 0;
    ph.rel.push_back(r);
    const uint64_t item_tile = uint64_t(tile_bytes) >> reduce;
    ph.n_tiles += (r.total + item_tile - 1) / item_tile;
  }
  ph.tile_base.push_back(ph.n_tiles);
  ph.emit_chunks.clear();
  for (size_t k = 0; k < ph.rel.size(); ++k) {
    const uint64_t cnt = ph.tile_base[k + 1] - ph.tile_base[k];
    for (uint64_t c = 0; c * kEmitTiles < cnt; ++c) ph.emit_chunks.push_back(EmitChunk{uint32_t(k), uint32_t(c)});
  }
  if (!row_groups) return;
  struct Side {
    int64_t slot;
    uint64_t off, stride, width;
  };
  auto side = [&](const HostItem& h) -> Side {
    if (group_by_src) return {h.src_slot, h.src_off, h.src_stride, h.row_bytes};
    if (h.dst_slot >= 0) return {h.dst_slot, h.dst_off, h.dst_stride, h.row_bytes};
    return {h.dst2_slot, h.dst2_off, h.dst2_stride, h.row_bytes / 2};
  };
  size_t first = 0;
  for (size_t i = 1; i <= order.size(); ++i) {
    bool chain = false;
    if (i < order.size()) {
      const HostItem& a = ph.items[order[i - 1]];
      const HostItem& b = ph.items[order[i]];
      const Side sa = side(a), sb = side(b);
      chain = !a.contiguous && !b.contiguous && a.kind == b.kind && tile_reduce(a) == tile_reduce(b) &&
              a.rows == b.rows &&
              a.row_bytes == b.row_bytes && sa.slot >= 0 && sa.slot == sb.slot &&
              sa.stride == sb.stride && sb.off == sa.off + sa.width;
    }
    if (!chain) {
      const uint32_t m = uint32_t(i - first);
      for (size_t g = first; g < i; ++g) {
        ph.rel[g].group_size = m;
        ph.rel[g].group_index = uint32_t(g - first);
      }
      first = i;
    }
  }
}

// Order a phase's items by the tensor address they start at: the source
// side for pack, the destination side for unpack.  Pieces of one tensor then
// run next to each other (tiles are generated in this order).
std::vector<uint32_t> item_order(const Phase& ph, bool by_src) {
  struct Key {
    int64_t slot;
    uint64_t off;
    uint32_t idx;
  };
  std::vector<Key> keys(ph.items.size());
  for (uint32_t i = 0; i < ph.items.size(); ++i) {
    const HostItem& it = ph.items[i];
    if (by_src) keys[i] = {it.src_slot, it.src_off, i};
    else if (it.dst_slot >= 0) keys[i] = {it.dst_slot, it.dst_off, i};
    else keys[i] = {it.dst2_slot, it.dst2_off * 2, i};
  }
  std::stable_sort(keys.begin(), keys.end(), [](const Key& x, const Key& y) {
    return x.slot != y.slot ? x.slot < y.slot : x.off < y.off;
  });
  std::vector<uint32_t> order(keys.size());
  for (size_t i = 0; i < keys.size(); ++i) order[i] = keys[i].idx;
  return order;
}

// ---------------------------------------------------------------- table memory
//
// One drop-in call builds and destroys several short-lived plans.  Their
// table memory (a device block and a pinned block per phase, one of each for
// the buffer offsets) and their events are kept for reuse instead of being
// freed: each allocation or free costs tens of microseconds on the host and
// hipFree synchronizes the device, and the last launch group of a call waits
// for them.  Blocks come in power-of-two sizes (at least 64 KiB) so plans of
// different sizes share them; at most kCacheDeviceBytes / kCacheHostBytes
// stay cached per process and the rest is freed as before.  A block goes back
// only after the events of the launches that used it have completed.
constexpr size_t kCacheDeviceBytes = size_t(256) << 20;
constexpr size_t kCacheHostBytes = size_t(64) << 20;
constexpr size_t kCacheEvents = 256;

size_t block_class(size_t bytes) {
  size_t c = size_t(64) << 10;
  while (c < bytes) c <<= 1;
  return c;
}

class TableCache {
 public:
  int get(bool pinned, int device, size_t bytes, void** out, size_t* cap) {
    const size_t want = block_class(bytes);
    {
      std::lock_guard<std::mutex> lock(mu_);
      std::vector<Block>& list = pinned ? host_ : dev_;
      for (size_t i = 0; i < list.size(); ++i)
        if (list[i].device == device && list[i].bytes == want) {
          *out = list[i].p;
          *cap = want;
          (pinned ? host_bytes_ : dev_bytes_) -= want;
          list[i] = list.back();
          list.pop_back();
          return SR_OK;
        }
    }
    if (pinned) SR_HIP_TRY(hipHostMalloc(out, want, hipHostMallocDefault));
    else SR_HIP_TRY(hipMalloc(out, want));
    *cap = want;
    return SR_OK;
  }

  void put(bool pinned, int device, void* p, size_t cap) {
    if (!p) return;
    {
      std::lock_guard<std::mutex> lock(mu_);
      size_t& held = pinned ? host_bytes_ : dev_bytes_;
      if (held + cap <= (pinned ? kCacheHostBytes : kCacheDeviceBytes)) {
        (pinned ? host_ : dev_).push_back(Block{p, cap, device});
        held += cap;
        return;
      }
    }
    if (pinned) (void)hipHostFree(p);
    else (void)hipFree(p);
  }

  // Events are created on the current device, which must be `device`.
  int get_event(int device, hipEvent_t* ev) {
    {
      std::lock_guard<std::mutex> lock(mu_);
      for (size_t i = events_.size(); i-- > 0;)
        if (events_[i].first == device) {
          *ev = events_[i].second;
          events_.erase(events_.begin() + i);
          return SR_OK;
        }
    }
    SR_HIP_TRY(hipEventCreateWithFlags(ev, hipEventDisableTiming));
    return SR_OK;
  }

  // One stream per device for the first-use setup of plans (table uploads,
  // tile scan/emit, first bind): default priority, non-blocking, kept for
  // the process.  It lets a launch group's setup run while the previous
  // group's copy kernel still occupies the caller's stream.
  int setup_stream(int device, hipStream_t* out) {
    std::lock_guard<std::mutex> lock(mu_);
    for (const auto& ds : streams_)
      if (ds.first == device) {
        *out = ds.second;
        return SR_OK;
      }
    hipStream_t s = nullptr;
    SR_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    streams_.emplace_back(device, s);
    *out = s;
    return SR_OK;
  }

  void put_event(int device, hipEvent_t ev) {
    if (!ev) return;
    {
      std::lock_guard<std::mutex> lock(mu_);
      if (events_.size() < kCacheEvents) {
        events_.emplace_back(device, ev);
        return;
      }
    }
    (void)hipEventDestroy(ev);
  }

 private:
  struct Block {
    void* p;
    size_t bytes;
    int device;
  };
  std::mutex mu_;
  std::vector<Block> dev_, host_;
  std::vector<std::pair<int, hipEvent_t>> events_;
  std::vector<std::pair<int, hipStream_t>> streams_;
  size_t dev_bytes_ = 0, host_bytes_ = 0;
};

// Never destroyed: cached blocks live until the process exits, so no HIP call
// runs from a static destructor after the runtime may have shut down.
TableCache& table_cache() {
  static TableCache* cache = new TableCache();
  return *cache;
}

int ensure_device(sr_plan* p) {
  int dev = -1;
  SR_HIP_TRY(hipGetDevice(&dev));
  if (p->device < 0) {
    p->device = dev;
  } else if (p->device != dev) {
    return fail(SR_EINVAL, "plan was first used on device %d, current device is %d", p->device, dev);
  }
  return SR_OK;
}

enum PhaseKind { kPack, kUnpack, kGather };

// Next 256-byte aligned offset for a carved sub-buffer of `bytes`.
size_t carve(size_t& end, size_t bytes) {
  const size_t at = (end + 255) & ~size_t(255);
  end = at + bytes;
  return at;
}

// Per-peer buffer offsets on the device (shared by pack and unpack).  The
// inputs go up asynchronously on `stream` from pinned memory, so the call
// never waits for earlier work on the stream.
int setup_offsets(sr_plan* p, hipStream_t stream) {
  if (p->offsets_ready) return SR_OK;
  int rc;
  if (!p->ev_offsets && (rc = table_cache().get_event(p->device, &p->ev_offsets)) != SR_OK) return rc;
  if (p->n_peers > 0 && !p->peer_list.empty()) {
    const size_t np = p->pieces.size();
    size_t in_end = 0;   // layout of the uploaded part: payloads, peer_begin, peer_list
    const size_t o_pay = carve(in_end, np * sizeof(uint64_t));
    const size_t o_beg = carve(in_end, p->peer_begin.size() * sizeof(uint32_t));
    const size_t o_lst = carve(in_end, p->peer_list.size() * sizeof(uint32_t));
    size_t dev_end = in_end;
    const size_t o_off = carve(dev_end, np * sizeof(uint64_t));
    // allocations survive a failed attempt and are reused by the retry
    if (!p->d_offmem && (rc = table_cache().get(false, p->device, dev_end, &p->d_offmem, &p->d_offcap)) != SR_OK)
      return rc;
    if (!p->h_offmem &&
        (rc = table_cache().get(true, p->device, in_end, reinterpret_cast<void**>(&p->h_offmem),
                                &p->h_offcap)) != SR_OK)
      return rc;
    unsigned char* d = static_cast<unsigned char*>(p->d_offmem);
    p->d_payload = reinterpret_cast<uint64_t*>(d + o_pay);
    p->d_peer_begin = reinterpret_cast<uint32_t*>(d + o_beg);
    p->d_peer_list = reinterpret_cast<uint32_t*>(d + o_lst);
    p->d_offset = reinterpret_cast<uint64_t*>(d + o_off);
    std::memcpy(p->h_offmem + o_pay, p->payload.data(), np * sizeof(uint64_t));
    std::memcpy(p->h_offmem + o_beg, p->peer_begin.data(), p->peer_begin.size() * sizeof(uint32_t));
    std::memcpy(p->h_offmem + o_lst, p->peer_list.data(), p->peer_list.size() * sizeof(uint32_t));
    SR_HIP_TRY(hipMemcpyAsync(p->d_offmem, p->h_offmem, in_end, hipMemcpyHostToDevice, stream));
    hipLaunchKernelGGL(sr_offsets_kernel, dim3(uint32_t(p->n_peers)), dim3(kSetupBlock), 0, stream,
                       p->d_peer_begin, p->d_peer_list, p->d_payload, p->d_offset);
    SR_HIP_TRY(hipGetLastError());
  }
  SR_HIP_TRY(hipEventRecord(p->ev_offsets, stream));
  p->offsets_ready = true;
  return SR_OK;
}

// First use of a phase: its descriptors, tile prefix and pointer table go
// up in one copy from pinned memory, then one kernel builds the tile table
// and binds the items to `ptrs`, stream-ordered on `stream`.  With
// `mark`, ev_setup marks completion (for a copy kernel on another stream);
// else the phase's next copy kernel follows on `stream` and its ev_kernel
// stands for the bind.
int setup_phase(sr_plan* p, Phase& ph, bool needs_offsets, const std::vector<uint64_t>& ptrs,
                hipStream_t stream, bool mark) {
  if (ph.ready) return SR_OK;
  TableCache& cache = table_cache();
  int rc;
  if (mark && !ph.ev_setup && (rc = cache.get_event(p->device, &ph.ev_setup)) != SR_OK) return rc;
  if (!ph.ev_kernel && (rc = cache.get_event(p->device, &ph.ev_kernel)) != SR_OK) return rc;
  const uint32_t n = uint32_t(ph.rel.size());
  if (n > 0) {
    const size_t nptr = std::max<size_t>(1, size_t(ph.n_src_base) + ph.n_dst_base);
    size_t end = 0;   // the first three are uploaded (pinned staging, same layout)
    const size_t o_rel = carve(end, n * sizeof(DevRel));
    const size_t o_base = carve(end, (size_t(n) + 1) * sizeof(uint64_t));
    const size_t o_chunk = carve(end, ph.emit_chunks.size() * sizeof(EmitChunk));
    const size_t o_ptr = carve(end, nptr * sizeof(uint64_t));
    const size_t up_end = o_ptr + nptr * sizeof(uint64_t);
    const size_t o_items = carve(end, n * sizeof(DevItem));
    const size_t o_tiles = carve(end, ph.n_tiles * sizeof(DevTile));
    // allocations survive a failed attempt and are reused by the retry
    if (!ph.d_mem && (rc = cache.get(false, p->device, end, &ph.d_mem, &ph.d_cap)) != SR_OK) return rc;
    if (!ph.h_staging &&
        (rc = cache.get(true, p->device, up_end, reinterpret_cast<void**>(&ph.h_staging), &ph.h_cap)) != SR_OK)
      return rc;
    unsigned char* d = static_cast<unsigned char*>(ph.d_mem);
    ph.d_rel = reinterpret_cast<DevRel*>(d + o_rel);
    ph.d_tile_base = reinterpret_cast<uint64_t*>(d + o_base);
    ph.d_ptrs = reinterpret_cast<uint64_t*>(d + o_ptr);
    ph.d_items = reinterpret_cast<DevItem*>(d + o_items);
    ph.d_tiles = reinterpret_cast<DevTile*>(d + o_tiles);
    ph.h_ptrs = reinterpret_cast<uint64_t*>(ph.h_staging + o_ptr);
    std::memcpy(ph.h_staging + o_rel, ph.rel.data(), n * sizeof(DevRel));
    std::memcpy(ph.h_staging + o_base, ph.tile_base.data(), (size_t(n) + 1) * sizeof(uint64_t));
    std::memcpy(ph.h_staging + o_chunk, ph.emit_chunks.data(), ph.emit_chunks.size() * sizeof(EmitChunk));
    std::memcpy(ph.h_ptrs, ptrs.data(), ptrs.size() * sizeof(uint64_t));
    SR_HIP_TRY(hipMemcpyAsync(ph.d_mem, ph.h_staging, up_end, hipMemcpyHostToDevice, stream));
    if (needs_offsets) {
      rc = setup_offsets(p, stream);
      if (rc != SR_OK) return rc;
      SR_HIP_TRY(hipStreamWaitEvent(stream, p->ev_offsets, 0));
    }
    const uint32_t shift = log2u(p->opt.tile_bytes);
    const uint32_t n_chunks = uint32_t(ph.emit_chunks.size());
    hipLaunchKernelGGL(sr_tile_emit_kernel, dim3(std::min<uint32_t>(n_chunks, 65535u)), dim3(kSetupBlock), 0,
                       stream, ph.d_rel, ph.d_tile_base, reinterpret_cast<const EmitChunk*>(d + o_chunk), n_chunks,
                       shift, ph.n_tiles, ph.interleave ? kXcds : 1u, ph.d_tiles, ph.d_ptrs, p->d_offset,
                       ph.d_items);
    SR_HIP_TRY(hipGetLastError());
  }
  if (mark) {
    SR_HIP_TRY(hipEventRecord(ph.ev_setup, stream));
    ph.ev_bound = ph.ev_setup;
  } else {
    ph.ev_bound = ph.ev_kernel;   // recorded after the copy kernel, which follows on `stream`
  }
  ph.bound = ptrs;
  ph.bound_valid = true;
  ph.ready = true;
  return SR_OK;
}

// One launch reads and writes the caller's objects concurrently: objects it
// writes must be pairwise disjoint and must not overlap any object it reads.
int check_disjoint(const Phase& ph, const std::vector<uint64_t>& ptrs) {
  struct Span {
    uint64_t lo, hi;
    size_t slot;
  };
  std::vector<Span> w, r;
  for (size_t i = 0; i < ph.obj_use.size(); ++i) {
    if (!ph.obj_use[i]) continue;
    const Span sp{ptrs[i], ptrs[i] + ph.obj_bytes[i], i};
    if (ph.obj_use[i] & 2) w.push_back(sp);
    if (ph.obj_use[i] & 1) r.push_back(sp);
  }
  auto name = [&](size_t slot, char* buf, size_t n) {
    if (slot < ph.n_src_base) snprintf(buf, n, "%s[%zu]", ph.src_name, slot);
    else snprintf(buf, n, "%s[%zu]", ph.dst_name, slot - ph.n_src_base);
    return buf;
  };
  char a[64], b[64];
  std::sort(w.begin(), w.end(), [](const Span& x, const Span& y) { return x.lo < y.lo; });
  for (size_t k = 1; k < w.size(); ++k)
    if (w[k].lo < w[k - 1].hi)
      return fail(SR_EOVERLAP, "%s and %s are written by one launch and overlap",
                  name(w[k - 1].slot, a, sizeof a), name(w[k].slot, b, sizeof b));
  for (const Span& x : r) {
    // the written span starting last below x.hi is the only candidate
    auto it = std::lower_bound(w.begin(), w.end(), x.hi,
                               [](const Span& s, uint64_t v) { return s.lo < v; });
    if (it != w.begin() && std::prev(it)->hi > x.lo)
      return fail(SR_EOVERLAP, "%s is read while %s, which overlaps it, is written",
                  name(x.slot, a, sizeof a), name(std::prev(it)->slot, b, sizeof b));
  }
  return SR_OK;
}

int run_phase(sr_plan* p, Phase& ph, PhaseKind kind, const std::vector<uint64_t>& ptrs,
              hipStream_t stream) {
  if (ph.rel.empty()) return SR_OK;
  const bool rebind = !ph.bound_valid || ptrs != ph.bound;
  int rc;
  if (rebind && (rc = check_disjoint(ph, ptrs)) != SR_OK) return rc;
  rc = ensure_device(p);
  if (rc != SR_OK) return rc;
  const uint32_t n = uint32_t(ph.rel.size());
  if (!ph.ready) {
    // A phase's first use builds its tables and binds the pointers.  They
    // are the library's own memory and read no caller data: while earlier
    // work on `stream` (such as the previous launch group's copy) is still
    // going, a large phase's setup runs beside it on the device's setup
    // stream; on an idle `stream`, or for a small phase, it runs on
    // `stream` directly, since a wait across streams costs the host more
    // than the setup kernel takes on the GPU.
    hipStream_t setup = stream;
    if (ph.n_tiles > kInlineSetupTiles) {
      const hipError_t busy = hipStreamQuery(stream);
      (void)hipGetLastError();   // "not ready" is an answer, not an error
      if (busy != hipSuccess && busy != hipErrorNotReady)
        return fail(SR_EHIP, "hipStreamQuery failed: %s", hipGetErrorString(busy));
      if (busy == hipErrorNotReady && (rc = table_cache().setup_stream(p->device, &setup)) != SR_OK) return rc;
    }
    rc = setup_phase(p, ph, kind != kGather, ptrs, setup, setup != stream);
    if (rc != SR_OK) return rc;
    if (setup != stream) SR_HIP_TRY(hipStreamWaitEvent(stream, ph.ev_setup, 0));
  } else if (rebind) {
    // Later rebinds run on `stream`, after the latest bind (whose copy out
    // of the staging buffer must be done before the host rewrites it) and
    // after the phase's previous launch (which may still read the item and
    // pointer tables).
    if (!ph.ev_staging && (rc = table_cache().get_event(p->device, &ph.ev_staging)) != SR_OK) return rc;
    SR_HIP_TRY(hipEventSynchronize(ph.ev_bound));
    std::memcpy(ph.h_ptrs, ptrs.data(), ptrs.size() * sizeof(uint64_t));
    SR_HIP_TRY(hipStreamWaitEvent(stream, ph.ev_bound, 0));
    SR_HIP_TRY(hipStreamWaitEvent(stream, ph.ev_kernel, 0));
    SR_HIP_TRY(hipMemcpyAsync(ph.d_ptrs, ph.h_ptrs, ptrs.size() * sizeof(uint64_t), hipMemcpyHostToDevice,
                              stream));
    hipLaunchKernelGGL(sr_bind_kernel, dim3((n + kSetupBlock - 1) / kSetupBlock), dim3(kSetupBlock), 0,
                       stream, ph.d_rel, n, ph.d_ptrs, p->d_offset, ph.d_items);
    SR_HIP_TRY(hipGetLastError());
    SR_HIP_TRY(hipEventRecord(ph.ev_staging, stream));
    ph.ev_bound = ph.ev_staging;
    ph.bound = ptrs;
    ph.bound_valid = true;
  } else {
    // the latest bind (which follows the tables on its stream)
    SR_HIP_TRY(hipStreamWaitEvent(stream, ph.ev_bound, 0));
  }

  const uint32_t n_tiles = uint32_t(ph.n_tiles);
  uint32_t grid = n_tiles;
  if (p->opt.max_blocks != 0) grid = std::min(grid, p->opt.max_blocks);
  grid = std::min(grid, kMaxGrid);
  // A capped grid strides over the tile list; a multiple of the interleave
  // width keeps every position on the XCD the interleave placed it for.
  if (ph.interleave && grid < n_tiles && grid >= kXcds) grid -= grid % kXcds;
  const bool nt = (p->opt.flags & SR_OPT_TEMPORAL) == 0;
  typedef void (*KernelFn)(const DevItem*, const DevTile*, uint32_t);
  KernelFn fn;
  switch (kind) {
    case kPack: fn = nt ? sr_pack_kernel<true> : sr_pack_kernel<false>; break;
    case kUnpack: fn = nt ? sr_unpack_kernel<true> : sr_unpack_kernel<false>; break;
    default: fn = nt ? sr_gather_kernel<true> : sr_gather_kernel<false>; break;
  }
  hipLaunchKernelGGL(fn, dim3(grid), dim3(kBlock), 0, stream, ph.d_items, ph.d_tiles, n_tiles);
  SR_HIP_TRY(hipGetLastError());
  SR_HIP_TRY(hipEventRecord(ph.ev_kernel, stream));
  return SR_OK;
}

// Releases a phase's device tables (to the table cache).  Waits first for
// the last launches that read them (bind, copy kernel, setup), so a plan can
// be destroyed right after an asynchronous call.
void free_phase(Phase& ph, int device) {
  TableCache& cache = table_cache();
  for (hipEvent_t ev : {ph.ev_kernel, ph.ev_staging, ph.ev_setup})
    if (ev) (void)hipEventSynchronize(ev);
  cache.put(false, device, ph.d_mem, ph.d_cap);
  cache.put(true, device, ph.h_staging, ph.h_cap);
  for (hipEvent_t ev : {ph.ev_setup, ph.ev_staging, ph.ev_kernel}) cache.put_event(device, ev);
  ph = Phase();
}

// The phase's pointer table: source objects, then destination objects.
std::vector<uint64_t> pointer_table(const void* const* a, size_t na, const void* const* b, size_t nb) {
  std::vector<uint64_t> t(na + nb, 0);
  for (size_t i = 0; i < na; ++i) t[i] = reinterpret_cast<uintptr_t>(a ? a[i] : nullptr);
  for (size_t i = 0; i < nb; ++i) t[na + i] = reinterpret_cast<uintptr_t>(b ? b[i] : nullptr);
  return t;
}

int check_ptrs(const void* const* ptrs, size_t n, const std::vector<uint32_t>& align,
               const char* what) {
  if (n > 0 && ptrs == nullptr) return fail(SR_EINVAL, "%s: pointer array is null", what);
  for (size_t i = 0; i < n; ++i) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(ptrs[i]);
    if (align[i] == 0) continue;   // slot unused by this phase
    if (a == 0) return fail(SR_EINVAL, "%s[%zu] is null", what, i);
    if (a & (align[i] - 1))   // element sizes: powers of two
      return fail(SR_EALIGN, "%s[%zu] = %p is not %u-byte aligned", what, i, ptrs[i], align[i]);
  }
  return SR_OK;
}

// Alignment each pointer of a gather must satisfy: its element size; 0 =
// the slot is not used by the phase.  Computed once, when the plan is made.
void gather_alignment(sr_plan* plan) {
  std::vector<uint32_t>& sal = plan->gather_src_align;
  std::vector<uint32_t>& dal = plan->gather_dst_align;
  sal.assign(plan->src.size(), 0);
  dal.assign(plan->dst.size(), 0);
  for (const sr_piece& pc : plan->pieces) {
    if (pc.src >= 0) sal[pc.src] = dtype_size(plan->src[pc.src].dtype);
    if (pc.dst >= 0) dal[pc.dst] = dtype_size(plan->dst[pc.dst].dtype);
    if (pc.dst2 >= 0) dal[pc.dst2] = dtype_size(plan->dst[pc.dst2].dtype);
  }
}

}  // namespace

// ------------------------------------------------------- allocation-free gather
// The device tables of sr_gather_noalloc live in this array, one copy per GPU,
// allocated with the code object when the library is loaded on a device and
// held until the process exits.  On the host, `scratch` names a stand-in, not
// device memory: host code never passes it to a kernel or a copy, only the
// per-device address that hipGetSymbolAddress returns (scratch_base below).
static __device__ __align__(256) unsigned char scratch[SR_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 256;
std::mutex g_scratch_mu;
uint64_t g_scratch_addr[kMaxScratchDevices];   // 0 = not looked up yet

// Address of `scratch` on the current device `device`, looked up once per
// device (with that device current, as hipGetSymbolAddress requires).
int scratch_base(int device, unsigned char** out) {
  if (device < 0 || device >= kMaxScratchDevices)
    return fail(SR_EINVAL, "device %d out of range for the scratch table", device);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[device] == 0) {
    void* p = nullptr;
    SR_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (p == nullptr) return fail(SR_EHIP, "hipGetSymbolAddress(scratch) returned null on device %d", device);
    g_scratch_addr[device] = reinterpret_cast<uintptr_t>(p);
  }
  *out = reinterpret_cast<unsigned char*>(g_scratch_addr[device]);
  return SR_OK;
}

// Where the gather phase's tables sit in the scratch, and how much it needs.
struct ScratchLayout {
  size_t rel, ptrs, items, base, chunks, tiles, end;
};

ScratchLayout scratch_layout(const Phase& ph) {
  const size_t n = ph.rel.size();
  const size_t nptr = std::max<size_t>(1, size_t(ph.n_src_base) + ph.n_dst_base);
  ScratchLayout L{};
  size_t end = 0;
  L.rel = carve(end, n * sizeof(DevRel));
  L.base = carve(end, (n + 1) * sizeof(uint64_t));
  L.chunks = carve(end, ph.emit_chunks.size() * sizeof(EmitChunk));
  L.ptrs = carve(end, nptr * sizeof(uint64_t));
  L.items = carve(end, n * sizeof(DevItem));
  L.tiles = carve(end, size_t(ph.n_tiles) * sizeof(DevTile));
  L.end = end;
  return L;
}

}  // namespace

// ------------------------------------------------------------------ C ABI

extern "C" {

int sr_abi_version(void) { return SR_ABI_VERSION; }

const char* sr_last_error(void) { return sr_internal::last_error(); }

int sr_selftest(void) {
  // Division constants: exhaustive small divisors, then edge divisors, each
  // against numerators at the edges of the range and a pseudo-random sweep.
  uint64_t x = 0x9E3779B97F4A7C15ull;
  auto rnd = [&x]() {
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    return uint32_t(x >> 16);
  };
  std::vector<uint32_t> divisors;
  for (uint32_t d = 1; d <= 4096; ++d) divisors.push_back(d);
  for (uint32_t s = 12; s < 31; ++s) {
    divisors.push_back((1u << s) - 1);
    divisors.push_back(1u << s);
    divisors.push_back((1u << s) + 1);
    divisors.push_back((1u << s) * 3 / 2);
  }
  divisors.push_back(0x7fffffffu);
  for (uint32_t d : divisors) {
    const DivMagic m = div_magic(d);
    const uint32_t edge[] = {0u, 1u, d - 1, d, d + 1, 2 * d - 1, 0x7fffffffu, 0x80000000u,
                             0xfffffffeu, 0xffffffffu};
    for (uint32_t n : edge) {
      if (div_apply(n, m.m, m.s1, m.s2) != n / d)
        return fail(SR_EINVAL, "selftest: %u / %u gave %u", n, d, div_apply(n, m.m, m.s1, m.s2));
    }
    for (int k = 0; k < 64; ++k) {
      const uint32_t n = rnd();
      if (div_apply(n, m.m, m.s1, m.s2) != n / d)
        return fail(SR_EINVAL, "selftest: %u / %u gave %u", n, d, div_apply(n, m.m, m.s1, m.s2));
    }
  }
  return SR_OK;
}

int sr_plan_create(const sr_tensor* src_tensors, int32_t n_src, const sr_tensor* dst_tensors,
                   int32_t n_dst, int32_t n_peers, const sr_piece* pieces, int32_t n_pieces,
                   const sr_plan_options* options, sr_plan** out_plan) {
  if (out_plan == nullptr) return fail(SR_EINVAL, "out_plan is null");
  *out_plan = nullptr;
  if (n_src < 0 || n_dst < 0 || n_peers < 0 || n_pieces < 0)
    return fail(SR_EINVAL, "negative count (n_src=%d n_dst=%d n_peers=%d n_pieces=%d)", n_src,
                n_dst, n_peers, n_pieces);
  if ((n_src > 0 && !src_tensors) || (n_dst > 0 && !dst_tensors) || (n_pieces > 0 && !pieces))
    return fail(SR_EINVAL, "null array with non-zero count");

  sr_plan_options opt{};
  if (options) opt = *options;
  if (opt.reserved != 0) return fail(SR_EINVAL, "options.reserved must be 0");
  if (opt.flags & ~(SR_OPT_TEMPORAL | SR_OPT_SKIP_COVERAGE | SR_OPT_PIECE_ORDER | SR_OPT_NO_XCD_INTERLEAVE |
                    SR_OPT_NO_ROW_GROUPS | SR_OPT_GATHER_ONLY))
    return fail(SR_EINVAL, "unknown option flags 0x%x", opt.flags);
  if (opt.tile_bytes == 0) opt.tile_bytes = kDefaultTileBytes;
  if (opt.tile_bytes < 4096 || opt.tile_bytes > (16u << 20) ||
      (opt.tile_bytes & (opt.tile_bytes - 1)))
    return fail(SR_EINVAL, "tile_bytes %u must be a power of two in [4096, 16 MiB]",
                opt.tile_bytes);

  int rc;
  for (int32_t i = 0; i < n_src; ++i)
    if ((rc = check_tensor(src_tensors[i], "src", i)) != SR_OK) return rc;
  for (int32_t i = 0; i < n_dst; ++i)
    if ((rc = check_tensor(dst_tensors[i], "dst", i)) != SR_OK) return rc;

  sr_plan* p = new (std::nothrow) sr_plan();
  if (!p) return fail(SR_ENOMEM, "out of host memory");
  p->src.assign(src_tensors, src_tensors + n_src);
  p->dst.assign(dst_tensors, dst_tensors + n_dst);
  p->pieces.assign(pieces, pieces + n_pieces);
  p->n_peers = n_peers;
  p->opt = opt;
  p->piece_offset.assign(n_pieces, UINT64_MAX);
  p->peer_bytes.assign(n_peers, 0);

  std::vector<Box> cover;   // every destination region, for the coverage check
  cover.reserve(size_t(n_pieces) * 2);
  const uint64_t max_row = (uint64_t(1) << 31) - opt.tile_bytes;
  const bool buffers = (opt.flags & SR_OPT_GATHER_ONLY) == 0;   // build the pack and unpack phases
  if (buffers) {
    p->pack.items.reserve(size_t(n_pieces));
    p->unpack.items.reserve(size_t(n_pieces));
  }
  p->gather.items.reserve(size_t(n_pieces));

  for (int32_t k = 0; k < n_pieces; ++k) {
    const sr_piece& pc = pieces[k];
    auto bad = [&](int code) {
      delete p;
      return code;
    };
    if (pc.reserved != 0) return bad(fail(SR_EINVAL, "piece %d: reserved field must be 0", k));
    if (pc.rows == 0 || pc.cols == 0) return bad(fail(SR_EINVAL, "piece %d: empty region", k));
    if (pc.kind != SR_PIECE_COPY && pc.kind != SR_PIECE_RECAST && pc.kind != SR_PIECE_ZERO)
      return bad(fail(SR_EINVAL, "piece %d: unknown kind %d", k, pc.kind));

    if (pc.kind == SR_PIECE_ZERO) {
      if (pc.src != -1 || pc.dst2 != -1)
        return bad(fail(SR_EINVAL, "piece %d: ZERO takes no src/dst2", k));
      if (pc.dst < 0 || pc.dst >= n_dst) return bad(fail(SR_EINVAL, "piece %d: bad dst slot %d", k, pc.dst));
      const sr_tensor& dt = p->dst[pc.dst];
      if ((rc = check_region(dt, pc.dst_row, pc.dst_col, pc.rows, pc.cols, "dst", k)) != SR_OK) return bad(rc);
      const uint32_t es = dtype_size(dt.dtype);
      HostItem it{};
      it.kind = kKindZero;
      it.src_slot = -1;
      it.dst_slot = pc.dst;
      it.dst2_slot = -1;
      it.dst_off = (pc.dst_row * dt.cols + pc.dst_col) * es;
      it.dst_stride = dt.cols * es;
      it.rows = pc.rows;
      it.row_bytes = pc.cols * es;
      it.esize = es;
      it.piece = k;
      it.contiguous = pc.rows == 1 || it.dst_stride == it.row_bytes;
      if (it.contiguous) {
        it.row_bytes *= it.rows;
        it.rows = 1;
      } else if (it.row_bytes > max_row) {
        return bad(fail(SR_EINVAL, "piece %d: strided row of %llu bytes too wide", k,
                        (unsigned long long)it.row_bytes));
      }
      if (buffers) p->unpack.items.push_back(it);
      p->unpack.bytes_written += pc.rows * pc.cols * es;
      p->gather.items.push_back(it);
      p->gather.bytes_written += pc.rows * pc.cols * es;
      cover.push_back({pc.dst_row, pc.dst_row + pc.rows, pc.dst_col, pc.dst_col + pc.cols, k, pc.dst});
      continue;
    }

    if (pc.src < 0 || pc.src >= n_src) return bad(fail(SR_EINVAL, "piece %d: bad src slot %d", k, pc.src));
    if (pc.peer < 0 || pc.peer >= n_peers) return bad(fail(SR_EINVAL, "piece %d: bad peer %d", k, pc.peer));
    const sr_tensor& st = p->src[pc.src];
    if ((rc = check_region(st, pc.src_row, pc.src_col, pc.rows, pc.cols, "src", k)) != SR_OK) return bad(rc);
    const uint32_t es = dtype_size(st.dtype);

    int32_t dst = pc.dst, dst2 = -1;
    if (pc.kind == SR_PIECE_COPY) {
      if (pc.dst2 != -1) return bad(fail(SR_EINVAL, "piece %d: COPY takes no dst2", k));
      if (dst < 0 || dst >= n_dst) return bad(fail(SR_EINVAL, "piece %d: bad dst slot %d", k, dst));
      if (p->dst[dst].dtype != st.dtype)
        return bad(fail(SR_EDTYPE, "piece %d: src dtype %d != dst dtype %d", k, st.dtype, p->dst[dst].dtype));
    } else {
      dst2 = pc.dst2;
      if (st.dtype != SR_DT_F32) return bad(fail(SR_EDTYPE, "piece %d: RECAST source must be f32", k));
      if (dst2 < 0 || dst2 >= n_dst) return bad(fail(SR_EINVAL, "piece %d: bad dst2 slot %d", k, dst2));
      if (p->dst[dst2].dtype != SR_DT_BF16)
        return bad(fail(SR_EDTYPE, "piece %d: RECAST dst2 must be bf16", k));
      if (dst < -1 || dst >= n_dst) return bad(fail(SR_EINVAL, "piece %d: bad dst slot %d", k, dst));
      if (dst >= 0 && p->dst[dst].dtype != SR_DT_F32)
        return bad(fail(SR_EDTYPE, "piece %d: RECAST dst must be f32", k));
      if (dst == dst2) return bad(fail(SR_EINVAL, "piece %d: dst and dst2 are the same slot", k));
      if ((rc = check_region(p->dst[dst2], pc.dst_row, pc.dst_col, pc.rows, pc.cols, "dst2", k)) != SR_OK)
        return bad(rc);
      cover.push_back({pc.dst_row, pc.dst_row + pc.rows, pc.dst_col, pc.dst_col + pc.cols, k, dst2});
    }
    if (dst >= 0) {
      if ((rc = check_region(p->dst[dst], pc.dst_row, pc.dst_col, pc.rows, pc.cols, "dst", k)) != SR_OK)
        return bad(rc);
      cover.push_back({pc.dst_row, pc.dst_row + pc.rows, pc.dst_col, pc.dst_col + pc.cols, k, dst});
    }

    // Buffer placement: pieces of a peer in piece order, 256-byte aligned.
    const uint64_t payload = pc.rows * pc.cols * es;
    uint64_t& cur = p->peer_bytes[pc.peer];
    const uint64_t off = (cur + kBufAlign - 1) / kBufAlign * kBufAlign;
    p->piece_offset[k] = off;
    cur = off + payload;

    // Pack item: source region -> contiguous payload.
    HostItem pk{};
    pk.kind = kKindCopy;
    pk.src_slot = pc.src;
    pk.dst_slot = pc.peer;
    pk.dst2_slot = -1;
    pk.src_off = (pc.src_row * st.cols + pc.src_col) * es;
    pk.src_stride = st.cols * es;
    pk.dst_off = off;
    pk.rows = pc.rows;
    pk.row_bytes = pc.cols * es;
    pk.dst_stride = pk.row_bytes;
    pk.esize = es;
    pk.piece = k;
    pk.contiguous = pc.rows == 1 || pk.src_stride == pk.row_bytes;
    if (pk.contiguous) {
      pk.row_bytes *= pk.rows;
      pk.rows = 1;
    } else if (pk.row_bytes > max_row) {
      return bad(fail(SR_EINVAL, "piece %d: strided row of %llu bytes too wide", k,
                      (unsigned long long)pk.row_bytes));
    }
    if (buffers) p->pack.items.push_back(pk);
    p->pack.bytes_read += payload;
    p->pack.bytes_written += payload;

    // Unpack item: contiguous payload -> destination region(s).
    HostItem up{};
    up.kind = pc.kind == SR_PIECE_COPY ? kKindCopy : kKindRecast;
    up.src_slot = pc.peer;
    up.dst_slot = dst;
    up.dst2_slot = dst2;
    up.src_off = off;
    up.rows = pc.rows;
    up.row_bytes = pc.cols * es;
    up.src_stride = up.row_bytes;
    up.esize = es;
    up.piece = k;
    if (dst >= 0) {
      up.dst_off = (pc.dst_row * p->dst[dst].cols + pc.dst_col) * es;
      up.dst_stride = p->dst[dst].cols * es;
    }
    if (dst2 >= 0) {
      up.dst2_off = (pc.dst_row * p->dst[dst2].cols + pc.dst_col) * 2;
      up.dst2_stride = p->dst[dst2].cols * 2;
    }
    up.contiguous = pc.rows == 1 || ((dst < 0 || up.dst_stride == up.row_bytes) &&
                                     (dst2 < 0 || up.dst2_stride * 2 == up.row_bytes));
    if (up.contiguous) {
      up.row_bytes *= up.rows;
      up.rows = 1;
    } else if (up.row_bytes > max_row) {
      return bad(fail(SR_EINVAL, "piece %d: strided row of %llu bytes too wide", k,
                      (unsigned long long)up.row_bytes));
    }
    if (buffers) p->unpack.items.push_back(up);
    p->unpack.bytes_read += payload;
    if (dst >= 0) p->unpack.bytes_written += payload;
    if (dst2 >= 0) p->unpack.bytes_written += payload / 2;

    // Gather item: source region -> destination region(s), no buffer.
    HostItem ga = up;
    ga.src_slot = pc.src;
    ga.src_off = pk.src_off;
    ga.src_stride = st.cols * es;
    ga.rows = pc.rows;
    ga.row_bytes = pc.cols * es;
    ga.contiguous = pc.rows == 1 ||
                    (ga.src_stride == ga.row_bytes && (dst < 0 || ga.dst_stride == ga.row_bytes) &&
                     (dst2 < 0 || ga.dst2_stride * 2 == ga.row_bytes));
    if (ga.contiguous) {
      ga.row_bytes *= ga.rows;
      ga.rows = 1;
    } else if (ga.row_bytes > max_row) {
      return bad(fail(SR_EINVAL, "piece %d: strided row of %llu bytes too wide", k,
                      (unsigned long long)ga.row_bytes));
    }
    p->gather.items.push_back(ga);
    p->gather.bytes_read += payload;
    if (dst >= 0) p->gather.bytes_written += payload;
    if (dst2 >= 0) p->gather.bytes_written += payload / 2;
  }

  if (!(opt.flags & SR_OPT_SKIP_COVERAGE)) {
    if ((rc = check_coverage(cover, p->dst)) != SR_OK) {
      delete p;
      return rc;
    }
  }
  {
    auto identity = [](size_t n) {
      std::vector<uint32_t> o(n);
      for (uint32_t i = 0; i < n; ++i) o[i] = i;
      return o;
    };
    const bool by_piece = (opt.flags & SR_OPT_PIECE_ORDER) != 0;
    p->pack.n_src_base = uint32_t(n_src);
    p->pack.n_dst_base = uint32_t(n_peers);
    p->unpack.n_src_base = uint32_t(n_peers);
    p->unpack.n_dst_base = uint32_t(n_dst);
    p->gather.n_src_base = uint32_t(n_src);
    p->gather.n_dst_base = uint32_t(n_dst);
    const bool groups = !(opt.flags & SR_OPT_NO_ROW_GROUPS);
    if (buffers) {
      build_rel(p->pack, by_piece ? identity(p->pack.items.size()) : item_order(p->pack, true),
                opt.tile_bytes, false, true, true, groups);
      build_rel(p->unpack, by_piece ? identity(p->unpack.items.size()) : item_order(p->unpack, false),
                opt.tile_bytes, true, false, false, groups);
    }
    build_rel(p->gather, by_piece ? identity(p->gather.items.size()) : item_order(p->gather, false),
              opt.tile_bytes, false, false, false, groups);
  }
  {
    // object sizes of each phase's pointer table, and the caller's names
    std::vector<uint64_t> sb(n_src), db(n_dst);
    for (int32_t i = 0; i < n_src; ++i)
      sb[i] = p->src[i].rows * p->src[i].cols * uint64_t(dtype_size(p->src[i].dtype));
    for (int32_t i = 0; i < n_dst; ++i)
      db[i] = p->dst[i].rows * p->dst[i].cols * uint64_t(dtype_size(p->dst[i].dtype));
    auto fill = [](Phase& ph, const std::vector<uint64_t>& a, const std::vector<uint64_t>& b,
                   const char* an, const char* bn) {
      ph.obj_bytes = a;
      ph.obj_bytes.insert(ph.obj_bytes.end(), b.begin(), b.end());
      ph.obj_use.resize(ph.obj_bytes.size(), 0);
      ph.src_name = an;
      ph.dst_name = bn;
    };
    if (buffers) {
      fill(p->pack, sb, p->peer_bytes, "src_ptrs", "peer_bufs");
      fill(p->unpack, p->peer_bytes, db, "peer_bufs", "dst_ptrs");
    }
    fill(p->gather, sb, db, "src_ptrs", "dst_ptrs");
  }
  for (Phase* ph : {&p->pack, &p->unpack, &p->gather}) {
    if (ph->n_tiles > UINT32_MAX) {
      delete p;
      return fail(SR_EINVAL, "plan has too many tiles; raise tile_bytes");
    }
    ph->interleave = !(opt.flags & SR_OPT_NO_XCD_INTERLEAVE) && ph->n_tiles >= 2 * uint64_t(kXcds);
  }
  // Per-peer piece lists (piece order) and payloads, from which the device
  // recomputes the buffer offsets.
  p->payload.assign(n_pieces, 0);
  p->peer_begin.assign(size_t(n_peers) + 1, 0);
  for (int32_t k = 0; k < n_pieces; ++k) {
    const sr_piece& pc = pieces[k];
    if (pc.kind == SR_PIECE_ZERO) continue;
    p->payload[k] = pc.rows * pc.cols * uint64_t(dtype_size(p->src[pc.src].dtype));
    ++p->peer_begin[pc.peer + 1];
  }
  for (int32_t q = 0; q < n_peers; ++q) p->peer_begin[q + 1] += p->peer_begin[q];
  p->peer_list.assign(p->peer_begin[n_peers], 0);
  {
    std::vector<uint32_t> fill(p->peer_begin.begin(), p->peer_begin.end() - 1);
    for (int32_t k = 0; k < n_pieces; ++k)
      if (pieces[k].kind != SR_PIECE_ZERO) p->peer_list[fill[pieces[k].peer]++] = uint32_t(k);
  }
  gather_alignment(p);
  // Item tables are rebuilt from the descriptors; the per-item host copies
  // are no longer needed.
  for (Phase* ph : {&p->pack, &p->unpack, &p->gather}) std::vector<HostItem>().swap(ph->items);
  *out_plan = p;
  return SR_OK;
}

int sr_plan_peer_bytes(const sr_plan* plan, int32_t peer, uint64_t* out_bytes) {
  if (!plan || !out_bytes) return fail(SR_EINVAL, "null argument");
  if (peer < 0 || peer >= plan->n_peers) return fail(SR_EINVAL, "peer %d out of range", peer);
  *out_bytes = plan->peer_bytes[peer];
  return SR_OK;
}

int sr_plan_piece_offset(const sr_plan* plan, int32_t piece, uint64_t* out_offset) {
  if (!plan || !out_offset) return fail(SR_EINVAL, "null argument");
  if (piece < 0 || size_t(piece) >= plan->pieces.size())
    return fail(SR_EINVAL, "piece %d out of range", piece);
  *out_offset = plan->piece_offset[piece];
  return SR_OK;
}

int sr_plan_info_get(const sr_plan* plan, sr_plan_info* out) {
  if (!plan || !out) return fail(SR_EINVAL, "null argument");
  out->n_pieces = int64_t(plan->pieces.size());
  out->n_peers = plan->n_peers;
  out->n_src = int64_t(plan->src.size());
  out->n_dst = int64_t(plan->dst.size());
  out->pack_tiles = int64_t(plan->pack.n_tiles);
  out->unpack_tiles = int64_t(plan->unpack.n_tiles);
  out->pack_bytes_read = plan->pack.bytes_read;
  out->pack_bytes_written = plan->pack.bytes_written;
  out->unpack_bytes_read = plan->unpack.bytes_read;
  out->unpack_bytes_written = plan->unpack.bytes_written;
  out->gather_tiles = int64_t(plan->gather.n_tiles);
  out->gather_bytes_read = plan->gather.bytes_read;
  out->gather_bytes_written = plan->gather.bytes_written;
  uint64_t b = 0;
  for (uint64_t v : plan->peer_bytes) b += v;
  out->buffer_bytes = b;
  return SR_OK;
}

int sr_pack(sr_plan* plan, const void* const* src_ptrs, void* const* peer_bufs, hipStream_t stream) {
  if (!plan) return fail(SR_EINVAL, "plan is null");
  if (plan->opt.flags & SR_OPT_GATHER_ONLY) return fail(SR_EINVAL, "sr_pack: the plan was created gather-only");
  // Alignment each pointer must satisfy: its element size; 0 = not read.
  std::vector<uint32_t> sal(plan->src.size(), 0), bal(plan->n_peers, 0);
  for (const sr_piece& pc : plan->pieces) {
    if (pc.kind == SR_PIECE_ZERO) continue;
    sal[pc.src] = dtype_size(plan->src[pc.src].dtype);
    bal[pc.peer] = 16;
  }
  int rc = check_ptrs(src_ptrs, plan->src.size(), sal, "src_ptrs");
  if (rc != SR_OK) return rc;
  rc = check_ptrs(reinterpret_cast<const void* const*>(peer_bufs), plan->n_peers, bal, "peer_bufs");
  if (rc != SR_OK) return rc;
  return run_phase(plan, plan->pack, kPack,
                   pointer_table(src_ptrs, plan->src.size(), peer_bufs, size_t(plan->n_peers)), stream);
}

int sr_unpack(sr_plan* plan, const void* const* peer_bufs, void* const* dst_ptrs, hipStream_t stream) {
  if (!plan) return fail(SR_EINVAL, "plan is null");
  if (plan->opt.flags & SR_OPT_GATHER_ONLY) return fail(SR_EINVAL, "sr_unpack: the plan was created gather-only");
  std::vector<uint32_t> bal(plan->n_peers, 0), dal(plan->dst.size(), 0);
  for (const sr_piece& pc : plan->pieces) {
    if (pc.kind != SR_PIECE_ZERO) bal[pc.peer] = 16;
    if (pc.dst >= 0) dal[pc.dst] = dtype_size(plan->dst[pc.dst].dtype);
    if (pc.dst2 >= 0) dal[pc.dst2] = dtype_size(plan->dst[pc.dst2].dtype);
  }
  int rc = check_ptrs(peer_bufs, plan->n_peers, bal, "peer_bufs");
  if (rc != SR_OK) return rc;
  rc = check_ptrs(reinterpret_cast<const void* const*>(dst_ptrs), plan->dst.size(), dal, "dst_ptrs");
  if (rc != SR_OK) return rc;
  return run_phase(plan, plan->unpack, kUnpack,
                   pointer_table(peer_bufs, size_t(plan->n_peers), dst_ptrs, plan->dst.size()), stream);
}

int sr_gather(sr_plan* plan, const void* const* src_ptrs, void* const* dst_ptrs, hipStream_t stream) {
  if (!plan) return fail(SR_EINVAL, "plan is null");
  int rc = check_ptrs(src_ptrs, plan->src.size(), plan->gather_src_align, "src_ptrs");
  if (rc != SR_OK) return rc;
  rc = check_ptrs(reinterpret_cast<const void* const*>(dst_ptrs), plan->dst.size(), plan->gather_dst_align,
                  "dst_ptrs");
  if (rc != SR_OK) return rc;
  return run_phase(plan, plan->gather, kGather,
                   pointer_table(src_ptrs, plan->src.size(), dst_ptrs, plan->dst.size()), stream);
}

int sr_prepare(hipStream_t stream) {
  int dev = -1;
  SR_HIP_TRY(hipGetDevice(&dev));
  TableCache& cache = table_cache();
  hipStream_t setup = nullptr;
  int rc = cache.setup_stream(dev, &setup);
  if (rc != SR_OK) return rc;
  // one upload of half a block on each stream (a first copy of that size
  // sets up the runtime's copy path for the stream) and one launch (loads
  // the library's GPU code); the blocks then go back to the cache
  constexpr size_t kBytes = size_t(1) << 20;
  void* d = nullptr;
  unsigned char* h = nullptr;
  size_t dcap = 0, hcap = 0;
  if ((rc = cache.get(false, dev, kBytes, &d, &dcap)) != SR_OK) return rc;
  if ((rc = cache.get(true, dev, kBytes, reinterpret_cast<void**>(&h), &hcap)) != SR_OK) {
    cache.put(false, dev, d, dcap);
    return rc;
  }
  std::memset(h, 0, hcap);
  const size_t half = std::min(dcap, hcap) / 2;
  const hipStream_t streams[2] = {stream, setup};
  hipError_t err = hipSuccess;
  for (int i = 0; i < 2 && err == hipSuccess; ++i) {
    err = hipMemcpyAsync(static_cast<unsigned char*>(d) + i * half, h + i * half, half, hipMemcpyHostToDevice,
                         streams[i]);
    if (err == hipSuccess) {
      hipLaunchKernelGGL(sr_prepare_kernel, dim3(1), dim3(64), 0, streams[i]);
      err = hipGetLastError();
    }
  }
  for (hipStream_t st : streams) {
    const hipError_t e = hipStreamSynchronize(st);
    if (err == hipSuccess) err = e;
  }
  cache.put(false, dev, d, dcap);
  cache.put(true, dev, h, hcap);
  if (err != hipSuccess) return fail(SR_EHIP, "sr_prepare: %s", hipGetErrorString(err));
  // events for the first plans' phases
  hipEvent_t ev[8] = {};
  for (hipEvent_t& e : ev)
    if ((rc = cache.get_event(dev, &e)) != SR_OK) break;
  for (hipEvent_t e : ev) cache.put_event(dev, e);
  return rc;
}

int sr_gather_noalloc(const sr_plan* plan, const void* const* src_ptrs, void* const* dst_ptrs,
                      hipStream_t stream) {
  if (!plan) return fail(SR_EINVAL, "plan is null");
  const Phase& ph = plan->gather;
  // The size check comes first: it needs neither the pointers nor a device.
  const ScratchLayout L = scratch_layout(ph);
  if (L.end > size_t(SR_SCRATCH_BYTES))
    return fail(SR_ENOMEM,
                "sr_gather_noalloc: the plan's gather tables need %zu bytes (%zu items, %llu tiles) but "
                "the scratch holds %zu; create the plan with a larger tile_bytes or split the transfer",
                L.end, ph.rel.size(), (unsigned long long)ph.n_tiles, size_t(SR_SCRATCH_BYTES));
  int rc = check_ptrs(src_ptrs, plan->src.size(), plan->gather_src_align, "src_ptrs");
  if (rc != SR_OK) return rc;
  rc = check_ptrs(reinterpret_cast<const void* const*>(dst_ptrs), plan->dst.size(), plan->gather_dst_align,
                  "dst_ptrs");
  if (rc != SR_OK) return rc;
  if (ph.rel.empty()) return SR_OK;
  const std::vector<uint64_t> ptrs = pointer_table(src_ptrs, plan->src.size(), dst_ptrs, plan->dst.size());
  if ((rc = check_disjoint(ph, ptrs)) != SR_OK) return rc;
  // The tables go up from pageable host memory that is released when the
  // call returns: a graph captured from this call would replay copies out of
  // freed memory, so a capturing stream is refused before any device work
  // (the argument checks above need no device).
  {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    SR_HIP_TRY(hipStreamIsCapturing(stream, &cap));
    if (cap != hipStreamCaptureStatusNone)
      return fail(SR_EINVAL,
                  "sr_gather_noalloc: the stream is capturing a graph; this call uploads its tables from "
                  "pageable host memory at every call and cannot be captured");
  }

  int dev = -1;
  SR_HIP_TRY(hipGetDevice(&dev));
  unsigned char* s = nullptr;
  if ((rc = scratch_base(dev, &s)) != SR_OK) return rc;
  DevRel* d_rel = reinterpret_cast<DevRel*>(s + L.rel);
  uint64_t* d_ptrs = reinterpret_cast<uint64_t*>(s + L.ptrs);
  DevItem* d_items = reinterpret_cast<DevItem*>(s + L.items);
  uint64_t* d_base = reinterpret_cast<uint64_t*>(s + L.base);
  DevTile* d_tiles = reinterpret_cast<DevTile*>(s + L.tiles);
  const uint32_t n = uint32_t(ph.rel.size());

  // Descriptors, tile prefix and pointers come from pageable host memory,
  // which HIP copies synchronously: each copy waits for the work queued on
  // `stream` before it (a previous call may still read the scratch) and the
  // host buffers may be released on return.  Every table is then written
  // whole -- the uploaded ones by the copies, each tile position by the emit
  // (the interleave is a permutation) and each item by the bind it folds in --
  // so nothing needs clearing.
  SR_HIP_TRY(hipMemcpyAsync(d_rel, ph.rel.data(), n * sizeof(DevRel), hipMemcpyHostToDevice, stream));
  SR_HIP_TRY(hipMemcpyAsync(d_base, ph.tile_base.data(), (size_t(n) + 1) * sizeof(uint64_t),
                            hipMemcpyHostToDevice, stream));
  EmitChunk* d_chunks = reinterpret_cast<EmitChunk*>(s + L.chunks);
  const uint32_t n_chunks = uint32_t(ph.emit_chunks.size());
  SR_HIP_TRY(hipMemcpyAsync(d_chunks, ph.emit_chunks.data(), n_chunks * sizeof(EmitChunk), hipMemcpyHostToDevice,
                            stream));
  SR_HIP_TRY(hipMemcpyAsync(d_ptrs, ptrs.data(), ptrs.size() * sizeof(uint64_t), hipMemcpyHostToDevice,
                            stream));
  const uint32_t shift = log2u(plan->opt.tile_bytes);
  // gather items read no buffer offsets (no side is a peer buffer)
  hipLaunchKernelGGL(sr_tile_emit_kernel, dim3(std::min<uint32_t>(n_chunks, 65535u)), dim3(kSetupBlock), 0,
                     stream, d_rel, d_base, d_chunks, n_chunks, shift, ph.n_tiles, ph.interleave ? kXcds : 1u,
                     d_tiles, d_ptrs, static_cast<const uint64_t*>(nullptr), d_items);
  SR_HIP_TRY(hipGetLastError());

  const uint32_t n_tiles = uint32_t(ph.n_tiles);
  uint32_t grid = n_tiles;
  if (plan->opt.max_blocks != 0) grid = std::min(grid, plan->opt.max_blocks);
  grid = std::min(grid, kMaxGrid);
  if (ph.interleave && grid < n_tiles && grid >= kXcds) grid -= grid % kXcds;
  const bool nt = (plan->opt.flags & SR_OPT_TEMPORAL) == 0;
  hipLaunchKernelGGL(nt ? sr_gather_kernel<true> : sr_gather_kernel<false>, dim3(grid), dim3(kBlock), 0,
                     stream, d_items, d_tiles, n_tiles);
  SR_HIP_TRY(hipGetLastError());
  return SR_OK;
}

void sr_plan_destroy(sr_plan* plan) {
  if (!plan) return;
  free_phase(plan->pack, plan->device);
  free_phase(plan->unpack, plan->device);
  free_phase(plan->gather, plan->device);
  TableCache& cache = table_cache();
  if (plan->ev_offsets) (void)hipEventSynchronize(plan->ev_offsets);
  cache.put(false, plan->device, plan->d_offmem, plan->d_offcap);
  cache.put(true, plan->device, plan->h_offmem, plan->h_offcap);
  cache.put_event(plan->device, plan->ev_offsets);
  delete plan;
}

}  // extern "C"
