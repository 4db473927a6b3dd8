// stage.cpp -- host-resident state for the reshard engine: sr_stage_pack
// (pack from sources in host memory into device peer buffers),
// sr_download (device regions back to host memory), their host thread pool
// and pinned window ring.
//
// Reference behaviour served (paths relative to the Suika repository): the
// fake-source (checkpoint) mode of execute_param_transfer slices sources in
// host memory with get_send_tensor and moves each piece with .to(device)
// (Suika/migration.py:290-312, 477-482); checkpoint_load asks for the new
// state on device="cpu" (:1235-1244).
//
// Design
//   * Only the pieces' bytes cross to the device, already in the peer-buffer
//     layout the unpack reads: each peer buffer is cut into spans of
//     consecutive host-resident pieces, the spans are packed into pinned
//     windows of SR_STAGE_WINDOW_BYTES, and each window goes to the device
//     with one host-to-device copy per span part it holds.  The host threads
//     fill window w + 1 while the copy engine moves window w; a window is
//     refilled only after the copy that read it has completed (its event).
//   * Host copies are split over the pool by window bytes; a piece whose rows
//     are contiguous in its source (every dim 0 piece) is one memcpy, a dim -1
//     piece one memcpy per row.  Sources memory-mapped from a file are paged
//     in by these reads, a page per piece boundary beyond the piece bytes.
//   * sr_download runs the ring the other way: up to SR_STAGE_WINDOWS
//     device-to-host copies in flight, each window drained to its host
//     destinations by the pool once its copy has completed.
//   * Device-resident sources in a staged plan (a caller mixing host and
//     device state) are copied on the device with hipMemcpy2DAsync, into
//     their own pieces' bytes only.

#include <hip/hip_runtime.h>
#include <sched.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "suika_reshard.h"
#include "sr_internal.h"

namespace {

using sr_internal::dtype_size;
using sr_internal::fail;
using sr_internal::PlanView;

#define ST_HIP_TRY(expr)                                                      \
  do {                                                                        \
    hipError_t e_ = (expr);                                                   \
    if (e_ != hipSuccess)                                                     \
      return fail(SR_EHIP, "%s failed: %s", #expr, hipGetErrorString(e_));    \
  } while (0)

constexpr size_t kWindow = SR_STAGE_WINDOW_BYTES;
constexpr int kWindows = SR_STAGE_WINDOWS;
constexpr int kMaxThreads = 256;
constexpr int kDefaultMaxThreads = 16;
// A window's bytes are split into tasks of at least this many bytes.
constexpr size_t kMinTaskBytes = size_t(256) << 10;

// ------------------------------------------------------------ thread pool
// Detached workers parked on a condition variable.  run() publishes one job
// (task indices claimed from an atomic counter) to its first `helpers`
// workers and takes part itself; it returns once those helpers have run out
// of tasks, so every task is complete.  A process forked after the pool
// started gets a pool of its own (the workers do not survive a fork).
class Pool {
 public:
  static Pool& get() {
    static std::mutex mu;
    static Pool* pool = nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!pool || pool->pid_ != getpid()) pool = new Pool();   // never destroyed
    return *pool;
  }

  int threads() {
    std::lock_guard<std::mutex> lock(run_mu_);
    return want_;
  }

  void set_threads(int n) {
    std::lock_guard<std::mutex> lock(run_mu_);
    want_ = n > 0 ? n : default_threads();
  }

  // fn(0) .. fn(n - 1), each once, on the workers and the calling thread.
  void run(int n, const std::function<void(int)>& fn) {
    if (n <= 0) return;
    std::lock_guard<std::mutex> run_lock(run_mu_);
    const int helpers = std::min(want_, n) - 1;
    if (helpers <= 0) {
      for (int i = 0; i < n; ++i) fn(i);
      return;
    }
    while (started_ < helpers) {   // gen_ changes only under run_mu_
      std::thread([this, id = started_, seen = gen_] { loop(id, seen); }).detach();
      ++started_;
    }
    {
      std::lock_guard<std::mutex> lock(mu_);
      fn_ = &fn;
      n_ = n;
      next_.store(0);
      job_helpers_ = helpers;
      active_ = helpers;
      ++gen_;
    }
    cv_.notify_all();
    work();
    std::unique_lock<std::mutex> lock(mu_);
    done_cv_.wait(lock, [&] { return active_ == 0; });
    fn_ = nullptr;
  }

 private:
  Pool() : pid_(getpid()), want_(default_threads()) {}

  static int default_threads() {
    cpu_set_t set;
    int n = 0;
    if (sched_getaffinity(0, sizeof(set), &set) == 0) n = CPU_COUNT(&set);
    if (n <= 0) n = int(std::thread::hardware_concurrency());
    return std::max(1, std::min(n, kDefaultMaxThreads));
  }

  void work() {
    for (int i; (i = next_.fetch_add(1)) < n_;) (*fn_)(i);
  }

  // Worker `id` takes part in jobs with more than `id` helpers.
  void loop(int id, uint64_t seen) {
    for (;;) {
      {
        std::unique_lock<std::mutex> lock(mu_);
        cv_.wait(lock, [&] { return gen_ != seen; });
        seen = gen_;
        if (id >= job_helpers_) continue;
      }
      work();
      {
        std::lock_guard<std::mutex> lock(mu_);
        --active_;
      }
      done_cv_.notify_all();
    }
  }

  const pid_t pid_;
  int want_;
  int started_ = 0;
  std::mutex run_mu_;   // one job at a time
  std::mutex mu_;       // job publication and completion
  std::condition_variable cv_, done_cv_;
  const std::function<void(int)>* fn_ = nullptr;
  int n_ = 0;
  std::atomic<int> next_{0};
  int job_helpers_ = 0;
  int active_ = 0;      // helpers of the current job still working
  uint64_t gen_ = 0;
};

// ------------------------------------------------------------ window ring
enum Direction { kUp = 0, kDown = 1 };

struct Ring {
  int device = -1;
  int direction = kUp;
  unsigned char* base = nullptr;            // kWindows * kWindow pinned bytes
  hipEvent_t ev[kWindows] = {};
  bool pending[kWindows] = {};              // ev[i] recorded after a copy of window i
  std::mutex mu;                            // one staging call at a time

  unsigned char* slot(int i) const { return base + size_t(i) * kWindow; }

  // Waits for the copy that last used window i.
  int wait(int i) {
    if (!pending[i]) return SR_OK;
    ST_HIP_TRY(hipEventSynchronize(ev[i]));
    pending[i] = false;
    return SR_OK;
  }

  int wait_all() {
    int rc = SR_OK;
    for (int i = 0; i < kWindows; ++i) {
      const int r = wait(i);
      if (rc == SR_OK) rc = r;
    }
    return rc;
  }
};

// One ring per device and direction (host to device for sr_stage_pack,
// device to host for sr_download, so that an upload and a download can run
// at once, one per copy direction of the link), created on first use with
// that device current and kept until the process exits (no HIP call from a
// static destructor).
int ring_of(int device, Direction dir, Ring** out) {
  static std::mutex mu;
  static std::vector<Ring*>* rings = new std::vector<Ring*>();
  std::lock_guard<std::mutex> lock(mu);
  for (Ring* r : *rings)
    if (r->device == device && r->direction == dir) {
      *out = r;
      return SR_OK;
    }
  Ring* r = new Ring();
  r->device = device;
  r->direction = dir;
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, size_t(kWindows) * kWindow, hipHostMallocDefault);
  if (e != hipSuccess) {
    delete r;
    return fail(SR_ENOMEM, "pinned staging windows (%zu bytes): %s", size_t(kWindows) * kWindow,
                hipGetErrorString(e));
  }
  r->base = static_cast<unsigned char*>(p);
  for (int i = 0; i < kWindows; ++i) {
    e = hipEventCreateWithFlags(&r->ev[i], hipEventDisableTiming);
    if (e != hipSuccess) {
      for (int j = 0; j < i; ++j) (void)hipEventDestroy(r->ev[j]);
      (void)hipHostFree(p);
      delete r;
      return fail(SR_EHIP, "hipEventCreateWithFlags failed: %s", hipGetErrorString(e));
    }
  }
  rings->push_back(r);
  *out = r;
  return SR_OK;
}

// ------------------------------------------------------------ counters
std::atomic<uint64_t> g_up{0}, g_up_pieces{0}, g_dev_pieces{0}, g_down{0}, g_windows{0};

bool on_device(const void* p) {
  hipPointerAttribute_t a{};
  const hipError_t e = hipPointerGetAttributes(&a, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();   // host memory HIP does not know: not an error here
    return false;
  }
  return a.type == hipMemoryTypeDevice;
}

// ------------------------------------------------------------ staging plan
// A window holds segments: byte ranges of one peer buffer, each at a window
// offset (segments follow each other in the window).
struct Segment {
  int32_t peer;
  uint64_t begin, end;    // peer-buffer bytes
  size_t at;              // window offset of `begin`
};

struct PieceGeom {
  const unsigned char* src;   // host address of the region origin
  uint64_t row_bytes;         // bytes per region row
  uint64_t stride;            // source bytes between rows
  uint64_t offset;            // buffer offset of the payload
  uint64_t bytes;             // payload bytes
};

// Copies buffer bytes [a, b) of one piece's payload (a, b relative to the
// payload) to `out`.
void copy_piece_part(const PieceGeom& g, uint64_t a, uint64_t b, unsigned char* out) {
  if (g.row_bytes == g.stride) {   // rows contiguous in the source
    std::memcpy(out, g.src + a, b - a);
    return;
  }
  uint64_t row = a / g.row_bytes, col = a % g.row_bytes;
  while (a < b) {
    const uint64_t n = std::min(g.row_bytes - col, b - a);
    std::memcpy(out, g.src + row * g.stride + col, n);
    out += n;
    a += n;
    ++row;
    col = 0;
  }
}

// Fills window bytes [w0, w1) of `segs` from the pieces of each segment's
// peer (geometry by piece, `list` = each peer's piece indices by offset).
void fill_range(const std::vector<Segment>& segs, size_t w0, size_t w1, unsigned char* window,
                const std::vector<PieceGeom>& geom, const PlanView& v) {
  // first segment that ends after w0
  size_t s = std::upper_bound(segs.begin(), segs.end(), w0,
                              [](size_t x, const Segment& g) { return x < g.at + (g.end - g.begin); }) -
             segs.begin();
  for (; s < segs.size() && segs[s].at < w1; ++s) {
    const Segment& g = segs[s];
    const uint64_t lo = g.begin + (std::max(w0, g.at) - g.at);
    const uint64_t hi = g.begin + (std::min(w1, g.at + size_t(g.end - g.begin)) - g.at);
    const uint32_t* first = v.peer_list + v.peer_begin[g.peer];
    const uint32_t* last = v.peer_list + v.peer_begin[g.peer + 1];
    // the piece holding `lo` (or the first after it): pieces are in offset order
    const uint32_t* k = std::upper_bound(first, last, lo, [&](uint64_t x, uint32_t idx) {
      return x < v.piece_offset[idx];
    });
    if (k != first) --k;
    for (; k != last && v.piece_offset[*k] < hi; ++k) {
      const PieceGeom& pg = geom[*k];
      const uint64_t a = std::max(lo, pg.offset), b = std::min(hi, pg.offset + pg.bytes);
      if (a >= b) continue;   // an alignment gap, or a piece that ends before lo
      copy_piece_part(pg, a - pg.offset, b - pg.offset, window + g.at + (a - g.begin));
    }
  }
}

// Fills one window on the pool: tasks of equal byte share.
void fill_window(const std::vector<Segment>& segs, size_t fill, unsigned char* window,
                 const std::vector<PieceGeom>& geom, const PlanView& v) {
  Pool& pool = Pool::get();
  const int n = int(std::max<size_t>(1, std::min<size_t>(size_t(pool.threads()), fill / kMinTaskBytes)));
  const size_t share = (fill + size_t(n) - 1) / size_t(n);
  pool.run(n, [&](int t) {
    const size_t w0 = std::min(fill, size_t(t) * share), w1 = std::min(fill, w0 + share);
    if (w0 < w1) fill_range(segs, w0, w1, window, geom, v);
  });
}

// Every source slot and peer buffer a non-ZERO piece uses: non-null and
// aligned (element size; 16 bytes for buffers).  `all_host`: every slot is
// host memory (sr_pack_host, whose null buffers skip their peer); otherwise
// each slot is classified by its address (1 = device memory).
int check_stage_args(const PlanView& v, const void* const* src_ptrs, void* const* peer_bufs, bool all_host,
                     std::vector<int8_t>& dev_slot, std::vector<uint8_t>& peer_used) {
  if (v.n_pieces > 0 && v.n_src > 0 && !src_ptrs) return fail(SR_EINVAL, "src_ptrs: pointer array is null");
  if (v.n_peers > 0 && !peer_bufs) return fail(SR_EINVAL, "peer_bufs: pointer array is null");
  dev_slot.assign(v.n_src, -1);
  peer_used.assign(size_t(std::max(0, v.n_peers)), 0);
  for (size_t k = 0; k < v.n_pieces; ++k) {
    const sr_piece& pc = v.pieces[k];
    if (pc.kind == SR_PIECE_ZERO) continue;
    const uintptr_t b = reinterpret_cast<uintptr_t>(peer_bufs[pc.peer]);
    if (all_host && b == 0) continue;   // peer skipped
    if (!peer_used[pc.peer]) {
      if (b == 0) return fail(SR_EINVAL, "peer_bufs[%d] is null", pc.peer);
      if (b % 16 != 0) return fail(SR_EALIGN, "peer_bufs[%d] = %p is not 16-byte aligned", pc.peer,
                                   peer_bufs[pc.peer]);
      peer_used[pc.peer] = 1;
    }
    if (dev_slot[pc.src] < 0) {
      const uintptr_t a = reinterpret_cast<uintptr_t>(src_ptrs[pc.src]);
      const uint32_t es = uint32_t(dtype_size(v.src[pc.src].dtype));
      if (a == 0) return fail(SR_EINVAL, "src_ptrs[%d] is null", pc.src);
      if (a % es != 0) return fail(SR_EALIGN, "src_ptrs[%d] = %p is not %u-byte aligned", pc.src, src_ptrs[pc.src], es);
      dev_slot[pc.src] = all_host ? 0 : (on_device(src_ptrs[pc.src]) ? 1 : 0);
    }
  }
  return SR_OK;
}

// Source address, row width, stride, buffer offset and payload of every
// non-ZERO piece whose slot has an address (ZERO pieces: all zero).
void piece_geometry(const PlanView& v, const void* const* src_ptrs, std::vector<PieceGeom>& geom) {
  geom.assign(v.n_pieces, PieceGeom{nullptr, 0, 0, 0, 0});
  for (size_t k = 0; k < v.n_pieces; ++k) {
    const sr_piece& pc = v.pieces[k];
    if (pc.kind == SR_PIECE_ZERO || !src_ptrs[pc.src]) continue;
    const sr_tensor& st = v.src[pc.src];
    const uint64_t es = uint64_t(dtype_size(st.dtype));
    PieceGeom& g = geom[k];
    g.src = static_cast<const unsigned char*>(src_ptrs[pc.src]) + (pc.src_row * st.cols + pc.src_col) * es;
    g.row_bytes = pc.cols * es;
    g.stride = st.cols * es;
    g.offset = v.piece_offset[k];
    g.bytes = pc.rows * g.row_bytes;
  }
}

}  // namespace

extern "C" {

int sr_set_host_threads(int32_t n) {
  if (n < 0 || n > kMaxThreads) return fail(SR_EINVAL, "host threads %d outside [0, %d]", n, kMaxThreads);
  Pool::get().set_threads(n);
  return SR_OK;
}

int sr_stage_counters_get(sr_stage_counters* out) {
  if (!out) return fail(SR_EINVAL, "null argument");
  out->host_bytes_up = g_up.load();
  out->host_piece_bytes = g_up_pieces.load();
  out->device_piece_bytes = g_dev_pieces.load();
  out->bytes_down = g_down.load();
  out->windows = g_windows.load();
  return SR_OK;
}

int sr_pack_host(const sr_plan* plan, const void* const* src_ptrs, void* const* peer_bufs) {
  if (!plan) return fail(SR_EINVAL, "plan is null");
  const PlanView v = sr_internal::plan_view(plan);
  std::vector<int8_t> dev_slot;
  std::vector<uint8_t> peer_used;
  int rc = check_stage_args(v, src_ptrs, peer_bufs, true, dev_slot, peer_used);
  if (rc != SR_OK) return rc;
  std::vector<PieceGeom> geom;
  piece_geometry(v, src_ptrs, geom);
  // peer by peer: the buffer itself is the window, its pieces the segments
  for (int32_t q = 0; q < v.n_peers; ++q) {
    if (!peer_bufs[q]) continue;
    std::vector<Segment> segs;
    for (uint32_t i = v.peer_begin[q]; i < v.peer_begin[q + 1]; ++i) {
      const PieceGeom& g = geom[v.peer_list[i]];
      if (g.bytes) segs.push_back(Segment{q, g.offset, g.offset + g.bytes, size_t(g.offset)});
    }
    if (!segs.empty())
      fill_window(segs, size_t(segs.back().end), static_cast<unsigned char*>(peer_bufs[q]), geom, v);
  }
  return SR_OK;
}

int sr_stage_pack(sr_plan* plan, const void* const* src_ptrs, void* const* peer_bufs, hipStream_t stream) {
  if (!plan) return fail(SR_EINVAL, "plan is null");
  const PlanView v = sr_internal::plan_view(plan);
  std::vector<int8_t> dev_slot;
  std::vector<uint8_t> peer_used;
  int rc = check_stage_args(v, src_ptrs, peer_bufs, false, dev_slot, peer_used);
  if (rc != SR_OK) return rc;
  int dev = -1;
  ST_HIP_TRY(hipGetDevice(&dev));

  // geometry of every piece; device-resident pieces are copied on the device
  std::vector<PieceGeom> geom;
  piece_geometry(v, src_ptrs, geom);
  uint64_t dev_bytes = 0;
  for (size_t k = 0; k < v.n_pieces; ++k) {
    const sr_piece& pc = v.pieces[k];
    if (pc.kind == SR_PIECE_ZERO) continue;
    const PieceGeom& g = geom[k];
    if (dev_slot[pc.src] == 1 && g.bytes > 0) {
      unsigned char* to = static_cast<unsigned char*>(peer_bufs[pc.peer]) + g.offset;
      if (g.row_bytes == g.stride || pc.rows == 1)
        ST_HIP_TRY(hipMemcpyAsync(to, g.src, g.bytes, hipMemcpyDeviceToDevice, stream));
      else
        ST_HIP_TRY(hipMemcpy2DAsync(to, g.row_bytes, g.src, g.stride, g.row_bytes, pc.rows,
                                    hipMemcpyDeviceToDevice, stream));
      dev_bytes += g.bytes;
    }
  }
  g_dev_pieces += dev_bytes;

  // spans of consecutive host pieces per peer, cut into windows
  Ring* ring = nullptr;
  bool any_host = false;
  for (size_t s = 0; s < v.n_src && !any_host; ++s) any_host = dev_slot[s] == 0;
  if (!any_host) return SR_OK;
  if ((rc = ring_of(dev, kUp, &ring)) != SR_OK) return rc;
  std::lock_guard<std::mutex> lock(ring->mu);
  std::vector<Segment> segs;
  size_t fill = 0;
  int w = 0;   // next window slot
  uint64_t up = 0, up_pieces = 0;
  auto flush = [&]() -> int {
    if (segs.empty()) return SR_OK;
    int r = ring->wait(w);
    if (r != SR_OK) return r;
    unsigned char* window = ring->slot(w);
    fill_window(segs, fill, window, geom, v);
    for (const Segment& g : segs)
      ST_HIP_TRY(hipMemcpyAsync(static_cast<unsigned char*>(peer_bufs[g.peer]) + g.begin, window + g.at,
                                g.end - g.begin, hipMemcpyHostToDevice, stream));
    ST_HIP_TRY(hipEventRecord(ring->ev[w], stream));
    ring->pending[w] = true;
    up += fill;
    ++g_windows;
    segs.clear();
    fill = 0;
    w = (w + 1) % kWindows;
    return SR_OK;
  };
  auto add_span = [&](int32_t q, uint64_t a, uint64_t b) -> int {
    while (a < b) {
      const uint64_t n = std::min<uint64_t>(b - a, kWindow - fill);
      segs.push_back(Segment{q, a, a + n, fill});
      fill += size_t(n);
      a += n;
      if (fill == kWindow) {
        const int r = flush();
        if (r != SR_OK) return r;
      }
    }
    return SR_OK;
  };
  for (int32_t q = 0; q < v.n_peers && rc == SR_OK; ++q) {
    bool open = false;
    uint64_t a = 0, b = 0;
    for (uint32_t i = v.peer_begin[q]; i < v.peer_begin[q + 1] && rc == SR_OK; ++i) {
      const uint32_t k = v.peer_list[i];
      const PieceGeom& g = geom[k];
      if (dev_slot[v.pieces[k].src] != 0 || g.bytes == 0) {
        if (open && dev_slot[v.pieces[k].src] != 0) {   // a device piece ends the span
          rc = add_span(q, a, b);
          open = false;
        }
        continue;
      }
      up_pieces += g.bytes;
      if (!open) {
        a = g.offset;
        open = true;
      }
      b = g.offset + g.bytes;
    }
    if (open && rc == SR_OK) rc = add_span(q, a, b);
  }
  if (rc == SR_OK) rc = flush();
  g_up += up;
  g_up_pieces += up_pieces;
  if (rc != SR_OK) (void)ring->wait_all();   // no copy may still read a window on return
  return rc;
}

int sr_download(const void* const* dev_ptrs, void* const* host_ptrs, const uint64_t* bytes, int32_t n,
                hipStream_t stream) {
  if (n < 0) return fail(SR_EINVAL, "region count %d is negative", n);
  if (n == 0) return SR_OK;
  if (!dev_ptrs || !host_ptrs || !bytes) return fail(SR_EINVAL, "null argument");
  uint64_t total = 0;
  for (int32_t i = 0; i < n; ++i) {
    if (bytes[i] == 0) continue;
    if (!dev_ptrs[i]) return fail(SR_EINVAL, "dev_ptrs[%d] is null", i);
    if (!host_ptrs[i]) return fail(SR_EINVAL, "host_ptrs[%d] is null", i);
    total += bytes[i];
  }
  if (total == 0) return SR_OK;
  // Fresh host memory is mapped at its first write, a 4 KiB page per fault
  // unless the range asks for transparent huge pages: large destinations do
  // (a hint; the kernel may decline it, and the call does not depend on it).
  for (int32_t i = 0; i < n; ++i) {
    constexpr uintptr_t kHuge = uintptr_t(2) << 20;
    const uintptr_t a = reinterpret_cast<uintptr_t>(host_ptrs[i]);
    const uintptr_t lo = (a + kHuge - 1) & ~(kHuge - 1), hi = (a + bytes[i]) & ~(kHuge - 1);
    if (bytes[i] && hi > lo) (void)madvise(reinterpret_cast<void*>(lo), hi - lo, MADV_HUGEPAGE);
  }
  int dev = -1;
  ST_HIP_TRY(hipGetDevice(&dev));
  Ring* ring = nullptr;
  int rc = ring_of(dev, kDown, &ring);
  if (rc != SR_OK) return rc;
  std::lock_guard<std::mutex> lock(ring->mu);
  if ((rc = ring->wait_all()) != SR_OK) return rc;

  // A window's segments: (region, region offset, length, window offset).
  struct Part {
    int32_t region;
    uint64_t off, len;
    size_t at;
  };
  std::vector<std::vector<Part>> parts(kWindows);
  std::vector<size_t> filled(kWindows, 0);
  int32_t region = 0;
  uint64_t roff = 0;
  auto next_window = [&](std::vector<Part>& out) -> size_t {
    out.clear();
    size_t fill = 0;
    while (region < n && fill < kWindow) {
      const uint64_t left = bytes[region] - roff;
      if (left == 0) {
        ++region;
        roff = 0;
        continue;
      }
      const uint64_t len = std::min<uint64_t>(left, kWindow - fill);
      out.push_back(Part{region, roff, len, fill});
      fill += size_t(len);
      roff += len;
    }
    return fill;
  };
  auto issue = [&](int s) -> int {
    const std::vector<Part>& ps = parts[s];
    unsigned char* window = ring->slot(s);
    for (size_t i = 0; i < ps.size();) {
      // adjacent device regions go up in one copy
      size_t j = i + 1;
      const unsigned char* from = static_cast<const unsigned char*>(dev_ptrs[ps[i].region]) + ps[i].off;
      uint64_t len = ps[i].len;
      while (j < ps.size() && ps[j].off == 0 &&
             static_cast<const unsigned char*>(dev_ptrs[ps[j].region]) == from + len) {
        len += ps[j].len;
        ++j;
      }
      ST_HIP_TRY(hipMemcpyAsync(window + ps[i].at, from, len, hipMemcpyDeviceToHost, stream));
      i = j;
    }
    ST_HIP_TRY(hipEventRecord(ring->ev[s], stream));
    ring->pending[s] = true;
    return SR_OK;
  };
  auto drain = [&](int s) -> int {
    const int r = ring->wait(s);
    if (r != SR_OK) return r;
    const std::vector<Part>& ps = parts[s];
    const unsigned char* window = ring->slot(s);
    const size_t fill = filled[s];
    Pool& pool = Pool::get();
    const int nt = int(std::max<size_t>(1, std::min<size_t>(size_t(pool.threads()), fill / kMinTaskBytes)));
    const size_t share = (fill + size_t(nt) - 1) / size_t(nt);
    pool.run(nt, [&](int t) {
      const size_t w0 = std::min(fill, size_t(t) * share), w1 = std::min(fill, w0 + share);
      for (const Part& p : ps) {
        const size_t lo = std::max(w0, p.at), hi = std::min(w1, p.at + size_t(p.len));
        if (lo >= hi) continue;
        std::memcpy(static_cast<unsigned char*>(host_ptrs[p.region]) + p.off + (lo - p.at), window + lo, hi - lo);
      }
    });
    ++g_windows;
    return SR_OK;
  };
  // up to kWindows copies in flight; window i is drained before its slot is reused
  int issued = 0, drained = 0;
  for (;;) {
    while (issued - drained < kWindows) {
      const int s = issued % kWindows;
      filled[s] = next_window(parts[s]);
      if (filled[s] == 0) break;
      if ((rc = issue(s)) != SR_OK) break;
      ++issued;
    }
    if (rc != SR_OK || drained == issued) break;
    if ((rc = drain(drained % kWindows)) != SR_OK) break;
    ++drained;
  }
  if (rc != SR_OK) {
    (void)ring->wait_all();
    return rc;
  }
  g_down += total;
  return SR_OK;
}

}  // extern "C"
