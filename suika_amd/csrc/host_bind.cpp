// host_bind.cpp -- per-tensor and per-meta host work of the drop-in operators, native
// (suika_amd/lib/_suika_host.so, a CPython extension on torch's C++ API).
//
// execute_param_transfer (Suika/migration.py:397-556) touches every source
// tensor (to check it and read its shape, dtype and address) and allocates
// every destination tensor.  In Python that costs a few microseconds per
// tensor, which on transfers of many small tensors exceeds the GPU time of
// the copy itself.  These functions do the same walks over the state dicts,
// the ops and the slot tables in C++:
//
//   collect_sources: (ops, rank -> state dict, fields) -> source specs
//                    (sr_src_spec rows), dtypes and device addresses, with
//                    the same checks and messages as the Python host;
//   alloc_dst:       destination slot rows (sr_slot_key) -> fresh tensors in
//                    {name: {field: tensor}} and their addresses;
//   bind_dst:        caller-provided destinations (e.g. an arena's tensors) checked
//                    against the slot rows -> their addresses;
//   arena_views:     the same dict of typed tensors on one allocation's storage;
//   arena_tensors:   the drop-in call's destination arena: every (name, field)
//                    of a transfer laid out and allocated in one go;
//   encode_layout:   a ParamLayout as an sr_meta table (sr_schedule's input);
//   make_ops:        sr_schedule's op table as TransferOp objects;
//   encode_ops:      one rank's TransferOps as sr_lower's op and meta tables;
//   piece_numels:    elements per op's piece (launch-group balancing);
//   rank_runs:       the ops one destination rank executes, grouped by tensor
//                    with their elements (the drop-in call's prologue);
//   take_ops:        one launch group's ops;
//   device_views:    tensors over a mapped hand-off allocation (no copy);
//   plan_sources:    one launch group: the above in one call, with the
//                    destinations' allocations made on a helper thread while
//                    this thread plans, and the launch;
//   blocks_ahead:    counts of destinations built on the helper's blocks.
//
// Apart from plan_sources' launch, no device work happens here; the tensors
// come from torch's caching allocator on the device's current stream, as
// torch.empty would.

#include <torch/extension.h>
#include <c10/core/DeviceGuard.h>
#include <c10/core/StreamGuard.h>
#include <c10/core/impl/VirtualGuardImpl.h>
#include <torch/csrc/Dtype.h>
#include <torch/csrc/DynamicTypes.h>
#include <pybind11/numpy.h>

#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <deque>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "sr_meta.h"
#include "suika_planner.h"
#include "suika_reshard.h"

namespace py = pybind11;

namespace {

[[noreturn]] void assertion(const std::string& msg) {
  PyErr_SetString(PyExc_AssertionError, msg.c_str());
  throw py::error_already_set();
}

// sr_dtype of a torch element type (include/suika_reshard.h); -1: unsupported.
int64_t sr_code(at::ScalarType st) {
  switch (st) {
    case at::kByte:
    case at::kChar:
    case at::kBool:
    case at::kFloat8_e4m3fn:
    case at::kFloat8_e5m2:
    case at::kFloat8_e4m3fnuz:
    case at::kFloat8_e5m2fnuz:
      return 0;
    case at::kBFloat16: return 1;
    case at::kHalf: return 2;
    case at::kFloat: return 3;
    case at::kDouble: return 4;
    case at::kInt: return 5;
    case at::kLong: return 6;
    default: return -1;
  }
}

py::object dtype_object(at::ScalarType st) {
  return py::reinterpret_borrow<py::object>(reinterpret_cast<PyObject*>(torch::getTHPDtype(st)));
}

// d[key], or an empty object when the key is absent (dicts and other mappings).
py::object lookup(PyObject* d, PyObject* key) {
  if (PyDict_Check(d)) {
    PyObject* v = PyDict_GetItemWithError(d, key);   // borrowed
    if (!v && PyErr_Occurred()) throw py::error_already_set();
    return py::reinterpret_borrow<py::object>(v);
  }
  PyObject* v = PyObject_GetItem(d, key);   // new reference
  if (!v) {
    if (!PyErr_ExceptionMatches(PyExc_KeyError)) throw py::error_already_set();
    PyErr_Clear();
  }
  return py::reinterpret_steal<py::object>(v);
}

// Interned attribute names (created once, never released).
struct Names {
  PyObject *dtype, *shape, *kind_args, *tp_meta, *kind, *rows, *name, *dict;
  PyObject *param_name, *src_rank, *dst_rank, *src_meta, *dst_meta, *dst_shard_meta, *tables;
  PyObject *chunk, *vocab_pad, *qkv_heads;
  Names() {
    auto in = [](const char* s) { return PyUnicode_InternFromString(s); };
    dtype = in("dtype"); shape = in("shape"); kind_args = in("kind_args"); tp_meta = in("tp_meta");
    kind = in("kind"); rows = in("rows"); name = in("name"); dict = in("__dict__");
    param_name = in("param_name"); src_rank = in("src_rank"); dst_rank = in("dst_rank");
    src_meta = in("src_meta"); dst_meta = in("dst_meta"); dst_shard_meta = in("dst_shard_meta");
    tables = in("_tables");
    chunk = in("chunk"); vocab_pad = in("vocab_pad"); qkv_heads = in("qkv_heads");
  }
};

const Names& names_() {
  static Names* n = new Names();
  return *n;
}

py::object attr(PyObject* o, PyObject* key) {
  PyObject* v = PyObject_GetAttr(o, key);
  if (!v) throw py::error_already_set();
  return py::reinterpret_steal<py::object>(v);
}

constexpr int64_t kSpecWords = 10;   // sr_src_spec: dtype, ndim, shape[8]
constexpr int64_t kKeyWords = 13;    // sr_slot_key: op, field, recast, dtype, ndim, shape[8]

// A source in host memory met where only device sources are taken:
// suika_amd._lib.HostSourceError (an AssertionError), which the drop-in
// call answers by staging the transfer from host memory.
[[noreturn]] void host_source(const std::string& msg) {
  static PyObject* cls = py::object(py::module_::import("suika_amd._lib").attr("HostSourceError")).release().ptr();
  PyErr_SetString(cls, msg.c_str());
  throw py::error_already_set();
}

// The source tensor of every (op, field), checked once.  `source(rank)`
// returns a rank's state dict; it is called once per rank, when the first op
// of that rank is reached, so errors come in op order as in the reference's
// loop (migration.py:426-494).  A tensor is on device `device_index`, or,
// with `host_ok`, in host memory (the addresses are then host addresses,
// for sr_stage_pack only).
py::tuple collect_sources(py::list ops, py::function source, py::list fields, int64_t device_index,
                          const std::string& who, bool host_ok) {
  const Names& N = names_();
  py::dict sources;
  const int64_t n = int64_t(ops.size()), nf = int64_t(fields.size());
  py::array_t<int64_t> specs({n * nf * kSpecWords});
  py::array_t<uint64_t> ptrs({n * nf});
  py::list dtypes(n * nf);
  int64_t* sp = specs.mutable_data();
  uint64_t* pp = ptrs.mutable_data();
  std::fill(sp, sp + n * nf * kSpecWords, 0);
  const std::string want_device = "cuda:" + std::to_string(device_index);
  for (int64_t k = 0; k < n; ++k) {
    PyObject* op = PyList_GET_ITEM(ops.ptr(), k);
    py::object rank = attr(op, N.src_rank);
    py::object name = attr(op, N.param_name);
    py::object sd = lookup(sources.ptr(), rank.ptr());
    if (!sd) {
      sd = source(rank);
      sources[rank] = sd;
    }
    py::object entry = lookup(sd.ptr(), name.ptr());
    // messages are built only on the failing path
    auto nm = [&]() { return py::str(name).cast<std::string>(); };
    if (!entry) assertion(who + ": param missing in source " + nm());
    for (int64_t f = 0; f < nf; ++f) {
      py::handle field = PyList_GET_ITEM(fields.ptr(), f);
      py::object obj = lookup(entry.ptr(), field.ptr());
      if (!obj) assertion("expected_sub_fields mismatch: " + nm() + " has no " + py::str(field).cast<std::string>());
      if (!THPVariable_Check(obj.ptr()))
        assertion("source " + nm() + "/" + py::str(field).cast<std::string>() + " of rank " +
                  py::str(rank).cast<std::string>() + ": not a tensor");
      const at::Tensor& t = THPVariable_Unpack(obj.ptr());
      const int64_t code = sr_code(t.scalar_type());
      const int64_t nd = t.dim();
      const bool here = (t.is_cuda() && t.get_device() == device_index) || (host_ok && t.is_cpu());
      if (!here || !t.is_contiguous() || code < 0 || nd > 8) {
        // the rare path: build the message
        const std::string fs = py::str(field).cast<std::string>();
        const std::string what = "source " + nm() + "/" + fs + " of rank " + py::str(rank).cast<std::string>();
        if (!here && t.is_cpu()) host_source(what + " is in host memory, not on " + want_device);
        if (!here) assertion(what + " is on " + t.device().str() + ", not on " + want_device);
        if (!t.is_contiguous()) assertion(what + " is not contiguous");
        assertion("source " + nm() + "/" + fs + ": " + py::str(dtype_object(t.scalar_type())).cast<std::string>() +
                  ", " + std::to_string(nd) + "-D is not supported by the reshard engine");
      }
      int64_t* row = sp + (k * nf + f) * kSpecWords;
      row[0] = code;
      row[1] = nd;
      const at::IntArrayRef sizes = t.sizes();
      for (int64_t d = 0; d < nd; ++d) row[2 + d] = sizes[size_t(d)];
      PyList_SET_ITEM(dtypes.ptr(), k * nf + f, dtype_object(t.scalar_type()).release().ptr());
      pp[k * nf + f] = reinterpret_cast<uint64_t>(t.data_ptr());
    }
  }
  return py::make_tuple(specs, dtypes, ptrs);
}

using RowTable = py::array_t<int64_t, py::array::c_style | py::array::forcecast>;

// Fresh tensors on the device's caching allocator, built without the
// dispatcher: each one gets an allocation and a storage of its own, exactly as
// at::empty gives (same allocator, current stream, resizable storage), at a
// fraction of at::empty's per-call cost -- the drop-in call allocates one per
// destination tensor and field.
// A dense tensor of `device` as at::empty makes it: its dispatch keys
// (autograd keys included) and the allocator its storage comes from.  Outside
// inference mode (whose tensors carry other keys) they are read once per
// device and kept for the process.
struct TensorKind {
  c10::DispatchKeySet keys;
  c10::Allocator* alloc;
};

TensorKind tensor_kind(at::Device device) {
  auto read = [&] {
    at::Tensor t = at::empty({0}, at::TensorOptions().device(device));
    TensorKind k{t.key_set(), t.storage().allocator()};
    if (k.alloc == nullptr) throw std::runtime_error("no allocator for " + device.str());
    return k;
  };
  if (c10::InferenceMode::is_enabled()) return read();
  static std::mutex mu;
  static std::vector<std::pair<at::Device, TensorKind>>* kinds = new std::vector<std::pair<at::Device, TensorKind>>();
  std::lock_guard<std::mutex> lock(mu);
  for (const auto& dk : *kinds)
    if (dk.first == device) return dk.second;
  const TensorKind k = read();
  kinds->emplace_back(device, k);
  return k;
}

class FreshTensors {
 public:
  explicit FreshTensors(at::Device device) : guard_(device), kind_(tensor_kind(device)),
                                             keys_(kind_.keys), alloc_(kind_.alloc) {}

  static size_t bytes_of(at::IntArrayRef sizes, at::ScalarType st) {
    int64_t numel = 1;
    for (int64_t s : sizes) {
      if (s < 0 || __builtin_mul_overflow(numel, s, &numel)) throw py::value_error("bad destination shape");
    }
    return size_t(numel) * c10::elementSize(st);
  }

  // A tensor on `block` (nbytes from this allocator, see BlockJob), else on
  // a new allocation.
  at::Tensor make(at::IntArrayRef sizes, at::ScalarType st, c10::DataPtr* block = nullptr) const {
    const size_t nbytes = bytes_of(sizes, st);
    c10::Storage storage(c10::Storage::use_byte_size_t(), nbytes,
                         block ? std::move(*block) : alloc_->allocate(nbytes), alloc_, /*resizable=*/true);
    auto impl = c10::make_intrusive<c10::TensorImpl>(std::move(storage), keys_, c10::scalarTypeToTypeMeta(st));
    impl->set_sizes_contiguous(sizes);
    return at::Tensor(std::move(impl));
  }

  c10::Allocator* allocator() const { return alloc_; }

 private:
  c10::DeviceGuard guard_;   // the allocator serves the current device
  TensorKind kind_;
  c10::DispatchKeySet keys_;
  c10::Allocator* alloc_;
};

// ------------------------------------------------------------ destination blocks made ahead
//
// On a share of many small tensors the caching-allocator call behind each
// fresh destination tensor is a large part of the host's time per tensor.
// In the drop-in call's prologue every destination's block is handed to a
// helper thread, tensor by tensor in launch order, which allocates them on
// the call's device and current stream -- the allocations at::empty would
// make -- while the calling thread reads, lowers and plans the launch
// groups.  A block's size is the tensor's elements (its pieces' total) times
// the element size its field has in the first sources the prologue reads.
// The tensors are then built on those blocks, on the calling thread (built
// on the helper, they cost both threads more than they saved): each still
// has an allocation of its own.  A block the helper did not make (an
// allocation failed, the job was stopped) or whose size is not the planned
// tensor's (another dtype, a padded vocabulary shard) is not used; the
// tensor is allocated on the calling thread instead, which also reports any
// allocation failure.  Unused blocks are freed when the call ends, on the
// calling thread.

// The blocks of one job: slot i has nbytes[i] bytes (0: no block).
class BlockJob {
 public:
  BlockJob(c10::Allocator* alloc, c10::Stream stream, std::vector<size_t> nbytes)
      : alloc_(alloc), stream_(stream), nbytes_(std::move(nbytes)), blocks_(nbytes_.size()) {}

  // On the helper thread.  Slot i belongs to the helper until ready_ > i.
  void run() noexcept {
    try {
      c10::StreamGuard guard(stream_);   // the device and stream the calling thread allocates on
      for (size_t i = 0; i < nbytes_.size() && !stop_.load(std::memory_order_relaxed); ++i) {
        if (nbytes_[i]) blocks_[i] = alloc_->allocate(nbytes_[i]);
        ready_.store(i + 1, std::memory_order_release);
      }
    } catch (...) {
      // out of device memory, say: the remaining slots get no block
    }
    done_.store(true, std::memory_order_release);
  }

  // Slot i's block when the helper made one of `bytes` bytes, moved into
  // `out`; waits for the helper (without the GIL, which it may need).
  bool take(size_t i, size_t bytes, c10::DataPtr* out) {
    if (i >= nbytes_.size() || bytes == 0 || nbytes_[i] != bytes) return false;
    if (ready_.load(std::memory_order_acquire) <= i) {
      py::gil_scoped_release nogil;
      while (ready_.load(std::memory_order_acquire) <= i && !done_.load(std::memory_order_acquire))
        std::this_thread::yield();
    }
    if (ready_.load(std::memory_order_acquire) <= i || !blocks_[i]) return false;
    *out = std::move(blocks_[i]);
    return true;
  }

  // Stops the helper on this job, waits until it is done with it and frees
  // the blocks nobody took.  Called with or without the GIL; never throws.
  void finish() noexcept {
    stop_.store(true, std::memory_order_relaxed);
    if (!done_.load(std::memory_order_acquire)) {
      auto wait = [this] {
        while (!done_.load(std::memory_order_acquire)) std::this_thread::yield();
      };
      if (PyGILState_Check()) {
        py::gil_scoped_release nogil;
        wait();
      } else {
        wait();
      }
    }
    std::vector<c10::DataPtr>().swap(blocks_);
  }

 private:
  c10::Allocator* const alloc_;
  const c10::Stream stream_;
  const std::vector<size_t> nbytes_;
  std::vector<c10::DataPtr> blocks_;
  std::atomic<size_t> ready_{0};
  std::atomic<bool> done_{false}, stop_{false};
};

// The helper thread: runs jobs in submission order.  Its state is created
// by the first submission (under the GIL, so once per process) and again in
// a forked child, which has no helper thread; it is never destroyed, so the
// detached thread never outlives it.
class BlockHelper {
 public:
  // false when no helper thread could be started (the caller then allocates
  // everything itself)
  static bool submit(std::shared_ptr<BlockJob> job) {
    BlockHelper* h = instance();
    if (!h) return false;
    {
      std::lock_guard<std::mutex> lk(h->mutex_);
      h->queue_.push_back(std::move(job));
    }
    h->cv_.notify_one();
    return true;
  }

 private:
  static BlockHelper* instance() {
    static BlockHelper* helper = nullptr;
    static pid_t owner = 0;
    if (helper && owner == getpid()) return helper;
    BlockHelper* h = new BlockHelper();
    try {
      std::thread([h] { h->loop(); }).detach();
    } catch (const std::exception&) {
      delete h;
      return nullptr;
    }
    helper = h;
    owner = getpid();
    return helper;
  }

  void loop() {
    for (;;) {
      std::shared_ptr<BlockJob> job;
      {
        std::unique_lock<std::mutex> lk(mutex_);
        cv_.wait(lk, [this] { return !queue_.empty(); });
        job = std::move(queue_.front());
        queue_.pop_front();
      }
      job->run();
    }
  }

  std::mutex mutex_;
  std::condition_variable cv_;
  std::deque<std::shared_ptr<BlockJob>> queue_;
};

// Destination tensors built on a block made ahead, and those a job covered
// that were allocated on the calling thread instead (process totals).
std::atomic<uint64_t> g_blocks_taken{0}, g_blocks_missed{0};

// Slot of (tensor nid of a group, field f, recast copy or not) in the
// group's BlockJob, nf fields.
inline size_t block_slot(size_t nid, int64_t f, bool recast, int64_t nf) {
  return (nid * 2 + (recast ? 1 : 0)) * size_t(nf) + size_t(f);
}

constexpr size_t kNoBlock = SIZE_MAX;

// The destination blocks of one drop-in call, made on the helper thread in
// launch order: tensor t (a rank_runs index) is position pos_[t] of the
// order, its field f (and f's bf16 copy) slot block_slot(pos, f, copy, nf).
class AheadBlocks {
 public:
  // order: tensor indices in launch order; numel / padded: per tensor (rank_runs);
  // itemsize: bytes per element of each field (0: no block); copies: 1 for a
  // field with a bf16 copy
  AheadBlocks(int64_t device_index, const RowTable& order, const RowTable& numel, py::array_t<bool> padded,
              std::vector<int64_t> itemsize, std::vector<int64_t> copies)
      : nf_(int64_t(itemsize.size())) {
    if (order.ndim() != 1 || numel.ndim() != 1 || padded.ndim() != 1 || numel.shape(0) != padded.shape(0) ||
        copies.size() != itemsize.size())
      throw py::value_error("ahead blocks: order, numel and padded must be 1-D, one itemsize and copy flag per field");
    const int64_t n_tensors = numel.shape(0);
    pos_.assign(size_t(n_tensors), kNoBlock);
    std::vector<size_t> nbytes(size_t(order.shape(0)) * 2 * size_t(nf_), 0);
    const bool* pd = padded.data();
    for (int64_t p = 0; p < order.shape(0); ++p) {
      const int64_t t = order.data()[p];
      if (t < 0 || t >= n_tensors || pos_[size_t(t)] != kNoBlock) throw py::value_error("ahead blocks: bad order");
      pos_[size_t(t)] = size_t(p);
      const int64_t elems = numel.data()[t];
      if (pd[t] || elems <= 0) continue;
      for (int64_t f = 0; f < nf_; ++f) {
        if (itemsize[size_t(f)] > 0) nbytes[block_slot(size_t(p), f, false, nf_)] = size_t(elems * itemsize[size_t(f)]);
        if (copies[size_t(f)]) nbytes[block_slot(size_t(p), f, true, nf_)] = size_t(elems) * c10::elementSize(at::kBFloat16);
      }
    }
    const at::Device device(at::kCUDA, c10::DeviceIndex(device_index));
    FreshTensors fresh(device);
    const c10::Stream current = c10::impl::VirtualGuardImpl(device.type()).getStream(device);
    job_ = std::make_shared<BlockJob>(fresh.allocator(), current, std::move(nbytes));
    if (!BlockHelper::submit(job_)) job_.reset();
  }
  ~AheadBlocks() { finish(); }

  // Position of tensor t in the job, kNoBlock if none.
  size_t pos(int64_t t) const { return t >= 0 && size_t(t) < pos_.size() ? pos_[size_t(t)] : kNoBlock; }
  int64_t fields() const { return nf_; }
  BlockJob* job() const { return job_.get(); }
  // Stops the helper on this job and frees the blocks no tensor took.
  void finish() {
    if (job_) job_->finish();
  }

 private:
  int64_t nf_;
  std::vector<size_t> pos_;
  std::shared_ptr<BlockJob> job_;
};

// Fresh destination tensors for the slot rows (and the zero-element ones).
// With `job`, a tensor takes the block made ahead for it (slot block_slot of
// op k's job position op_pos[k]) when there is one of its size.
py::tuple alloc_dst(const RowTable& rows, const RowTable& empty_rows, py::list names, py::list fields,
                    py::list recast_names, py::list dtypes, at::Device device, const FreshTensors* made = nullptr,
                    BlockJob* job = nullptr, const std::vector<size_t>* op_pos = nullptr) {
  const int64_t nf = int64_t(fields.size());
  py::dict out;
  const int64_t n = rows.ndim() == 2 ? rows.shape(0) : 0;
  py::array_t<uint64_t> ptrs({n});
  uint64_t* pp = ptrs.mutable_data();
  std::unique_ptr<FreshTensors> own;
  if (!made) made = (own = std::make_unique<FreshTensors>(device)).get();
  const FreshTensors& fresh = *made;
  const Py_ssize_t n_names = PyList_GET_SIZE(names.ptr());
  if (PyList_GET_SIZE(recast_names.ptr()) != nf || PyList_GET_SIZE(dtypes.ptr()) < n_names * nf)
    throw py::value_error("one recast name per field and one dtype per (op, field)");
  int64_t last_k = -1;   // the rows of one tensor come together: its entry is kept
  PyObject* entry = nullptr;
  for (int pass = 0; pass < 2; ++pass) {
    const auto& tbl = pass == 0 ? rows : empty_rows;
    const int64_t m = tbl.ndim() == 2 ? tbl.shape(0) : 0;
    if (m && tbl.shape(1) != kKeyWords) throw py::value_error("slot rows must have 13 columns");
    const int64_t* r = tbl.data();
    for (int64_t i = 0; i < m; ++i, r += kKeyWords) {
      const int64_t k = r[0], f = r[1], is_recast = r[2], nd = r[4];
      if (k < 0 || k >= n_names || f < 0 || f >= nf || nd < 0 || nd > 8)
        throw py::value_error("malformed slot row");
      at::ScalarType st;
      PyObject* field;
      if (is_recast) {
        st = at::kBFloat16;
        field = PyList_GET_ITEM(recast_names.ptr(), f);
      } else {
        PyObject* dt = PyList_GET_ITEM(dtypes.ptr(), k * nf + f);
        if (!THPDtype_Check(dt)) throw py::type_error("dtypes must hold torch.dtype objects");
        st = reinterpret_cast<THPDtype*>(dt)->scalar_type;
        field = PyList_GET_ITEM(fields.ptr(), f);
      }
      const at::IntArrayRef sizes(r + 5, size_t(nd));
      c10::DataPtr block;
      const size_t pos = job ? (*op_pos)[size_t(k)] : kNoBlock;
      const bool ahead = pos != kNoBlock && job->take(block_slot(pos, f, is_recast != 0, nf),
                                                      FreshTensors::bytes_of(sizes, st), &block);
      if (job) (ahead ? g_blocks_taken : g_blocks_missed).fetch_add(1, std::memory_order_relaxed);
      at::Tensor t = fresh.make(sizes, st, ahead ? &block : nullptr);
      if (k != last_k) {
        PyObject* name = PyList_GET_ITEM(names.ptr(), k);
        entry = PyDict_GetItemWithError(out.ptr(), name);
        if (!entry) {
          if (PyErr_Occurred()) throw py::error_already_set();
          py::dict e;
          if (PyDict_SetItem(out.ptr(), name, e.ptr()) != 0) throw py::error_already_set();
          entry = e.ptr();   // held by `out`
        }
        last_k = k;
      }
      if (pass == 0) pp[i] = reinterpret_cast<uint64_t>(t.data_ptr());
      py::object wrapped = py::reinterpret_steal<py::object>(THPVariable_Wrap(std::move(t)));
      if (!wrapped || PyDict_SetItem(entry, field, wrapped.ptr()) != 0) throw py::error_already_set();
    }
  }
  return py::make_tuple(out, ptrs);
}

// Addresses of caller-provided destination tensors for the slot rows, each
// checked against its slot: a contiguous tensor of the slot's shape and
// dtype on `device`.
py::array_t<uint64_t> bind_dst(py::dict part, const RowTable& rows, py::list names, py::list fields,
                               py::list recast_names, py::list dtypes, at::Device device) {
  const int64_t nf = int64_t(fields.size());
  const int64_t n = rows.ndim() == 2 ? rows.shape(0) : 0;
  if (n && rows.shape(1) != kKeyWords) throw py::value_error("slot rows must have 13 columns");
  py::array_t<uint64_t> ptrs({n});
  uint64_t* pp = ptrs.mutable_data();
  const int64_t* r = rows.data();
  for (int64_t i = 0; i < n; ++i, r += kKeyWords) {
    const int64_t k = r[0], f = r[1], is_recast = r[2], nd = r[4];
    if (k < 0 || k >= int64_t(names.size()) || f < 0 || f >= nf || nd < 0 || nd > 8)
      throw py::value_error("malformed slot row");
    py::handle name = names[k];
    py::handle field = is_recast ? recast_names[f] : fields[f];
    at::ScalarType st = at::kBFloat16;
    if (!is_recast) {
      py::handle dt = dtypes[k * nf + f];
      if (!THPDtype_Check(dt.ptr())) throw py::type_error("dtypes must hold torch.dtype objects");
      st = reinterpret_cast<THPDtype*>(dt.ptr())->scalar_type;
    }
    // the message is built only when a check fails
    auto what = [&]() {
      return "(" + py::repr(name).cast<std::string>() + ", " + py::repr(field).cast<std::string>() + ")";
    };
    py::object entry = lookup(part.ptr(), name.ptr());
    py::object obj = entry ? lookup(entry.ptr(), field.ptr()) : py::object();
    if (!obj) assertion(what() + ": no destination tensor");
    if (!THPVariable_Check(obj.ptr())) assertion(what() + ": not a tensor");
    const at::Tensor& t = THPVariable_Unpack(obj.ptr());
    if (t.device() != device)
      assertion(what() + ": tensor is on " + t.device().str() + ", the kernels run on " + device.str());
    if (!t.is_contiguous()) assertion(what() + ": tensor is not contiguous");
    if (t.scalar_type() != st) assertion(what() + ": dtype differs from the planned one");
    bool same = t.dim() == nd;
    for (int64_t d = 0; same && d < nd; ++d) same = t.size(d) == r[5 + d];
    if (!same) assertion(what() + ": shape differs from the planned one");
    pp[i] = reinterpret_cast<uint64_t>(t.data_ptr());
  }
  return ptrs;
}

// Typed tensors on the storage of one byte buffer (a destination arena): row i is
// (byte offset, ndim, shape[8]); out[names[i]][fields[i]] is its tensor.
py::dict arena_views(const at::Tensor& buf, py::list names, py::list fields, const RowTable& rows,
                     py::list dtypes) {
  const int64_t n = rows.ndim() == 2 ? rows.shape(0) : 0;
  if (n && rows.shape(1) != 10) throw py::value_error("arena rows must have 10 columns");
  if (int64_t(names.size()) != n || int64_t(fields.size()) != n || int64_t(dtypes.size()) != n)
    throw py::value_error("one name, field and dtype per arena row");
  if (buf.scalar_type() != at::kByte || buf.dim() != 1 || !buf.is_contiguous())
    throw py::value_error("the arena must be a contiguous 1-D uint8 tensor");
  py::dict out;
  const c10::Storage& storage = buf.storage();
  const int64_t* r = rows.data();
  for (int64_t i = 0; i < n; ++i, r += 10) {
    py::handle dt = dtypes[i];
    if (!THPDtype_Check(dt.ptr())) throw py::type_error("dtypes must hold torch.dtype objects");
    const at::ScalarType st = reinterpret_cast<THPDtype*>(dt.ptr())->scalar_type;
    const int64_t nd = r[1];
    if (nd < 0 || nd > 8) throw py::value_error("malformed arena row");
    int64_t numel = 1;
    for (int64_t d = 0; d < nd; ++d) numel *= r[2 + d];
    const int64_t bytes = numel * int64_t(c10::elementSize(st));
    const int64_t esize = int64_t(c10::elementSize(st));
    if (r[0] < 0 || r[0] + bytes > buf.size(0) || (buf.storage_offset() + r[0]) % esize != 0)
      throw py::value_error("arena row outside the buffer or misaligned");
    // One tensor on the arena's storage at the row's offset (what
    // narrow().view(dtype).view(shape) gives, without the three dispatched
    // ops and two intermediate tensors per view).
    auto impl = c10::make_intrusive<c10::TensorImpl>(c10::Storage(storage), buf.key_set(),
                                                     c10::scalarTypeToTypeMeta(st));
    impl->set_storage_offset((buf.storage_offset() + r[0]) / esize);
    impl->set_sizes_contiguous(at::IntArrayRef(r + 2, size_t(nd)));
    at::Tensor v(std::move(impl));
    py::handle name = names[i];
    PyObject* entry = PyDict_GetItemWithError(out.ptr(), name.ptr());
    if (!entry) {
      if (PyErr_Occurred()) throw py::error_already_set();
      py::dict fresh;
      out[name] = fresh;
      entry = fresh.ptr();
    }
    py::object wrapped = py::reinterpret_steal<py::object>(THPVariable_Wrap(v));
    if (PyDict_SetItem(entry, fields[i].ptr(), wrapped.ptr()) != 0) throw py::error_already_set();
  }
  return out;
}

// ------------------------------------------------------------ layouts and ops

constexpr int64_t kMetaWords = 21;   // sr_meta: rank, name, itemsize, ndim, shape[8], tp[3], kind, args[3], rows[2]
static_assert(sizeof(sr_meta) == kMetaWords * sizeof(int64_t), "an sr_meta row is 21 int64 words");

int64_t as_int(PyObject* o) {
  const long long v = PyLong_AsLongLong(o);
  if (v == -1 && PyErr_Occurred()) throw py::error_already_set();
  return int64_t(v);
}

// An attribute the reference's own objects do not carry: TensorMeta has only
// name, dtype, shape and tp_meta (Suika/migration.py:29-58; tp_meta is left
// unset when built from dtype and shape alone) and TransferOp only
// param_name, src_rank, dst_rank, src_meta and dst_meta (:257-282).  Such an
// object reads as `fallback`: a chunk layout, no kind arguments, no row
// interval, no attached destination shard.
py::object opt_attr(PyObject* o, PyObject* key, PyObject* fallback) {
  PyObject* v = PyObject_GetAttr(o, key);
  if (v) return py::reinterpret_steal<py::object>(v);
  if (!PyErr_ExceptionMatches(PyExc_AttributeError)) throw py::error_already_set();
  PyErr_Clear();
  return py::reinterpret_borrow<py::object>(fallback);
}

PyObject* empty_tuple() {
  static PyObject* t = PyTuple_New(0);
  return t;
}

py::object kind_of(PyObject* m) { return opt_attr(m, names_().kind, names_().chunk); }
py::object kind_args_of(PyObject* m) { return opt_attr(m, names_().kind_args, empty_tuple()); }
py::object tp_meta_of(PyObject* m) { return opt_attr(m, names_().tp_meta, Py_None); }
py::object rows_of(PyObject* m) { return opt_attr(m, names_().rows, Py_None); }
py::object shard_of(PyObject* op) { return opt_attr(op, names_().dst_shard_meta, Py_None); }

// One sr_meta row of a TensorMeta (the attributes its constructor sets).
void meta_row(PyObject* m, int64_t rank, int64_t name_id, int64_t* row) {
  const Names& N = names_();
  std::fill(row, row + kMetaWords, 0);
  row[0] = rank;
  row[1] = name_id;
  py::object dt = attr(m, N.dtype);
  if (!THPDtype_Check(dt.ptr())) throw py::type_error("TensorMeta.dtype is not a torch.dtype");
  row[2] = int64_t(c10::elementSize(reinterpret_cast<THPDtype*>(dt.ptr())->scalar_type));
  py::object shape = attr(m, N.shape), args = kind_args_of(m);
  if (!PyTuple_Check(shape.ptr()) || !PyTuple_Check(args.ptr()))
    throw py::type_error("TensorMeta.shape and kind_args must be tuples");
  const int64_t nd = int64_t(PyTuple_GET_SIZE(shape.ptr())), na = int64_t(PyTuple_GET_SIZE(args.ptr()));
  if (nd > 8 || na > 3)
    assertion(py::str(attr(m, N.name)).cast<std::string>() + ": " + std::to_string(nd) + "-D shape / " +
              std::to_string(na) + " kind args");
  row[3] = nd;
  for (int64_t d = 0; d < nd; ++d) row[4 + d] = as_int(PyTuple_GET_ITEM(shape.ptr(), d));
  py::object tp = tp_meta_of(m);
  if (tp.ptr() != Py_None) {
    if (!PyTuple_Check(tp.ptr()) || PyTuple_GET_SIZE(tp.ptr()) != 3)
      throw py::value_error("tp_meta must be (slice_dim, tp_index, tp_deg)");
    for (int i = 0; i < 3; ++i) row[12 + i] = as_int(PyTuple_GET_ITEM(tp.ptr(), i));
  }
  py::object kind = kind_of(m);
  if (!PyUnicode_Check(kind.ptr())) throw py::type_error("TensorMeta.kind must be a str");
  if (PyUnicode_Compare(kind.ptr(), N.chunk) == 0) row[15] = 0;
  else if (PyUnicode_Compare(kind.ptr(), N.vocab_pad) == 0) row[15] = 1;
  else if (PyUnicode_Compare(kind.ptr(), N.qkv_heads) == 0) row[15] = 2;
  else throw py::value_error("unknown shard kind " + py::str(kind).cast<std::string>());
  if (PyErr_Occurred()) throw py::error_already_set();
  for (int64_t i = 0; i < na; ++i) row[16 + i] = as_int(PyTuple_GET_ITEM(args.ptr(), i));
  py::object rows = rows_of(m);
  if (rows.ptr() == Py_None) {
    row[19] = row[20] = -1;
  } else {
    if (!PyTuple_Check(rows.ptr()) || PyTuple_GET_SIZE(rows.ptr()) != 2)
      throw py::value_error("rows must be (first, end)");
    row[19] = as_int(PyTuple_GET_ITEM(rows.ptr(), 0));
    row[20] = as_int(PyTuple_GET_ITEM(rows.ptr(), 1));
  }
}

// The encoding of a scheduled op: the sr_meta rows of its source meta and of
// its destination shard, then its piece (tp index and degree, first and end
// row; as in sr_op).
constexpr int64_t kEncodingWords = 2 * kMetaWords + 4;

// The tables a schedule's ops are encoded from: suika_amd.meta.Schedule
// keeps them as `_tables` = (its sr_op table, the sr_meta tables of both
// layouts, the layouts' meta objects, each op's piece meta), row k for the
// op at position k, and drops them when the list changes.  An op is encoded
// from them while the schedule still holds its tables and the op at the
// position found for it, and the op still names the scheduled metas; any
// other op is read from its attributes.  TensorMeta objects are values:
// nothing edits one in place once scheduled.
//
// Positions are found by object identity in a table that rank_runs fills
// with the ops it takes (note), else with the whole list on first use.
class Encoded {
 public:
  Encoded(py::object schedule, py::object tables) {
    if (schedule.is_none() || tables.is_none()) return;
    py::tuple t = tables.cast<py::tuple>();
    if (t.size() != 6) throw py::value_error("schedule tables: 6 items expected");
    sched_ = schedule;
    tables_ = tables;
    ops_ = t[0].cast<RowTable>();
    src_ = t[1].cast<RowTable>();
    dst_ = t[2].cast<RowTable>();
    src_objs_ = t[3];
    dst_objs_ = t[4];
    pieces_ = t[5];
    if (!PyList_Check(sched_.ptr()) || !PyList_Check(src_objs_.ptr()) || !PyList_Check(dst_objs_.ptr()) ||
        !PyList_Check(pieces_.ptr()) || ops_.ndim() != 2 || ops_.shape(1) != 9 || src_.ndim() != 2 ||
        src_.shape(1) != kMetaWords || dst_.ndim() != 2 || dst_.shape(1) != kMetaWords ||
        ops_.shape(0) != PyList_GET_SIZE(sched_.ptr()) || ops_.shape(0) != PyList_GET_SIZE(pieces_.ptr()) ||
        src_.shape(0) != PyList_GET_SIZE(src_objs_.ptr()) || dst_.shape(0) != PyList_GET_SIZE(dst_objs_.ptr()))
      throw py::value_error("schedule tables: inconsistent");
    valid_ = true;
  }

  // Whether the schedule still holds these tables (checked once per native
  // call; a changed schedule has dropped them).
  bool current() const {
    if (!valid_) return false;
    PyObject* v = nullptr;
    if (_PyObject_LookupAttr(sched_.ptr(), names_().tables, &v) < 0) throw py::error_already_set();
    Py_XDECREF(v);   // compared by identity only; the schedule holds it
    return v == tables_.ptr();
  }

  // `op` is the schedule's op at position k.
  void note(PyObject* op, int64_t k) const {
    if (!valid_) return;
    if ((used_ + 1) * 2 > slots_.size()) grow();
    const size_t mask = slots_.size() - 1;
    size_t i = slot_of(op) & mask;
    while (slots_[i].op && slots_[i].op != op) i = (i + 1) & mask;
    if (!slots_[i].op) ++used_;
    slots_[i] = Slot{op, k};
  }

  // op's encoding into w and its destination shard object, when op is
  // encoded (see above; `source`: its source meta is checked too).
  bool get(PyObject* op, int64_t* w, bool source, PyObject** shard = nullptr) const {
    if (!valid_) return false;
    if (slots_.empty()) {
      const Py_ssize_t n = PyList_GET_SIZE(sched_.ptr());
      for (Py_ssize_t k = 0; k < n; ++k) note(PyList_GET_ITEM(sched_.ptr(), k), k);
      if (slots_.empty()) return false;
    }
    const size_t mask = slots_.size() - 1;
    size_t i = slot_of(op) & mask;
    while (slots_[i].op && slots_[i].op != op) i = (i + 1) & mask;
    if (!slots_[i].op) return false;
    const int64_t k = slots_[i].at;
    if (k < 0 || k >= ops_.shape(0) || k >= PyList_GET_SIZE(sched_.ptr()) ||
        PyList_GET_ITEM(sched_.ptr(), k) != op)
      return false;
    const Names& N = names_();
    const int64_t* r = ops_.data() + k * 9;
    const int64_t s_row = r[3], d_row = r[4];
    if (s_row < 0 || s_row >= src_.shape(0) || d_row < 0 || d_row >= dst_.shape(0)) return false;
    if (source && attr(op, N.src_meta).ptr() != PyList_GET_ITEM(src_objs_.ptr(), s_row)) return false;
    if (attr(op, N.dst_meta).ptr() != PyList_GET_ITEM(pieces_.ptr(), k)) return false;
    std::memcpy(w, src_.data() + s_row * kMetaWords, sizeof(int64_t) * kMetaWords);
    std::memcpy(w + kMetaWords, dst_.data() + d_row * kMetaWords, sizeof(int64_t) * kMetaWords);
    std::copy(r + 5, r + 9, w + 2 * kMetaWords);
    if (shard) *shard = PyList_GET_ITEM(dst_objs_.ptr(), d_row);
    return true;
  }

 private:
  struct Slot {
    PyObject* op;
    int64_t at;
  };
  static size_t slot_of(PyObject* op) {
    uint64_t x = uint64_t(reinterpret_cast<uintptr_t>(op)) >> 4;
    x *= 0x9E3779B97F4A7C15ull;
    return size_t(x ^ (x >> 32));
  }
  void grow() const {
    std::vector<Slot> old(std::max<size_t>(64, slots_.size() * 2), Slot{nullptr, -1});
    old.swap(slots_);
    used_ = 0;
    for (const Slot& s : old)
      if (s.op) note(s.op, s.at);
  }

  bool valid_ = false;
  py::object sched_, tables_, src_objs_, dst_objs_, pieces_;
  RowTable ops_, src_, dst_;
  mutable std::vector<Slot> slots_;   // keys are borrowed: the schedule holds every op
  mutable size_t used_ = 0;
};

// The encoding to use in one native call: E while its schedule still holds
// its tables, else none.
const Encoded* live(const Encoded* E) { return E && E->current() ? E : nullptr; }

// A ParamLayout's {rank: {name: TensorMeta}} as an [n, 21] sr_meta table,
// rank by rank in dict order; `names` maps names to ids (extended in first-
// seen order) and `objs` receives each row's TensorMeta.
py::array_t<int64_t> encode_layout(py::dict layout, py::dict names, py::list objs) {
  int64_t n = 0;
  for (auto kv : layout) {
    if (!PyDict_Check(kv.second.ptr())) throw py::type_error("a layout maps ranks to dicts of TensorMeta");
    n += int64_t(PyDict_GET_SIZE(kv.second.ptr()));
  }
  py::array_t<int64_t> out({n, kMetaWords});
  int64_t* row = out.mutable_data();
  for (auto kv : layout) {
    const int64_t rank = as_int(kv.first.ptr());
    PyObject *key, *value;
    Py_ssize_t pos = 0;
    while (PyDict_Next(kv.second.ptr(), &pos, &key, &value)) {
      PyObject* id = PyDict_GetItemWithError(names.ptr(), key);
      int64_t nid;
      if (id) {
        nid = as_int(id);
      } else {
        if (PyErr_Occurred()) throw py::error_already_set();
        nid = int64_t(PyDict_GET_SIZE(names.ptr()));
        py::int_ v(nid);
        if (PyDict_SetItem(names.ptr(), key, v.ptr()) != 0) throw py::error_already_set();
      }
      meta_row(value, rank, nid, row);
      if (PyList_Append(objs.ptr(), value) != 0) throw py::error_already_set();
      row += kMetaWords;
    }
  }
  return out;
}

// A new instance of a plain Python class without running its __init__, and
// its (fresh) instance dict.
py::object bare_instance(PyObject* cls, PyObject** dict_out) {
  static PyObject* empty = PyTuple_New(0);
  PyTypeObject* type = reinterpret_cast<PyTypeObject*>(cls);
  PyObject* obj = type->tp_new(type, empty, nullptr);
  if (!obj) throw py::error_already_set();
  py::object o = py::reinterpret_steal<py::object>(obj);
  PyObject* d = PyObject_GenericGetDict(obj, nullptr);   // new reference
  if (!d) throw py::error_already_set();
  Py_DECREF(d);   // the instance keeps its dict
  *dict_out = d;
  return o;
}

void set(PyObject* d, PyObject* key, PyObject* value) {
  if (PyDict_SetItem(d, key, value) != 0) throw py::error_already_set();
}

// A piece of `shard`: the same TensorMeta with another tp meta or a row
// interval, built without running the constructor.
py::object derived(PyObject* meta_cls, PyObject* shard, PyObject* tp_meta, PyObject* rows) {
  const Names& N = names_();
  PyObject* d;
  py::object m = bare_instance(meta_cls, &d);
  py::object src = attr(shard, N.dict);
  if (PyDict_Update(d, src.ptr()) != 0) throw py::error_already_set();
  set(d, N.tp_meta, tp_meta);
  set(d, N.rows, rows);
  // a shard of the reference's TensorMeta class lacks the extension fields
  if (PyDict_SetDefault(d, N.kind, N.chunk) == nullptr) throw py::error_already_set();
  if (PyDict_SetDefault(d, N.kind_args, empty_tuple()) == nullptr) throw py::error_already_set();
  return m;
}

// TransferOps of an sr_op table (sr_schedule's output): source metas and
// destination shards are the layouts' own objects, pieces derived from the
// shards.  A `pieces` list receives each op's piece meta: what the
// schedule's encoding (Encoded) needs besides the tables sr_schedule read.
py::list make_ops(const RowTable& ops, py::list names, py::list src_objs, py::list dst_objs, py::handle op_cls,
                  py::handle meta_cls, py::object pieces) {
  const Names& N = names_();
  if (!PyType_Check(op_cls.ptr()) || !PyType_Check(meta_cls.ptr())) throw py::type_error("classes expected");
  const int64_t n = ops.ndim() == 2 ? ops.shape(0) : 0;
  if (n && ops.shape(1) != 9) throw py::value_error("op rows must have 9 columns");
  const bool encode = !pieces.is_none();
  if (encode && (!PyList_Check(pieces.ptr()) || PyList_GET_SIZE(pieces.ptr()) != 0))
    throw py::value_error("pieces must be an empty list");
  py::list out(n);
  const int64_t* r = ops.data();
  for (int64_t i = 0; i < n; ++i, r += 9) {
    const int64_t nid = r[0], s_row = r[3], d_row = r[4], p_idx = r[5], p_deg = r[6], r0 = r[7], r1 = r[8];
    if (nid < 0 || nid >= int64_t(names.size()) || s_row < 0 || s_row >= int64_t(src_objs.size()) ||
        d_row < 0 || d_row >= int64_t(dst_objs.size()))
      throw py::value_error("malformed op row");
    PyObject* shard = PyList_GET_ITEM(dst_objs.ptr(), d_row);
    py::object piece;
    if (r0 >= 0) {
      py::object tp = tp_meta_of(shard);
      piece = derived(meta_cls.ptr(), shard, tp.ptr(), py::make_tuple(r0, r1).ptr());
    } else if (p_deg) {
      py::object tp = tp_meta_of(shard);
      if (!PyTuple_Check(tp.ptr()) || PyTuple_GET_SIZE(tp.ptr()) != 3) throw py::value_error("shard has no tp_meta");
      py::tuple ptp = py::make_tuple(py::reinterpret_borrow<py::object>(PyTuple_GET_ITEM(tp.ptr(), 0)), p_idx, p_deg);
      piece = derived(meta_cls.ptr(), shard, ptp.ptr(), Py_None);
    } else {
      piece = py::reinterpret_borrow<py::object>(shard);
    }
    PyObject* d;
    py::object op = bare_instance(op_cls.ptr(), &d);
    set(d, N.param_name, PyList_GET_ITEM(names.ptr(), nid));
    set(d, N.src_rank, py::int_(r[1]).ptr());
    set(d, N.dst_rank, py::int_(r[2]).ptr());
    set(d, N.src_meta, PyList_GET_ITEM(src_objs.ptr(), s_row));
    set(d, N.dst_meta, piece.ptr());
    set(d, N.dst_shard_meta, shard);
    if (encode && PyList_Append(pieces.ptr(), piece.ptr()) != 0) throw py::error_already_set();
    PyList_SET_ITEM(out.ptr(), i, op.release().ptr());
  }
  return out;
}

// sr_lower's op and meta tables for one destination rank's TransferOps:
// `shards` maps each name to its destination shard, `name_ids` to its id.
// Metas are numbered in first-use order (each object once per name); a piece
// is encoded relative to its shard: (0, 0) for the shard itself, else its tp
// index and degree (an unsplit piece of a split shard: (0, 1)) and rows.  An
// op encoded by the schedule (Encoded) whose shard is the one `shards` names
// is copied from its tables: its source meta gets a row of its own.
py::tuple encode_ops(py::list ops, py::dict shards, py::dict name_ids, const Encoded* E) {
  const Names& N = names_();
  E = live(E);
  const int64_t n = int64_t(ops.size());
  py::array_t<int64_t> op_rows({n, int64_t(9)});
  int64_t* orow = op_rows.mutable_data();
  std::vector<int64_t> metas;
  struct KeyHash {
    size_t operator()(const std::pair<PyObject*, int64_t>& k) const {
      return std::hash<PyObject*>()(k.first) * 31u + std::hash<int64_t>()(k.second);
    }
  };
  std::unordered_map<std::pair<PyObject*, int64_t>, int64_t, KeyHash> meta_of;   // (object, name id) -> row
  auto row_of = [&](PyObject* m, int64_t nid) -> int64_t {
    const std::pair<PyObject*, int64_t> key(m, nid);
    auto it = meta_of.find(key);
    if (it != meta_of.end()) return it->second;
    const int64_t row = int64_t(metas.size() / kMetaWords);
    metas.resize(metas.size() + kMetaWords);
    meta_row(m, 0, nid, metas.data() + row * kMetaWords);
    meta_of.emplace(key, row);
    return row;
  };
  for (int64_t k = 0; k < n; ++k, orow += 9) {
    PyObject* op = PyList_GET_ITEM(ops.ptr(), k);
    py::object name = attr(op, N.param_name);
    PyObject* nid_obj = PyDict_GetItemWithError(name_ids.ptr(), name.ptr());
    PyObject* shard = PyDict_GetItemWithError(shards.ptr(), name.ptr());
    if (!nid_obj || !shard) {
      if (PyErr_Occurred()) throw py::error_already_set();
      throw py::key_error("no shard for " + py::str(name).cast<std::string>());
    }
    const int64_t nid = as_int(nid_obj);
    int64_t w[kEncodingWords];
    PyObject* enc_shard = nullptr;
    if (E && E->get(op, w, /*source=*/true, &enc_shard) && enc_shard == shard) {
      orow[0] = nid;
      orow[1] = as_int(attr(op, N.src_rank).ptr());
      orow[2] = as_int(attr(op, N.dst_rank).ptr());
      const int64_t src_row = int64_t(metas.size() / kMetaWords);
      metas.insert(metas.end(), w, w + kMetaWords);
      metas[size_t(src_row * kMetaWords)] = 0;
      metas[size_t(src_row * kMetaWords + 1)] = nid;
      orow[3] = src_row;
      const std::pair<PyObject*, int64_t> key(shard, nid);
      auto it = meta_of.find(key);
      if (it == meta_of.end()) {
        const int64_t row = int64_t(metas.size() / kMetaWords);
        metas.insert(metas.end(), w + kMetaWords, w + 2 * kMetaWords);
        metas[size_t(row * kMetaWords)] = 0;
        metas[size_t(row * kMetaWords + 1)] = nid;
        it = meta_of.emplace(key, row).first;
      }
      orow[4] = it->second;
      std::copy(w + 2 * kMetaWords, w + kEncodingWords, orow + 5);
      continue;
    }
    py::object m = attr(op, N.dst_meta);
    int64_t idx = 0, deg = 0, r0 = -1, r1 = -1;
    if (m.ptr() != shard) {
      auto nm = [&]() { return py::str(name).cast<std::string>(); };   // for messages only
      py::object mk = kind_of(m.ptr()), sk = kind_of(shard);
      py::object ms = attr(m.ptr(), N.shape), ss = attr(shard, N.shape);
      const int same_kind = PyObject_RichCompareBool(mk.ptr(), sk.ptr(), Py_EQ);
      const int same_shape = PyObject_RichCompareBool(ms.ptr(), ss.ptr(), Py_EQ);
      if (same_kind < 0 || same_shape < 0) throw py::error_already_set();
      if (!same_kind || !same_shape)
        assertion(nm() + ": piece " + py::str(m).cast<std::string>() + " is not part of shard " +
                  py::str(py::handle(shard)).cast<std::string>());
      py::object tp = tp_meta_of(m.ptr()), stp = tp_meta_of(shard);
      if (tp.ptr() == Py_None) {   // an unsplit piece: the whole tensor
        deg = stp.ptr() != Py_None ? 1 : 0;
      } else {
        if (!PyTuple_Check(tp.ptr()) || PyTuple_GET_SIZE(tp.ptr()) != 3) throw py::value_error("malformed tp_meta");
        if (stp.ptr() != Py_None) {
          const int same_dim = PyObject_RichCompareBool(PyTuple_GET_ITEM(tp.ptr(), 0),
                                                        PyTuple_GET_ITEM(stp.ptr(), 0), Py_EQ);
          if (same_dim < 0) throw py::error_already_set();
          if (!same_dim)
            assertion(nm() + ": piece " + py::str(m).cast<std::string>() + " is split along another dim than shard " +
                      py::str(py::handle(shard)).cast<std::string>());
        }
        idx = as_int(PyTuple_GET_ITEM(tp.ptr(), 1));
        deg = as_int(PyTuple_GET_ITEM(tp.ptr(), 2));
      }
      py::object rows = rows_of(m.ptr());
      if (rows.ptr() != Py_None) {
        if (!PyTuple_Check(rows.ptr()) || PyTuple_GET_SIZE(rows.ptr()) != 2) throw py::value_error("malformed rows");
        r0 = as_int(PyTuple_GET_ITEM(rows.ptr(), 0));
        r1 = as_int(PyTuple_GET_ITEM(rows.ptr(), 1));
      }
    }
    py::object src = attr(op, N.src_meta);
    orow[0] = nid;
    orow[1] = as_int(attr(op, N.src_rank).ptr());
    orow[2] = as_int(attr(op, N.dst_rank).ptr());
    orow[3] = row_of(src.ptr(), nid);
    orow[4] = row_of(shard, nid);
    orow[5] = idx;
    orow[6] = deg;
    orow[7] = r0;
    orow[8] = r1;
  }
  const int64_t n_metas = int64_t(metas.size() / kMetaWords);
  py::array_t<int64_t> meta_arr({n_metas, kMetaWords});
  std::copy(metas.begin(), metas.end(), meta_arr.mutable_data());
  return py::make_tuple(meta_arr, op_rows);
}

// Elements of every op's piece (op.dst_meta): a row interval times the
// other dims, else the global size over the tp degree (TensorMeta.numel of
// a chunk piece).  Used to balance launch groups.  With `padded`, whether
// the piece belongs to a padded vocabulary shard (whose size is not its
// pieces' total: it also holds rows no piece covers).
int64_t piece_numel(PyObject* op, bool* padded = nullptr, const Encoded* E = nullptr) {
  const Names& N = names_();
  int64_t w[kEncodingWords];
  if (E && E->get(op, w, /*source=*/false)) {   // the piece alone
    // the schedule's encoding: shard row at kMetaWords (ndim at 3, shape
    // from 4, tp degree at 14, kind at 15), then the piece
    const int64_t* shard = w + kMetaWords;
    const int64_t nd = shard[3], p_deg = w[2 * kMetaWords + 1], r0 = w[2 * kMetaWords + 2],
                  r1 = w[2 * kMetaWords + 3];
    if (nd < 0 || nd > 8) throw py::value_error("malformed op encoding");
    if (padded) *padded = shard[15] == 1;
    int64_t v = 1;
    if (r0 >= 0) {
      v = r1 - r0;
      for (int64_t d = 1; d < nd; ++d) v *= shard[4 + d];
    } else {
      for (int64_t d = 0; d < nd; ++d) v *= shard[4 + d];
      const int64_t deg = p_deg > 0 ? p_deg : shard[14];
      if (deg > 0) v /= deg;
    }
    return v;
  }
  py::object m = attr(op, N.dst_meta);
  if (padded) {
    py::object kind = kind_of(m.ptr());
    const int eq = PyObject_RichCompareBool(kind.ptr(), N.vocab_pad, Py_EQ);
    if (eq < 0) throw py::error_already_set();
    *padded = eq != 0;
  }
  py::object shape = attr(m.ptr(), N.shape), tp = tp_meta_of(m.ptr()), rows = rows_of(m.ptr());
  if (!PyTuple_Check(shape.ptr())) throw py::type_error("TensorMeta.shape must be a tuple");
  const Py_ssize_t nd = PyTuple_GET_SIZE(shape.ptr());
  int64_t v = 1;
  if (rows.ptr() != Py_None) {
    if (!PyTuple_Check(rows.ptr()) || PyTuple_GET_SIZE(rows.ptr()) != 2) throw py::value_error("malformed rows");
    v = as_int(PyTuple_GET_ITEM(rows.ptr(), 1)) - as_int(PyTuple_GET_ITEM(rows.ptr(), 0));
    for (Py_ssize_t d = 1; d < nd; ++d) v *= as_int(PyTuple_GET_ITEM(shape.ptr(), d));
  } else {
    for (Py_ssize_t d = 0; d < nd; ++d) v *= as_int(PyTuple_GET_ITEM(shape.ptr(), d));
    if (tp.ptr() != Py_None) {
      if (!PyTuple_Check(tp.ptr()) || PyTuple_GET_SIZE(tp.ptr()) != 3) throw py::value_error("malformed tp_meta");
      const int64_t deg = as_int(PyTuple_GET_ITEM(tp.ptr(), 2));
      if (deg > 0) v /= deg;
    }
  }
  return v;
}

py::array_t<int64_t> piece_numels(py::list ops) {
  const int64_t n = int64_t(ops.size());
  py::array_t<int64_t> out({n});
  int64_t* o = out.mutable_data();
  for (int64_t k = 0; k < n; ++k) o[k] = piece_numel(PyList_GET_ITEM(ops.ptr(), k));
  return out;
}

// The ops grouped by tensor, tensors in order of first appearance: (op
// indices tensor by tensor, where each tensor's indices start (one entry
// per tensor plus the end), elements of each tensor's pieces, whether every
// tensor's ops are already consecutive -- the order is then the identity --,
// and {name: tensor index}).
py::tuple runs_of(py::list ops, const int64_t* e, Py_ssize_t n);

py::tuple name_runs(py::list ops) {
  py::array_t<int64_t> numel = piece_numels(ops);
  const int64_t* e = numel.data();
  const Py_ssize_t n = PyList_GET_SIZE(ops.ptr());
  return runs_of(ops, e, n);
}

// The ops of `rank` out of a whole schedule (any sequence; `positions`, when
// given, says where they are; `encoding`, the schedule's Encoded tables), and
// their name_runs, in one pass over the
// schedule: (ops, order, starts, elements
// per tensor, single, {name: tensor index}, padded per tensor, tensor indices
// largest first, running total of their elements in that order).  A padded
// tensor (a vocabulary shard with padding rows) has more elements than its
// pieces' total; every other tensor's size is its pieces' total.
py::tuple rank_runs(py::object schedule, int64_t rank, py::object positions, const Encoded* E) {
  const Names& N = names_();
  E = live(E);
  py::object seq = py::reinterpret_steal<py::object>(PySequence_Fast(schedule.ptr(), "ops must be a sequence"));
  if (!seq) throw py::error_already_set();
  const Py_ssize_t total = PySequence_Fast_GET_SIZE(seq.ptr());
  PyObject** items = PySequence_Fast_ITEMS(seq.ptr());
  // `positions`: where the schedule holds this rank's ops (ascending), used
  // when every one of them is in range and targets `rank`; else a scan
  std::vector<Py_ssize_t> cand;
  bool indexed = !positions.is_none();
  if (indexed) {
    const RowTable pos = positions.cast<RowTable>();
    indexed = pos.ndim() == 1;
    for (int64_t i = 0; indexed && i < pos.shape(0); ++i) {
      const int64_t k = pos.data()[i];
      indexed = k >= 0 && k < total && (i == 0 || k > pos.data()[i - 1]) &&
                as_int(attr(items[k], N.dst_rank).ptr()) == rank;
      cand.push_back(Py_ssize_t(k));
    }
  }
  if (!indexed) cand.clear();
  py::list ops;
  std::vector<int64_t> numel;
  std::vector<char> padded_op;
  const Py_ssize_t n_cand = indexed ? Py_ssize_t(cand.size()) : total;
  for (Py_ssize_t c = 0; c < n_cand; ++c) {
    const Py_ssize_t k = indexed ? cand[size_t(c)] : c;
    if (!indexed && as_int(attr(items[k], N.dst_rank).ptr()) != rank) continue;
    if (PyList_Append(ops.ptr(), items[k]) != 0) throw py::error_already_set();
    if (E) E->note(items[k], int64_t(k));
    bool padded = false;
    numel.push_back(piece_numel(items[k], &padded, E));
    padded_op.push_back(padded ? 1 : 0);
  }
  py::tuple runs = runs_of(ops, numel.data(), Py_ssize_t(numel.size()));
  const RowTable order = runs[0].cast<RowTable>(), starts = runs[1].cast<RowTable>();
  const int64_t m = starts.shape(0) - 1;
  py::array_t<bool> padded({m});
  bool* pd = padded.mutable_data();
  for (int64_t t = 0; t < m; ++t) {
    pd[t] = false;
    for (int64_t j = starts.data()[t]; j < starts.data()[t + 1]; ++j) pd[t] = pd[t] || padded_op[order.data()[j]];
  }
  // the launch order: tensors largest first (stable), and the running total
  // of their elements in that order
  const RowTable totals = runs[2].cast<RowTable>();
  std::vector<int64_t> idx(static_cast<size_t>(m));
  for (int64_t t = 0; t < m; ++t) idx[size_t(t)] = t;
  const int64_t* tot = totals.data();
  std::stable_sort(idx.begin(), idx.end(), [tot](int64_t a, int64_t b) { return tot[a] > tot[b]; });
  py::array_t<int64_t> launch({m});
  std::copy(idx.begin(), idx.end(), launch.mutable_data());
  py::list cum(m);
  int64_t acc = 0;
  for (int64_t i = 0; i < m; ++i) {
    acc += tot[idx[size_t(i)]];
    PyObject* v = PyLong_FromLongLong(acc);
    if (!v) throw py::error_already_set();
    PyList_SET_ITEM(cum.ptr(), i, v);
  }
  return py::make_tuple(ops, runs[0], runs[1], runs[2], runs[3], runs[4], padded, launch, cum);
}

py::tuple runs_of(py::list ops, const int64_t* e, Py_ssize_t n) {
  const Names& N = names_();
  // tensor id of every op: consecutive ops of one name (the usual case)
  // share the name object, so only a change of name consults the dict
  py::dict ids;
  std::vector<int64_t> nid(static_cast<size_t>(n)), sums;
  bool single = true;
  PyObject* prev_name = nullptr;
  int64_t prev = -1;
  for (Py_ssize_t k = 0; k < n; ++k) {
    py::object name = attr(PyList_GET_ITEM(ops.ptr(), k), N.param_name);
    int64_t id;
    if (name.ptr() == prev_name) {
      id = prev;
    } else {
      PyObject* found = PyDict_GetItemWithError(ids.ptr(), name.ptr());
      if (found) {
        id = as_int(found);
        if (id != prev) single = false;
      } else {
        if (PyErr_Occurred()) throw py::error_already_set();
        id = int64_t(sums.size());
        py::object v = py::reinterpret_steal<py::object>(PyLong_FromLongLong(id));
        if (!v || PyDict_SetItem(ids.ptr(), name.ptr(), v.ptr()) != 0) throw py::error_already_set();
        sums.push_back(0);
      }
      prev_name = name.ptr();   // alive: `ids` holds a reference
    }
    nid[size_t(k)] = id;
    sums[size_t(id)] += e[k];
    prev = id;
  }
  // op indices tensor by tensor (a counting sort, stable)
  const int64_t m = int64_t(sums.size());
  py::array_t<int64_t> order({int64_t(n)}), starts({m + 1}), total({m});
  int64_t* o = order.mutable_data();
  int64_t* st = starts.mutable_data();
  std::fill(st, st + m + 1, 0);
  for (Py_ssize_t k = 0; k < n; ++k) ++st[nid[size_t(k)] + 1];
  for (int64_t i = 0; i < m; ++i) st[i + 1] += st[i];
  std::vector<int64_t> fill(st, st + m);
  for (Py_ssize_t k = 0; k < n; ++k) o[fill[size_t(nid[size_t(k)])]++] = k;
  std::copy(sums.begin(), sums.end(), total.mutable_data());
  return py::make_tuple(order, starts, total, single, ids);
}

// The ops of the tensors `picked` (indices into runs_of's tensors, each
// once): tensor by tensor in `picked` order, each tensor's ops in schedule
// order.  A launch group, whose destinations are then allocated in the
// order the helper thread makes their blocks (AheadBlocks).
py::list take_ops(py::list ops, const RowTable& order, const RowTable& starts, const RowTable& picked) {
  const int64_t n_ops = int64_t(PyList_GET_SIZE(ops.ptr()));
  if (order.ndim() != 1 || order.shape(0) != n_ops || starts.ndim() != 1 || starts.shape(0) < 1 ||
      picked.ndim() != 1)
    throw py::value_error("take_ops: order, starts and picked must be 1-D, order one entry per op");
  const int64_t m = starts.shape(0) - 1;
  const int64_t *st = starts.data(), *o = order.data();
  const std::vector<int64_t> sel(picked.data(), picked.data() + picked.shape(0));
  std::vector<int64_t> sorted(sel);
  std::sort(sorted.begin(), sorted.end());
  Py_ssize_t total = 0;
  for (size_t j = 0; j < sorted.size(); ++j) {
    const int64_t i = sorted[j];
    if (i < 0 || i >= m || (j && sorted[j - 1] == i) || st[i] < 0 || st[i] > st[i + 1] || st[i + 1] > n_ops)
      throw py::value_error("take_ops: bad tensor index or runs");
    total += Py_ssize_t(st[i + 1] - st[i]);
  }
  py::list out(total);
  Py_ssize_t j = 0;
  for (int64_t i : sel)
    for (int64_t q = st[i]; q < st[i + 1]; ++q) {
      const int64_t k = o[q];
      if (k < 0 || k >= n_ops) throw py::value_error("take_ops: op index out of range");
      PyObject* op = PyList_GET_ITEM(ops.ptr(), k);
      Py_INCREF(op);
      PyList_SET_ITEM(out.ptr(), j++, op);
    }
  return out;
}

// The drop-in call's result: {name: {field: tensor}} with the names in
// order of first appearance in `ops` and each entry's fields in
// `field_order` (those present), from `target`, filled launch group by
// launch group.
py::dict ordered_result(py::list ops, py::dict target, py::list field_order) {
  const Names& N = names_();
  py::dict out;
  const Py_ssize_t n = PyList_GET_SIZE(ops.ptr()), nf = PyList_GET_SIZE(field_order.ptr());
  for (Py_ssize_t k = 0; k < n; ++k) {
    py::object name = attr(PyList_GET_ITEM(ops.ptr(), k), N.param_name);
    const int have = PyDict_Contains(out.ptr(), name.ptr());
    if (have < 0) throw py::error_already_set();
    if (have) continue;
    PyObject* entry = PyDict_GetItemWithError(target.ptr(), name.ptr());
    if (!entry) {
      if (PyErr_Occurred()) throw py::error_already_set();
      throw py::key_error(py::str(name).cast<std::string>());
    }
    // an entry whose fields already follow field_order is taken as it is
    bool in_order = PyDict_CheckExact(entry);
    {
      Py_ssize_t pos = 0, f = 0;
      PyObject *key, *value;
      while (in_order && PyDict_Next(entry, &pos, &key, &value)) {
        bool found = false;   // the key among the fields after the previous key's
        while (!found && f < nf) {
          PyObject* want = PyList_GET_ITEM(field_order.ptr(), f++);
          const int eq = want == key ? 1 : PyObject_RichCompareBool(want, key, Py_EQ);
          if (eq < 0) throw py::error_already_set();
          found = eq != 0;
        }
        in_order = found;
      }
    }
    if (in_order) {
      if (PyDict_SetItem(out.ptr(), name.ptr(), entry) != 0) throw py::error_already_set();
      continue;
    }
    py::dict e;
    for (Py_ssize_t f = 0; f < nf; ++f) {
      PyObject* field = PyList_GET_ITEM(field_order.ptr(), f);
      PyObject* t = PyDict_GetItemWithError(entry, field);
      if (t) {
        if (PyDict_SetItem(e.ptr(), field, t) != 0) throw py::error_already_set();
      } else if (PyErr_Occurred()) {
        throw py::error_already_set();
      }
    }
    if (PyDict_SetItem(out.ptr(), name.ptr(), e.ptr()) != 0) throw py::error_already_set();
  }
  return out;
}

}  // namespace

// The drop-in call's destination arena (an extension of
// execute_param_transfer): every destination tensor of `ops` in one
// allocation, field by field in `order`, names in schedule order within a
// field, each at a 256-byte aligned offset.  A name's shape is the actual
// shape of its destination shard: dst_shard_meta when attached, else the
// pieces' tp indices merged at the piece degree (infer_dst_shard).  A field
// in `targets` is bf16 (a recast target); any other takes the dtype of the
// name's source tensor.  Returns {name: {field: tensor}}.
py::dict arena_tensors(py::list ops, py::function source, py::list order, py::list targets, at::Device device) {
  const Names& N = names_();
  py::dict index;                          // name -> position in `groups`
  std::vector<std::vector<PyObject*>> groups;
  std::vector<py::object> names;
  for (py::handle op : ops) {
    py::object name = attr(op.ptr(), N.param_name);
    PyObject* at = PyDict_GetItemWithError(index.ptr(), name.ptr());
    if (!at && PyErr_Occurred()) throw py::error_already_set();
    size_t g;
    if (at) {
      g = size_t(PyLong_AsSize_t(at));
    } else {
      g = groups.size();
      index[name] = py::int_(g);
      groups.emplace_back();
      names.push_back(name);
    }
    groups[g].push_back(op.ptr());
  }
  const size_t n_names = names.size(), n_fields = order.size();
  std::vector<bool> is_target(n_fields, false);
  for (size_t k = 0; k < n_fields; ++k)
    for (py::handle t : targets)
      if (PyObject_RichCompareBool(order[k].ptr(), t.ptr(), Py_EQ) == 1) is_target[k] = true;
  std::vector<int64_t> ndim(n_names), numel(n_names, 1), dims(n_names * SR_MAX_DIMS, 0);
  std::vector<at::ScalarType> st(n_fields * n_names);
  py::dict sources;
  for (size_t i = 0; i < n_names; ++i) {
    PyObject* first = groups[i][0];
    auto nm = [&]() { return py::str(names[i]).cast<std::string>(); };   // for messages only
    sr_meta m;
    int64_t* row = reinterpret_cast<int64_t*>(&m);
    sr_internal::View v;
    py::object shard = shard_of(first);
    if (shard.ptr() != Py_None) {
      meta_row(shard.ptr(), 0, 0, row);
      v = sr_internal::view_of(m);
    } else {
      meta_row(attr(first, N.dst_meta).ptr(), 0, 0, row);
      if (m.row0 >= 0) assertion(nm() + ": vocab pieces need dst_shard_meta");
      v = sr_internal::view_of(m);
      if (m.tp_deg > 0 && groups[i].size() > 1) {
        std::vector<int64_t> idx;
        for (PyObject* op : groups[i]) {
          py::object tp = tp_meta_of(attr(op, N.dst_meta).ptr());
          if (!PyTuple_Check(tp.ptr()) || PyTuple_GET_SIZE(tp.ptr()) != 3)
            throw py::value_error("tp_meta must be (slice_dim, tp_index, tp_deg)");
          idx.push_back(as_int(PyTuple_GET_ITEM(tp.ptr(), 1)));
        }
        std::sort(idx.begin(), idx.end());
        const int64_t cnt = int64_t(idx.size()), T = m.tp_deg;
        bool ok = T % cnt == 0 && idx[0] % cnt == 0;
        for (int64_t j = 0; ok && j < cnt; ++j) ok = idx[j] == idx[0] + j;
        if (!ok) {
          std::string list = "[";
          for (int64_t j = 0; j < cnt; ++j) list += (j ? ", " : "") + std::to_string(idx[j]);
          assertion(nm() + ": pieces " + list + "] at degree " + std::to_string(T) + " do not form one shard");
        }
        v.tp_index = idx[0] / cnt;
        v.tp_deg = T / cnt;
        v.whole = false;
      }
    }
    if (!sr_internal::actual_shape(v, &dims[i * SR_MAX_DIMS]))
      assertion(nm() + ": destination shard shape overflows");
    ndim[i] = m.ndim;
    for (int64_t d = 0; d < m.ndim; ++d) {
      const int64_t e = dims[i * SR_MAX_DIMS + d];
      if (e < 0 || __builtin_mul_overflow(numel[i], e, &numel[i])) assertion(nm() + ": bad destination shape");
    }
    // dtypes: bf16 for recast targets, else the source tensor's
    py::object rank = attr(first, N.src_rank);
    py::object sd = lookup(sources.ptr(), rank.ptr());
    if (!sd) {
      sd = source(rank);
      sources[rank] = sd;
    }
    py::object entry = lookup(sd.ptr(), names[i].ptr());
    if (!entry) assertion("param missing in source " + nm());
    for (size_t k = 0; k < n_fields; ++k) {
      if (is_target[k]) {
        st[k * n_names + i] = at::kBFloat16;
        continue;
      }
      py::object t = lookup(entry.ptr(), order[k].ptr());
      if (!t || !THPVariable_Check(t.ptr()))
        assertion("expected_sub_fields mismatch: " + nm() + " has no tensor " + py::str(order[k]).cast<std::string>());
      st[k * n_names + i] = THPVariable_Unpack(t.ptr()).scalar_type();
    }
  }
  // field by field, names in schedule order, each start 256-byte aligned
  std::vector<int64_t> offset(n_fields * n_names);
  int64_t end = 0;
  for (size_t j = 0; j < n_fields * n_names; ++j) {
    const int64_t bytes = numel[j % n_names] * int64_t(c10::elementSize(st[j]));
    end = (end + 255) / 256 * 256;
    offset[j] = end;
    end += bytes;
  }
  at::Tensor buf = at::empty({std::max<int64_t>(1, end)}, at::TensorOptions().dtype(at::kByte).device(device));
  const c10::Storage& storage = buf.storage();
  std::vector<py::dict> entries(n_names);
  py::dict out;
  for (size_t i = 0; i < n_names; ++i) out[names[i]] = entries[i];
  for (size_t k = 0; k < n_fields; ++k)
    for (size_t i = 0; i < n_names; ++i) {
      const size_t j = k * n_names + i;
      auto impl = c10::make_intrusive<c10::TensorImpl>(c10::Storage(storage), buf.key_set(),
                                                       c10::scalarTypeToTypeMeta(st[j]));
      impl->set_storage_offset(offset[j] / int64_t(c10::elementSize(st[j])));
      impl->set_sizes_contiguous(at::IntArrayRef(&dims[i * SR_MAX_DIMS], size_t(ndim[i])));
      py::object wrapped = py::reinterpret_steal<py::object>(THPVariable_Wrap(at::Tensor(std::move(impl))));
      if (PyDict_SetItem(entries[i].ptr(), order[k].ptr(), wrapped.ptr()) != 0) throw py::error_already_set();
    }
  return out;
}

// Tensors over device memory this process does not own -- another process's
// hand-off allocation mapped here: one tensor per (byte offset, shape, dtype)
// of `views` at `base` on cuda:`device_index`.  The tensors never free the
// memory and must not outlive its mapping.
py::list device_views(uint64_t base, py::list views, int64_t device_index) {
  py::list out;
  const at::Device dev(at::kCUDA, c10::DeviceIndex(device_index));
  for (py::handle v : views) {
    if (!PyTuple_Check(v.ptr()) || PyTuple_GET_SIZE(v.ptr()) != 3)
      throw py::value_error("a view is (byte offset, shape, dtype)");
    const uint64_t off = py::reinterpret_borrow<py::object>(PyTuple_GET_ITEM(v.ptr(), 0)).cast<uint64_t>();
    const std::vector<int64_t> shape =
        py::reinterpret_borrow<py::object>(PyTuple_GET_ITEM(v.ptr(), 1)).cast<std::vector<int64_t>>();
    PyObject* dt = PyTuple_GET_ITEM(v.ptr(), 2);
    if (!THPDtype_Check(dt)) throw py::type_error("view dtype must be a torch.dtype");
    const at::ScalarType st = reinterpret_cast<THPDtype*>(dt)->scalar_type;
    if (off % c10::elementSize(st) != 0) throw py::value_error("view offset not aligned to its element size");
    at::Tensor t = at::from_blob(reinterpret_cast<void*>(base + off), shape, [](void*) {},
                                 at::TensorOptions().dtype(st).device(dev));
    out.append(py::reinterpret_steal<py::object>(THPVariable_Wrap(std::move(t))));
  }
  return out;
}

// ------------------------------------------------------------ one launch group's plan
// ReshardPlan.from_sources in one call: the ops grouped by tensor, each
// tensor's destination shard (op.dst_shard_meta, else `infer_shard(ops of the
// name)`), the op / meta tables (encode_ops), the source tensors
// (collect_sources), then sr_lower and sr_plan_create of libsuika_reshard.so
// on its tables, with nothing copied through Python in between.  With
// `gather`, also the destination tensors -- fresh ones (alloc_dst), or those
// of `dst_part` checked against their slots (bind_dst) -- and sr_gather into
// them on `stream` (the drop-in call's direct route).  Raises
// suika_amd._lib.PlanError (or ReshardError for device and memory failures)
// with the library's message, tensor ids replaced by names.

namespace {

PyObject* lib_exception(const char* name) {
  py::object mod = py::module_::import("suika_amd._lib");
  py::object cls = mod.attr(name);
  return cls.release().ptr();   // a new reference, kept for the process
}

const char* status_name(int rc) {
  switch (rc) {
    case SR_OK: return "SR_OK";
    case SR_EINVAL: return "SR_EINVAL";
    case SR_EBOUNDS: return "SR_EBOUNDS";
    case SR_EALIGN: return "SR_EALIGN";
    case SR_EOVERLAP: return "SR_EOVERLAP";
    case SR_EHIP: return "SR_EHIP";
    case SR_ENOMEM: return "SR_ENOMEM";
    case SR_EDTYPE: return "SR_EDTYPE";
    default: return nullptr;
  }
}

// "<what>: <status>: <message>", as suika_amd._lib.check words it.
[[noreturn]] void raise_status(int rc, const char* what, const std::string& msg) {
  static PyObject* plan_error = lib_exception("PlanError");
  static PyObject* reshard_error = lib_exception("ReshardError");
  const char* name = status_name(rc);
  const std::string text = std::string(what) + ": " + (name ? name : std::to_string(rc)) + ": " + msg;
  PyErr_SetString(rc == SR_EHIP || rc == SR_ENOMEM ? reshard_error : plan_error, text.c_str());
  throw py::error_already_set();
}

// "#<id>" in a library message -> the tensor's name.
std::string with_names(const char* msg, py::list names) {
  std::string out;
  for (const char* c = msg; *c; ++c) {
    if (*c == '#' && c[1] >= '0' && c[1] <= '9') {
      size_t id = 0;
      while (c[1] >= '0' && c[1] <= '9') id = id * 10 + size_t(*++c - '0');
      out += id < names.size() ? py::str(names[id]).cast<std::string>() : "#" + std::to_string(id);
    } else {
      out += *c;
    }
  }
  return out;
}

template <typename T>
py::array table(const T* rows, int64_t n, py::dtype dt) {
  if (dt.itemsize() != py::ssize_t(sizeof(T))) throw py::value_error("record dtype does not match the library");
  py::array out(dt, std::vector<py::ssize_t>{py::ssize_t(n)});
  if (n) std::memcpy(out.mutable_data(), rows, size_t(n) * sizeof(T));
  return out;
}

py::array_t<int64_t> key_table(const sr_slot_key* rows, int64_t n) {
  py::array_t<int64_t> out({n, kKeyWords});
  if (n) std::memcpy(out.mutable_data(), rows, size_t(n) * sizeof(sr_slot_key));
  return out;
}

static_assert(sizeof(sr_slot_key) == kKeyWords * sizeof(int64_t), "an sr_slot_key row is 13 int64 words");
static_assert(sizeof(sr_src_spec) == kSpecWords * sizeof(int64_t), "an sr_src_spec row is 10 int64 words");
static_assert(sizeof(sr_op) == 9 * sizeof(int64_t), "an sr_op row is 9 int64 words");

}  // namespace

py::tuple plan_sources(py::list ops, py::function source, py::list fields, py::list recast_names,
                       py::function infer_shard, int64_t device_index, const std::string& who,
                       uint32_t tile_bytes, uint32_t max_blocks, uint32_t flags, py::dtype tensor_dt,
                       py::dtype piece_dt, bool gather, uint64_t stream, py::object dst_part,
                       py::object ahead, bool host_ok, const Encoded* encoding) {
  // host addresses are for sr_stage_pack alone: a kernel must never see one
  if (gather && host_ok) throw py::value_error("host-resident sources cannot be gathered on the device");
  const Names& N = names_();
  const Py_ssize_t n = PyList_GET_SIZE(ops.ptr());
  const int64_t nf = int64_t(fields.size());
  if (int64_t(recast_names.size()) != nf) throw py::value_error("one recast name (or None) per field");
  std::vector<int64_t> recast(static_cast<size_t>(nf));
  for (int64_t f = 0; f < nf; ++f) recast[size_t(f)] = recast_names[f].is_none() ? 0 : 1;
  // tensors in order of first appearance, their ops, the destination rank
  py::dict name_ids;
  py::list names, op_names(n);
  std::vector<PyObject*> first_op;   // per tensor
  std::vector<size_t> op_nid(n);
  std::vector<int64_t> ranks;
  for (Py_ssize_t k = 0; k < n; ++k) {
    PyObject* op = PyList_GET_ITEM(ops.ptr(), k);
    py::object name = attr(op, N.param_name);
    PyObject* id = PyDict_GetItemWithError(name_ids.ptr(), name.ptr());
    size_t nid;
    if (id) {
      nid = size_t(as_int(id));
    } else {
      if (PyErr_Occurred()) throw py::error_already_set();
      nid = first_op.size();
      py::int_ v(nid);
      if (PyDict_SetItem(name_ids.ptr(), name.ptr(), v.ptr()) != 0) throw py::error_already_set();
      names.append(name);
      first_op.push_back(op);
    }
    op_nid[k] = nid;
    const int64_t r = as_int(attr(op, N.dst_rank).ptr());
    if (std::find(ranks.begin(), ranks.end(), r) == ranks.end()) ranks.push_back(r);
    PyList_SET_ITEM(op_names.ptr(), k, name.release().ptr());
  }
  if (ranks.size() > 1) {
    std::sort(ranks.begin(), ranks.end());
    std::string list;
    for (int64_t r : ranks) list += (list.empty() ? "" : ", ") + std::to_string(r);
    assertion("ops target several ranks [" + list + "]");
  }
  py::dict shards;
  std::vector<std::vector<Py_ssize_t>> members;   // each tensor's ops, when a shard is inferred
  for (size_t i = 0; i < first_op.size(); ++i) {
    py::object shard = shard_of(first_op[i]);
    if (shard.ptr() == Py_None) {
      if (members.empty()) {
        members.resize(first_op.size());
        for (Py_ssize_t k = 0; k < n; ++k) members[op_nid[size_t(k)]].push_back(k);
      }
      py::list group;
      for (Py_ssize_t k : members[i]) group.append(py::handle(PyList_GET_ITEM(ops.ptr(), k)));
      shard = infer_shard(group);
    }
    shards[names[i]] = shard;
  }
  py::tuple col = collect_sources(ops, source, fields, device_index, who, host_ok);
  py::array_t<int64_t> specs = col[0].cast<py::array_t<int64_t>>();
  py::array_t<uint64_t> ptrs = col[2].cast<py::array_t<uint64_t>>();
  // one torch dtype per (tensor, field) across its sources: the library
  // compares element types, which several torch dtypes share
  std::vector<PyObject*> first(first_op.size() * size_t(nf), nullptr);
  {
    py::list dtypes = col[1].cast<py::list>();
    for (Py_ssize_t k = 0; k < n; ++k)
      for (int64_t f = 0; f < nf; ++f) {
        PyObject* dt = PyList_GET_ITEM(dtypes.ptr(), k * nf + f);
        PyObject*& seen = first[op_nid[k] * size_t(nf) + size_t(f)];
        if (!seen) seen = dt;
        if (seen != dt)
          assertion(py::str(names[op_nid[k]]).cast<std::string>() + "/" + py::str(fields[f]).cast<std::string>() +
                    ": dtype differs between sources");
      }
  }
  // Fresh destinations: with `ahead` = ({name: tensor index}, AheadBlocks)
  // their blocks are being made on the helper thread (see AheadBlocks).
  const at::Device device(at::kCUDA, c10::DeviceIndex(device_index));
  std::unique_ptr<FreshTensors> fresh;
  BlockJob* job = nullptr;
  std::vector<size_t> op_pos;
  if (gather && dst_part.is_none()) {
    fresh = std::make_unique<FreshTensors>(device);
    if (!ahead.is_none()) {
      py::tuple a = ahead.cast<py::tuple>();
      if (a.size() != 2 || !PyDict_Check(a[0].ptr())) throw py::value_error("ahead must be (dict, AheadBlocks)");
      PyObject* index = a[0].ptr();
      const AheadBlocks* blocks = a[1].cast<const AheadBlocks*>();
      if (blocks->job() && blocks->fields() == nf) {
        std::vector<size_t> pos(first_op.size(), kNoBlock);
        for (size_t i = 0; i < first_op.size(); ++i) {
          PyObject* at = PyDict_GetItemWithError(index, names[i].ptr());
          if (!at) {
            if (PyErr_Occurred()) throw py::error_already_set();
            continue;
          }
          pos[i] = blocks->pos(as_int(at));
        }
        op_pos.resize(size_t(n));
        for (Py_ssize_t k = 0; k < n; ++k) op_pos[size_t(k)] = pos[op_nid[size_t(k)]];
        job = blocks->job();
      }
    }
  }
  py::tuple enc = encode_ops(ops, shards, name_ids, encoding);
  py::array_t<int64_t> metas = enc[0].cast<py::array_t<int64_t>>(), op_rows = enc[1].cast<py::array_t<int64_t>>();
  const int64_t no_recast = 0;

  sr_lowering* low = nullptr;
  int rc = sr_lower(reinterpret_cast<const sr_meta*>(metas.data()), metas.shape(0),
                    reinterpret_cast<const sr_op*>(op_rows.data()), int64_t(n),
                    reinterpret_cast<const sr_src_spec*>(specs.data()), nf, nf ? recast.data() : &no_recast, &low);
  if (rc != SR_OK) raise_status(rc, "sr_lower", with_names(sr_last_error(), names));
  std::unique_ptr<sr_lowering, void (*)(sr_lowering*)> hold(low, sr_lowering_destroy);
  // source slot s reads (op, field) = src_key[s].op, .field
  py::array_t<uint64_t> src_ptrs({low->n_src});
  {
    uint64_t* o = src_ptrs.mutable_data();
    const uint64_t* in = ptrs.data();
    for (int64_t s = 0; s < low->n_src; ++s) o[s] = in[low->src_key[s].op * nf + low->src_key[s].field];
  }
  if (low->n_src > INT32_MAX || low->n_dst > INT32_MAX || low->n_pieces > INT32_MAX || low->n_peers > INT32_MAX)
    throw py::value_error("lowering too large");
  sr_plan_options opt{tile_bytes, max_blocks, flags, 0};
  sr_plan* plan = nullptr;
  rc = sr_plan_create(low->src, int32_t(low->n_src), low->dst, int32_t(low->n_dst), int32_t(low->n_peers),
                      low->pieces, int32_t(low->n_pieces), &opt, &plan);
  if (rc != SR_OK) raise_status(rc, "sr_plan_create", sr_last_error());
  std::unique_ptr<sr_plan, void (*)(sr_plan*)> plan_hold(plan, sr_plan_destroy);
  py::list peers, peer_bytes;
  for (int64_t i = 0; i < low->n_peers; ++i) {
    uint64_t b = 0;
    if ((rc = sr_plan_peer_bytes(plan, int32_t(i), &b)) != SR_OK)
      raise_status(rc, "sr_plan_peer_bytes", sr_last_error());
    peers.append(low->peer_rank[i]);
    peer_bytes.append(b);
  }
  sr_plan_info info{};
  if ((rc = sr_plan_info_get(plan, &info)) != SR_OK)
    raise_status(rc, "sr_plan_info_get", sr_last_error());
  py::bytes info_bytes(reinterpret_cast<const char*>(&info), sizeof(info));
  py::array_t<int64_t> dst_rows = key_table(low->dst_key, low->n_dst), empty_rows = key_table(low->empty, low->n_empty);
  py::object part = py::none();
  if (gather) {
    // fresh destinations (or the caller's, each checked against its slot),
    // then the gather on `stream`
    py::array_t<uint64_t> dst_ptrs;
    if (dst_part.is_none()) {
      py::tuple made = alloc_dst(dst_rows, empty_rows, op_names, fields, recast_names, col[1].cast<py::list>(),
                                 device, fresh.get(), job, &op_pos);
      part = made[0];
      dst_ptrs = made[1].cast<py::array_t<uint64_t>>();
    } else {
      if (!PyDict_Check(dst_part.ptr())) throw py::type_error("destinations must be a dict");
      dst_ptrs = bind_dst(dst_part.cast<py::dict>(), dst_rows, op_names, fields, recast_names,
                          col[1].cast<py::list>(), device);
      part = dst_part;
    }
    rc = sr_gather(plan, reinterpret_cast<const void* const*>(src_ptrs.data()),
                   reinterpret_cast<void* const*>(dst_ptrs.data()), reinterpret_cast<hipStream_t>(stream));
    if (rc != SR_OK) raise_status(rc, "sr_gather", sr_last_error());
  }
  py::tuple out = py::make_tuple(
      reinterpret_cast<uintptr_t>(plan), names, shards, op_names,
      ranks.empty() ? py::object(py::none()) : py::object(py::int_(ranks[0])), col[1], src_ptrs,
      table(low->src, low->n_src, tensor_dt), table(low->dst, low->n_dst, tensor_dt),
      table(low->pieces, low->n_pieces, piece_dt), peers, key_table(low->src_key, low->n_src),
      dst_rows, empty_rows, peer_bytes, info_bytes, part);
  plan_hold.release();   // owned by the caller from here on
  return out;
}

PYBIND11_MODULE(_suika_host, m) {
  m.doc() = "Per-tensor host work of execute_param_transfer (source checks, destination allocation)";
  m.def("collect_sources", &collect_sources, py::arg("ops"), py::arg("source"), py::arg("fields"),
        py::arg("device_index"), py::arg("who"), py::arg("host_ok") = false);
  m.def(
      "alloc_dst",
      [](const RowTable& rows, const RowTable& empty_rows, py::list names, py::list fields, py::list recast_names,
         py::list dtypes, at::Device device) {
        return alloc_dst(rows, empty_rows, names, fields, recast_names, dtypes, device);
      },
      py::arg("rows"), py::arg("empty_rows"), py::arg("names"), py::arg("fields"), py::arg("recast_names"),
      py::arg("dtypes"), py::arg("device"));
  m.def("bind_dst", &bind_dst, py::arg("part"), py::arg("rows"), py::arg("names"), py::arg("fields"),
        py::arg("recast_names"), py::arg("dtypes"), py::arg("device"));
  m.def("arena_views", &arena_views, py::arg("buf"), py::arg("names"), py::arg("fields"), py::arg("rows"),
        py::arg("dtypes"));
  m.def("arena_tensors", &arena_tensors, py::arg("ops"), py::arg("source"), py::arg("order"), py::arg("targets"),
        py::arg("device"));
  py::class_<Encoded>(m, "ScheduleEncoding",
                      "a schedule and the tables its ops were made from (sr_op table, both layouts' sr_meta "
                      "tables and meta objects, each op's piece meta)")
      .def(py::init<py::object, py::object>(), py::arg("schedule"), py::arg("tables"));
  py::class_<AheadBlocks>(m, "AheadBlocks",
                          "Destination blocks of one drop-in call, made ahead on the helper thread")
      .def("finish", &AheadBlocks::finish, "stop the helper on these blocks and free those no tensor took");
  m.def(
      "start_blocks",
      [](int64_t device_index, const RowTable& order, const RowTable& numel, py::array_t<bool> padded,
         std::vector<int64_t> itemsize, std::vector<int64_t> copies) {
        return std::make_unique<AheadBlocks>(device_index, order, numel, padded, std::move(itemsize),
                                             std::move(copies));
      },
      py::arg("device_index"), py::arg("order"), py::arg("numel"), py::arg("padded"), py::arg("itemsize"),
      py::arg("copies"),
      "the destination blocks of tensors `order` (launch order), handed to the helper thread now");
  m.def(
      "blocks_ahead",
      [] { return py::make_tuple(g_blocks_taken.load(), g_blocks_missed.load()); },
      "(destination tensors built on blocks the helper thread made, those allocated on the calling "
      "thread instead) since the process started");
  m.def("encode_layout", &encode_layout, py::arg("layout"), py::arg("names"), py::arg("objs"));
  m.def("piece_numels", &piece_numels, py::arg("ops"));
  m.def("name_runs", &name_runs, py::arg("ops"));
  m.def("rank_runs", &rank_runs, py::arg("schedule"), py::arg("rank"), py::arg("positions") = py::none(),
        py::arg("encoding") = static_cast<const Encoded*>(nullptr));
  m.def("take_ops", &take_ops, py::arg("ops"), py::arg("order"), py::arg("starts"), py::arg("picked"));
  m.def("ordered_result", &ordered_result, py::arg("ops"), py::arg("target"), py::arg("field_order"));
  m.def(
      "encode_ops",
      &encode_ops, py::arg("ops"), py::arg("shards"), py::arg("name_ids"),
      py::arg("encoding") = static_cast<const Encoded*>(nullptr));
  m.def("make_ops", &make_ops, py::arg("ops"), py::arg("names"), py::arg("src_objs"), py::arg("dst_objs"),
        py::arg("op_cls"), py::arg("meta_cls"), py::arg("pieces") = py::none());
  m.def("device_views", &device_views, py::arg("base"), py::arg("views"), py::arg("device_index"));
  m.def("plan_sources", &plan_sources, py::arg("ops"), py::arg("source"), py::arg("fields"),
        py::arg("recast_names"), py::arg("infer_shard"), py::arg("device_index"), py::arg("who"),
        py::arg("tile_bytes"), py::arg("max_blocks"), py::arg("flags"), py::arg("tensor_dtype"),
        py::arg("piece_dtype"), py::arg("gather") = false, py::arg("stream") = 0, py::arg("dst_part") = py::none(),
        py::arg("ahead") = py::none(), py::arg("host_ok") = false,
        py::arg("encoding") = static_cast<const Encoded*>(nullptr));
}
