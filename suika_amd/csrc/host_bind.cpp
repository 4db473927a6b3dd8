// host_bind.cpp -- per-tensor host work of the drop-in operator, native
// (suika_amd/lib/_suika_host.so, a CPython extension on torch's C++ API).
//
// execute_param_transfer (Suika/migration.py:397-556) touches every source
// tensor (to check it and read its shape, dtype and address) and allocates
// every destination tensor.  In Python that costs a few microseconds per
// tensor, which on transfers of many small tensors exceeds the GPU time of
// the copy itself.  These two functions do the same walks over the state
// dicts and the slot tables in C++:
//
//   collect_sources: (ops, rank -> state dict, fields) -> source specs
//                    (sr_src_spec rows), dtypes and device addresses, with
//                    the same checks and messages as the Python host;
//   alloc_dst:       destination slot rows (sr_slot_key) -> fresh tensors in
//                    {name: {field: tensor}} and their addresses;
//   bind_dst:        caller-provided destinations (an arena's views) checked
//                    against the slot rows -> their addresses;
//   arena_views:     the same dict of typed views into one allocation.
//
// No device work happens here; the tensors come from torch's caching
// allocator on the device's current stream, as torch.empty would.

#include <torch/extension.h>
#include <torch/csrc/Dtype.h>
#include <torch/csrc/DynamicTypes.h>
#include <pybind11/numpy.h>

#include <cstdint>
#include <string>
#include <vector>

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

constexpr int64_t kSpecWords = 10;   // sr_src_spec: dtype, ndim, shape[8]
constexpr int64_t kKeyWords = 13;    // sr_slot_key: op, field, recast, dtype, ndim, shape[8]

// The source tensor of every (op, field), checked once.  `source(rank)`
// returns a rank's state dict; it is called once per rank, when the first op
// of that rank is reached, so errors come in op order as in the reference's
// loop (migration.py:426-494).
py::tuple collect_sources(py::list ops, py::function source, py::list fields, int64_t device_index,
                          const std::string& who) {
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
    py::handle op = ops[k];
    py::object rank = op.attr("src_rank");
    py::object name = op.attr("param_name");
    py::object sd = lookup(sources.ptr(), rank.ptr());
    if (!sd) {
      sd = source(rank);
      sources[rank] = sd;
    }
    py::object entry = lookup(sd.ptr(), name.ptr());
    const std::string nm = py::str(name).cast<std::string>();
    if (!entry) assertion(who + ": param missing in source " + nm);
    for (int64_t f = 0; f < nf; ++f) {
      py::handle field = fields[f];
      py::object obj = lookup(entry.ptr(), field.ptr());
      if (!obj) assertion("expected_sub_fields mismatch: " + nm + " has no " + py::str(field).cast<std::string>());
      if (!THPVariable_Check(obj.ptr()))
        assertion("source " + nm + "/" + py::str(field).cast<std::string>() + " of rank " +
                  py::str(rank).cast<std::string>() + ": not a tensor");
      const at::Tensor& t = THPVariable_Unpack(obj.ptr());
      const int64_t code = sr_code(t.scalar_type());
      const int64_t nd = t.dim();
      if (!t.is_cuda() || t.get_device() != device_index || !t.is_contiguous() || code < 0 || nd > 8) {
        // the rare path: build the message
        const std::string fs = py::str(field).cast<std::string>();
        const std::string what = "source " + nm + "/" + fs + " of rank " + py::str(rank).cast<std::string>();
        if (!t.is_cuda() || t.get_device() != device_index)
          assertion(what + " is on " + t.device().str() + ", not on " + want_device);
        if (!t.is_contiguous()) assertion(what + " is not contiguous");
        assertion("source " + nm + "/" + fs + ": " + py::str(dtype_object(t.scalar_type())).cast<std::string>() +
                  ", " + std::to_string(nd) + "-D is not supported by the reshard engine");
      }
      int64_t* row = sp + (k * nf + f) * kSpecWords;
      row[0] = code;
      row[1] = nd;
      for (int64_t d = 0; d < nd; ++d) row[2 + d] = t.size(d);
      dtypes[k * nf + f] = dtype_object(t.scalar_type());
      pp[k * nf + f] = reinterpret_cast<uint64_t>(t.data_ptr());
    }
  }
  return py::make_tuple(specs, dtypes, ptrs);
}

using RowTable = py::array_t<int64_t, py::array::c_style | py::array::forcecast>;

// Fresh destination tensors for the slot rows (and the zero-element ones).
py::tuple alloc_dst(const RowTable& rows, const RowTable& empty_rows, py::list names, py::list fields,
                    py::list recast_names, py::list dtypes, at::Device device) {
  const int64_t nf = int64_t(fields.size());
  py::dict out;
  const int64_t n = rows.ndim() == 2 ? rows.shape(0) : 0;
  py::array_t<uint64_t> ptrs({n});
  uint64_t* pp = ptrs.mutable_data();
  const at::TensorOptions base = at::TensorOptions().device(device);
  for (int pass = 0; pass < 2; ++pass) {
    const auto& tbl = pass == 0 ? rows : empty_rows;
    const int64_t m = tbl.ndim() == 2 ? tbl.shape(0) : 0;
    if (m && tbl.shape(1) != kKeyWords) throw py::value_error("slot rows must have 13 columns");
    const int64_t* r = tbl.data();
    for (int64_t i = 0; i < m; ++i, r += kKeyWords) {
      const int64_t k = r[0], f = r[1], is_recast = r[2], nd = r[4];
      if (k < 0 || k >= int64_t(names.size()) || f < 0 || f >= nf || nd < 0 || nd > 8)
        throw py::value_error("malformed slot row");
      at::ScalarType st;
      py::handle field;
      if (is_recast) {
        st = at::kBFloat16;
        field = recast_names[f];
      } else {
        py::handle dt = dtypes[k * nf + f];
        if (!THPDtype_Check(dt.ptr())) throw py::type_error("dtypes must hold torch.dtype objects");
        st = reinterpret_cast<THPDtype*>(dt.ptr())->scalar_type;
        field = fields[f];
      }
      at::Tensor t = at::empty(at::IntArrayRef(r + 5, size_t(nd)), base.dtype(st));
      py::handle name = names[k];
      PyObject* entry = PyDict_GetItemWithError(out.ptr(), name.ptr());
      if (!entry) {
        if (PyErr_Occurred()) throw py::error_already_set();
        py::dict fresh;
        out[name] = fresh;
        entry = fresh.ptr();
      }
      py::object wrapped = py::reinterpret_steal<py::object>(THPVariable_Wrap(t));
      if (PyDict_SetItem(entry, field.ptr(), wrapped.ptr()) != 0) throw py::error_already_set();
      if (pass == 0) pp[i] = reinterpret_cast<uint64_t>(t.data_ptr());
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
    const std::string what = "(" + py::repr(name).cast<std::string>() + ", " +
                             py::repr(field).cast<std::string>() + ")";
    py::object entry = lookup(part.ptr(), name.ptr());
    py::object obj = entry ? lookup(entry.ptr(), field.ptr()) : py::object();
    if (!obj) assertion(what + ": no destination tensor");
    if (!THPVariable_Check(obj.ptr())) assertion(what + ": not a tensor");
    const at::Tensor& t = THPVariable_Unpack(obj.ptr());
    if (t.device() != device)
      assertion(what + ": tensor is on " + t.device().str() + ", the kernels run on " + device.str());
    if (!t.is_contiguous()) assertion(what + ": tensor is not contiguous");
    if (t.scalar_type() != st) assertion(what + ": dtype differs from the planned one");
    bool same = t.dim() == nd;
    for (int64_t d = 0; same && d < nd; ++d) same = t.size(d) == r[5 + d];
    if (!same) assertion(what + ": shape differs from the planned one");
    pp[i] = reinterpret_cast<uint64_t>(t.data_ptr());
  }
  return ptrs;
}

// Typed views of one byte buffer (a destination arena): row i is
// (byte offset, ndim, shape[8]); out[names[i]][fields[i]] is the view.
py::dict arena_views(const at::Tensor& buf, py::list names, py::list fields, const RowTable& rows,
                     py::list dtypes) {
  const int64_t n = rows.ndim() == 2 ? rows.shape(0) : 0;
  if (n && rows.shape(1) != 10) throw py::value_error("arena rows must have 10 columns");
  if (int64_t(names.size()) != n || int64_t(fields.size()) != n || int64_t(dtypes.size()) != n)
    throw py::value_error("one name, field and dtype per arena row");
  if (buf.scalar_type() != at::kByte || buf.dim() != 1 || !buf.is_contiguous())
    throw py::value_error("the arena must be a contiguous 1-D uint8 tensor");
  py::dict out;
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
    if (r[0] < 0 || r[0] + bytes > buf.size(0) || r[0] % int64_t(c10::elementSize(st)) != 0)
      throw py::value_error("arena row outside the buffer or misaligned");
    at::Tensor v = buf.narrow(0, r[0], bytes).view(st).view(at::IntArrayRef(r + 2, size_t(nd)));
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

}  // namespace

PYBIND11_MODULE(_suika_host, m) {
  m.doc() = "Per-tensor host work of execute_param_transfer (source checks, destination allocation)";
  m.def("collect_sources", &collect_sources, py::arg("ops"), py::arg("source"), py::arg("fields"),
        py::arg("device_index"), py::arg("who"));
  m.def("alloc_dst", &alloc_dst, py::arg("rows"), py::arg("empty_rows"), py::arg("names"), py::arg("fields"),
        py::arg("recast_names"), py::arg("dtypes"), py::arg("device"));
  m.def("bind_dst", &bind_dst, py::arg("part"), py::arg("rows"), py::arg("names"), py::arg("fields"),
        py::arg("recast_names"), py::arg("dtypes"), py::arg("device"));
  m.def("arena_views", &arena_views, py::arg("buf"), py::arg("names"), py::arg("fields"), py::arg("rows"),
        py::arg("dtypes"));
}
