// Python launch callable of one planned operator instance (module fgw_amd._launch).
//
// The reference's launch callable (operators/mha/kernels/
// mha_paged_decode_ascend_v7.py:471-498) checks its tensors, allocates the
// output (and the split workspace) and launches on the current stream. This
// type does the same work in one C++ call, through the C ABI of
// libfgw_mha.so (include/fgw_mha.h): the time from the Python call to the
// first kernel's dispatch is a few microseconds instead of the tens of
// attribute reads, allocations and ctypes conversions of a Python body.
//
// The C entry points are not linked: their addresses come from the library
// that fgw_amd._lib loaded with ctypes, so the process holds one copy of it
// and one error state. Host code only; no device code is compiled here.
#include <Python.h>

#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/autograd/python_variable.h>

#include <cstring>
#include <map>
#include <utility>
#include <vector>

#include "../../include/fgw_mha.h"

namespace {

typedef int (*FwdFn)(const fgw_mha_shape*, const fgw_mha_plan_t*, const fgw_mha_tensors*,
                     hipStream_t);
typedef const char* (*ErrFn)(void);

struct Launcher {
  PyObject_HEAD
  fgw_mha_shape shape;
  fgw_mha_plan_t plan;
  FwdFn fwd;
  ErrFn last_error;
  int device;
  at::ScalarType dtype;
  int64_t out_sizes[4];
  int64_t kv_sizes[3];
  int64_t table_sizes[2];
  int64_t len_sizes[1];
  int64_t ws_floats;
};

bool same(c10::IntArrayRef a, const int64_t* b, size_t n) {
  if (a.size() != n) return false;
  for (size_t i = 0; i < n; ++i)
    if (a[i] != b[i]) return false;
  return true;
}

PyObject* value_error(const char* msg) {
  PyErr_SetString(PyExc_ValueError, msg);
  return nullptr;
}

int launcher_init(Launcher* self, PyObject* args, PyObject* kwds) {
  static const char* kw[] = {"shape", "plan", "device", "fwd", "last_error", nullptr};
  Py_buffer shape_buf, plan_buf;
  int device = 0;
  unsigned long long fwd = 0, err = 0;
  if (!PyArg_ParseTupleAndKeywords(args, kwds, "y*y*iKK", const_cast<char**>(kw), &shape_buf,
                                   &plan_buf, &device, &fwd, &err))
    return -1;
  const bool sizes_ok = shape_buf.len == (Py_ssize_t)sizeof(fgw_mha_shape) &&
                        plan_buf.len == (Py_ssize_t)sizeof(fgw_mha_plan_t);
  if (sizes_ok) {
    std::memcpy(&self->shape, shape_buf.buf, sizeof(fgw_mha_shape));
    std::memcpy(&self->plan, plan_buf.buf, sizeof(fgw_mha_plan_t));
  }
  PyBuffer_Release(&shape_buf);
  PyBuffer_Release(&plan_buf);
  if (!sizes_ok) {
    PyErr_SetString(PyExc_TypeError, "shape/plan buffers do not match the C ABI structs");
    return -1;
  }
  if (!fwd || !err) {
    PyErr_SetString(PyExc_TypeError, "fwd and last_error must be C function addresses");
    return -1;
  }
  self->fwd = reinterpret_cast<FwdFn>(static_cast<uintptr_t>(fwd));
  self->last_error = reinterpret_cast<ErrFn>(static_cast<uintptr_t>(err));
  self->device = device;
  const fgw_mha_shape& s = self->shape;
  self->dtype = s.dtype == FGW_MHA_BFLOAT16 ? at::kBFloat16 : at::kHalf;
  self->out_sizes[0] = s.batch;
  self->out_sizes[1] = s.sq;
  self->out_sizes[2] = s.heads;
  self->out_sizes[3] = s.dim;
  self->kv_sizes[0] = s.pool_rows;
  self->kv_sizes[1] = s.heads;
  self->kv_sizes[2] = s.dim;
  self->table_sizes[0] = s.batch;
  self->table_sizes[1] = s.width;
  self->len_sizes[0] = s.batch;
  self->ws_floats = self->plan.parts_floats + self->plan.lse_floats;
  return 0;
}

// Arrival counters of the fused split merge (fgw_mha_tensors.arrivals), one
// zeroed int32 buffer per (device, stream), grown as plans need more. Every
// completed call leaves its counters at zero, so calls in stream order share
// the buffer, and calls on other streams (which may overlap) use their own.
// While the stream is being captured into a graph the call merges in a
// second launch instead: a replay may run on any stream. The buffers live
// until the process ends (the map is never destroyed, so no device memory is
// released after the runtime has shut down).
int32_t* arrival_counters(int device, hipStream_t stream, int64_t need) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &status) != hipSuccess || status != hipStreamCaptureStatusNone)
    return nullptr;
  static auto* buffers = new std::map<std::pair<int, uintptr_t>, at::Tensor>();
  // A buffer replaced by a larger one stays allocated: a kernel still in
  // flight may be counting in it, and memory the caching allocator handed
  // to another stream could be written under it.
  static auto* retired = new std::vector<at::Tensor>();
  at::Tensor& buf = (*buffers)[{device, reinterpret_cast<uintptr_t>(stream)}];
  if (!buf.defined() || buf.numel() < need) {
    if (buf.defined()) retired->push_back(buf);
    buf = at::zeros({need}, at::TensorOptions().device(c10::kCUDA, device).dtype(at::kInt));
  }
  return static_cast<int32_t*>(buf.data_ptr());
}

// The checks of one call, in the order and with the messages of the Python
// operator (shape, then dtype, then int32 metadata, then device/layout).
PyObject* check_detail(const Launcher* self, const at::Tensor* x) {
  if (!same(x[0].sizes(), self->out_sizes, 4) || !same(x[1].sizes(), self->kv_sizes, 3) ||
      !same(x[2].sizes(), self->kv_sizes, 3) || !same(x[3].sizes(), self->table_sizes, 2) ||
      !same(x[4].sizes(), self->len_sizes, 1))
    return value_error("tensor shapes do not match the built kernel");
  for (int i = 0; i < 3; ++i)
    if (x[i].scalar_type() != self->dtype) return value_error("matching FP16/BF16 Q/K/V required");
  if (x[3].scalar_type() != at::kInt || x[4].scalar_type() != at::kInt)
    return value_error("int32 metadata required");
  return value_error("contiguous inputs on the same GPU required");
}

PyObject* launcher_call(PyObject* obj, PyObject* args, PyObject* kwargs) {
  Launcher* self = reinterpret_cast<Launcher*>(obj);
  if ((kwargs && PyDict_Size(kwargs)) || PyTuple_GET_SIZE(args) != 5) {
    PyErr_SetString(PyExc_TypeError, "expected (q, k_cache, v_cache, block_table, cache_seqlens)");
    return nullptr;
  }
  at::Tensor x[5];
  for (int i = 0; i < 5; ++i) {
    PyObject* a = PyTuple_GET_ITEM(args, i);
    if (!THPVariable_Check(a)) {
      PyErr_SetString(PyExc_TypeError, "arguments must be torch tensors");
      return nullptr;
    }
    x[i] = THPVariable_Unpack(a);
  }
  bool ok = same(x[0].sizes(), self->out_sizes, 4) && same(x[1].sizes(), self->kv_sizes, 3) &&
            same(x[2].sizes(), self->kv_sizes, 3) && same(x[3].sizes(), self->table_sizes, 2) &&
            same(x[4].sizes(), self->len_sizes, 1) && x[0].scalar_type() == self->dtype &&
            x[1].scalar_type() == self->dtype && x[2].scalar_type() == self->dtype &&
            x[3].scalar_type() == at::kInt && x[4].scalar_type() == at::kInt;
  for (int i = 0; ok && i < 5; ++i) {
    const c10::Device d = x[i].device();
    ok = d.is_cuda() && d.index() == self->device && x[i].is_contiguous();
  }
  if (!ok) return check_detail(self, x);

  try {
    const at::TensorOptions on_device = at::TensorOptions().device(c10::kCUDA, self->device);
    at::Tensor out = at::empty(c10::IntArrayRef(self->out_sizes, 4), on_device.dtype(self->dtype));
    at::Tensor ws;
    fgw_mha_tensors t;
    t.q = x[0].data_ptr();
    t.k_cache = x[1].data_ptr();
    t.v_cache = x[2].data_ptr();
    t.block_table = static_cast<const int32_t*>(x[3].data_ptr());
    t.cache_seqlens = static_cast<const int32_t*>(x[4].data_ptr());
    t.out = out.data_ptr();
    t.parts = nullptr;
    t.lse = nullptr;
    t.arrivals = nullptr;
    if (self->ws_floats > 0) {
      ws = at::empty({self->ws_floats}, on_device.dtype(at::kFloat));
      t.parts = static_cast<float*>(ws.data_ptr());
      t.lse = t.parts + self->plan.parts_floats;
    }
    const hipStream_t stream = c10::hip::getCurrentHIPStream(self->device).stream();
    if (self->plan.arrival_counters > 0)
      t.arrivals = arrival_counters(self->device, stream, self->plan.arrival_counters);
    const int rc = self->fwd(&self->shape, &self->plan, &t, stream);
    if (rc != FGW_MHA_OK) {
      PyErr_SetString(rc == FGW_MHA_EHIP ? PyExc_RuntimeError : PyExc_ValueError,
                      self->last_error());
      return nullptr;
    }
    return THPVariable_Wrap(std::move(out));
  } catch (const std::exception& e) {
    PyErr_SetString(PyExc_RuntimeError, e.what());
    return nullptr;
  }
}

PyTypeObject LauncherType = {PyVarObject_HEAD_INIT(nullptr, 0)};

PyModuleDef module_def = {PyModuleDef_HEAD_INIT, "_launch",
                          "C++ launch callable over the fgw_mha C ABI", -1, nullptr};

}  // namespace

PyMODINIT_FUNC PyInit__launch(void) {
  LauncherType.tp_name = "fgw_amd._launch.Launcher";
  LauncherType.tp_basicsize = sizeof(Launcher);
  LauncherType.tp_flags = Py_TPFLAGS_DEFAULT | Py_TPFLAGS_BASETYPE;
  LauncherType.tp_doc =
      "Launcher(shape, plan, device, fwd, last_error): calls fgw_mha_fwd on the current stream";
  LauncherType.tp_new = PyType_GenericNew;
  LauncherType.tp_init = reinterpret_cast<initproc>(launcher_init);
  LauncherType.tp_call = launcher_call;
  if (PyType_Ready(&LauncherType) < 0) return nullptr;
  PyObject* m = PyModule_Create(&module_def);
  if (!m) return nullptr;
  Py_INCREF(&LauncherType);
  if (PyModule_AddObject(m, "Launcher", reinterpret_cast<PyObject*>(&LauncherType)) < 0) {
    Py_DECREF(&LauncherType);
    Py_DECREF(m);
    return nullptr;
  }
  return m;
}
