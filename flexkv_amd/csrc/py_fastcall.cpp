// _fkv_py: the per-call path of flexkv_amd.c_ext.transfer_kv_blocks and
// transfer_kv_blocks_kv_ptrs as a CPython extension (vectorcall, no argument
// tuple).  It unpacks the torch tensors in C++, checks them, takes the current
// torch stream and calls the C-ABI entry with the GIL released, the work that
// csrc/bindings.cpp:25-55 does for the reference through pybind11.
//
// The C-ABI functions are not linked: c_ext hands over their addresses in the
// library it already loaded (bind()), so both routes drive one copy of the
// library's state.  When a check fails the functions return False without
// raising, and the Python wrapper then names the argument and the reason; a
// failed transfer raises RuntimeError with the library's last error.
#include <Python.h>

#include <c10/hip/HIPFunctions.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/autograd/python_variable.h>

#include <climits>
#include <cstdint>
#include <cstring>
#include <exception>

namespace {

using TransferFn = int (*)(int, int, int, const int64_t*, void* const*, int64_t, int64_t,
                           const int64_t*, void*, int64_t, int64_t, int64_t, int64_t, int64_t,
                           void*, int, int, int, int);
using TransferKvPtrsFn = int (*)(int, int, int, const int64_t*, void* const*, int64_t,
                                 const int64_t*, void*, int64_t, int64_t, int64_t, int64_t,
                                 int64_t, void*, int, int, int, int);
using LastErrorFn = const char* (*)();

TransferFn g_transfer = nullptr;
TransferKvPtrsFn g_transfer_kv_ptrs = nullptr;
LastErrorFn g_last_error = nullptr;
int g_mode_kernel = 0;
int g_mode_ce = 1;
int g_device_visible = -1;   // unknown until the first call that needs the current stream

// an int64 host tensor, contiguous (the id and pointer tables)
bool int64_host(PyObject* o, const at::Tensor** out) {
  if (!THPVariable_Check(o)) return false;
  const at::Tensor& t = THPVariable_Unpack(o);
  if (t.scalar_type() != at::kLong || !t.device().is_cpu() || !t.is_contiguous()) return false;
  *out = &t;
  return true;
}

bool as_i64(PyObject* o, int64_t* v) {
  const long long x = PyLong_AsLongLong(o);
  if (x == -1 && PyErr_Occurred()) return false;
  *v = x;
  return true;
}

// an argument the C-ABI takes as int
bool as_int(PyObject* o, int* v) {
  const long x = PyLong_AsLong(o);
  if (x == -1 && PyErr_Occurred()) return false;
  if (x < INT_MIN || x > INT_MAX) {
    PyErr_Format(PyExc_OverflowError, "%ld does not fit a C int", x);
    return false;
  }
  *v = static_cast<int>(x);
  return true;
}

// block and layer counts the C-ABI takes as int
bool count_fits(int64_t n, const char* what) {
  if (n <= INT_MAX) return true;
  PyErr_Format(PyExc_RuntimeError, "%lld %s in one call; at most %d", static_cast<long long>(n),
               what, INT_MAX);
  return false;
}

// a numpy scalar bool (numpy 1.x names its type numpy.bool_, 2.x numpy.bool)
bool is_numpy_bool(PyObject* o) {
  const char* n = Py_TYPE(o)->tp_name;
  return std::strcmp(n, "numpy.bool_") == 0 || std::strcmp(n, "numpy.bool") == 0;
}

// use_ce_transfer: a bool (Python or numpy) picks the copy engines or the
// kernel, an integer is a mode
bool as_mode(PyObject* o, int* mode) {
  if (PyBool_Check(o) || is_numpy_bool(o)) {
    const int r = PyObject_IsTrue(o);
    if (r < 0) return false;
    *mode = r ? g_mode_ce : g_mode_kernel;
    return true;
  }
  int64_t v = 0;
  if (!as_i64(o, &v)) return false;
  *mode = static_cast<int>(v);
  return true;
}

bool as_flag(PyObject* o, int* v) {
  const int r = PyObject_IsTrue(o);
  if (r < 0) return false;
  *v = r;
  return true;
}

// The stream argument: None -> the current torch stream of the current device.
// Returns 0 with *ok false (no Python error) when no device is visible.
bool stream_of(PyObject* o, void** s, bool* ok) {
  *ok = true;
  if (o != Py_None) {
    *s = PyLong_AsVoidPtr(o);
    return !(*s == nullptr && PyErr_Occurred());
  }
  if (g_device_visible < 0) g_device_visible = c10::hip::device_count() > 0 ? 1 : 0;
  if (!g_device_visible) {
    *ok = false;
    return true;
  }
  try {
    *s = c10::hip::getCurrentHIPStream().stream();
  } catch (const std::exception& e) {
    PyErr_SetString(PyExc_RuntimeError, e.what());
    return false;
  }
  return true;
}

PyObject* finish(int rc) {
  if (rc == 0) Py_RETURN_NONE;
  const char* msg = g_last_error ? g_last_error() : nullptr;
  if (msg && *msg)
    PyErr_SetString(PyExc_RuntimeError, msg);
  else
    PyErr_Format(PyExc_RuntimeError, "transfer failed (%d)", rc);
  return nullptr;
}

PyObject* not_bound() {
  PyErr_SetString(PyExc_RuntimeError, "_fkv_py.bind() has not been called");
  return nullptr;
}

// transfer_kv_blocks(gpu_block_ids, gpu_layer_ptrs, gpu_kv_stride, gpu_block_stride,
//                    cpu_block_ids, cpu_tensor, cpu_kv_stride, cpu_layer_stride,
//                    cpu_block_stride, chunk, start_layer, transfer_sms,
//                    is_host_to_device, use_ce_transfer, is_mla, stream)
PyObject* transfer_kv_blocks(PyObject*, PyObject* const* a, Py_ssize_t n) {
  if (!g_transfer) return not_bound();
  if (n != 16) {
    PyErr_Format(PyExc_TypeError, "transfer_kv_blocks takes 16 arguments (%zd given)", n);
    return nullptr;
  }
  const at::Tensor *gids, *ptrs, *cids;
  if (!int64_host(a[0], &gids) || !int64_host(a[1], &ptrs) || !int64_host(a[4], &cids) ||
      !THPVariable_Check(a[5]))
    Py_RETURN_FALSE;
  const at::Tensor& cpu = THPVariable_Unpack(a[5]);
  const int64_t nb = gids->numel();
  if (cids->numel() != nb) Py_RETURN_FALSE;
  int64_t gkv, gblk, ckv, clay, cblk, chunk;
  int start, sms, h2d, mla, mode;
  if (!as_i64(a[2], &gkv) || !as_i64(a[3], &gblk) || !as_i64(a[6], &ckv) ||
      !as_i64(a[7], &clay) || !as_i64(a[8], &cblk) || !as_i64(a[9], &chunk) ||
      !as_int(a[10], &start) || !as_int(a[11], &sms) || !as_flag(a[12], &h2d) ||
      !as_mode(a[13], &mode) || !as_flag(a[14], &mla) || !count_fits(nb, "block ids") ||
      !count_fits(ptrs->numel(), "layer pointers"))
    return nullptr;
  void* stream = nullptr;
  bool ok = true;
  if (!stream_of(a[15], &stream, &ok)) return nullptr;
  if (!ok) Py_RETURN_FALSE;
  const int64_t* g = static_cast<const int64_t*>(gids->data_ptr());
  void* const* p = static_cast<void* const*>(ptrs->data_ptr());
  const int64_t* c = static_cast<const int64_t*>(cids->data_ptr());
  void* host = cpu.data_ptr();
  const int nl = static_cast<int>(ptrs->numel());
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = g_transfer(static_cast<int>(nb), start, nl, g, p, gkv, gblk, c, host, ckv, clay, cblk, 0,
                  chunk, stream, sms, h2d, mode, mla);
  Py_END_ALLOW_THREADS
  return finish(rc);
}

// transfer_kv_blocks_kv_ptrs(gpu_block_ids, gpu_kv_ptrs, gpu_block_stride,
//                            cpu_block_ids, cpu_tensor, cpu_kv_stride, cpu_layer_stride,
//                            cpu_block_stride, chunk, start_layer, transfer_sms,
//                            is_host_to_device, use_ce_transfer, is_mla, stream)
PyObject* transfer_kv_blocks_kv_ptrs(PyObject*, PyObject* const* a, Py_ssize_t n) {
  if (!g_transfer_kv_ptrs) return not_bound();
  if (n != 15) {
    PyErr_Format(PyExc_TypeError, "transfer_kv_blocks_kv_ptrs takes 15 arguments (%zd given)", n);
    return nullptr;
  }
  const at::Tensor *gids, *ptrs, *cids;
  if (!int64_host(a[0], &gids) || !int64_host(a[1], &ptrs) || !int64_host(a[3], &cids) ||
      !THPVariable_Check(a[4]))
    Py_RETURN_FALSE;
  const at::Tensor& cpu = THPVariable_Unpack(a[4]);
  const int64_t nb = gids->numel();
  int64_t gblk, ckv, clay, cblk, chunk;
  int start, sms, h2d, mla, mode;
  if (!as_i64(a[2], &gblk) || !as_i64(a[5], &ckv) || !as_i64(a[6], &clay) ||
      !as_i64(a[7], &cblk) || !as_i64(a[8], &chunk) || !as_int(a[9], &start) ||
      !as_int(a[10], &sms) || !as_flag(a[11], &h2d) || !as_mode(a[12], &mode) ||
      !as_flag(a[13], &mla) || !count_fits(nb, "block ids") ||
      !count_fits(ptrs->numel(), "layer pointers"))
    return nullptr;
  const int kv = mla ? 1 : 2;
  if (cids->numel() != nb || ptrs->numel() % kv) Py_RETURN_FALSE;
  void* stream = nullptr;
  bool ok = true;
  if (!stream_of(a[14], &stream, &ok)) return nullptr;
  if (!ok) Py_RETURN_FALSE;
  const int64_t* g = static_cast<const int64_t*>(gids->data_ptr());
  void* const* p = static_cast<void* const*>(ptrs->data_ptr());
  const int64_t* c = static_cast<const int64_t*>(cids->data_ptr());
  void* host = cpu.data_ptr();
  const int nl = static_cast<int>(ptrs->numel() / kv);
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = g_transfer_kv_ptrs(static_cast<int>(nb), start, nl, g, p, gblk, c, host, ckv, clay, cblk,
                          0, chunk, stream, sms, h2d, mode, mla);
  Py_END_ALLOW_THREADS
  return finish(rc);
}

// bind(transfer, transfer_kv_ptrs, last_error, mode_kernel, mode_ce): addresses
// of the C-ABI functions in the loaded library and the two mode values.
PyObject* bind(PyObject*, PyObject* const* a, Py_ssize_t n) {
  if (n != 5) {
    PyErr_SetString(PyExc_TypeError, "bind takes 5 arguments");
    return nullptr;
  }
  void* f[3];
  for (int i = 0; i < 3; ++i) {
    f[i] = PyLong_AsVoidPtr(a[i]);
    if (!f[i]) {
      if (!PyErr_Occurred()) PyErr_SetString(PyExc_ValueError, "null function address");
      return nullptr;
    }
  }
  int64_t mk = 0, mc = 0;
  if (!as_i64(a[3], &mk) || !as_i64(a[4], &mc)) return nullptr;
  g_transfer = reinterpret_cast<TransferFn>(f[0]);
  g_transfer_kv_ptrs = reinterpret_cast<TransferKvPtrsFn>(f[1]);
  g_last_error = reinterpret_cast<LastErrorFn>(f[2]);
  g_mode_kernel = static_cast<int>(mk);
  g_mode_ce = static_cast<int>(mc);
  Py_RETURN_NONE;
}

PyMethodDef kMethods[] = {
    {"transfer_kv_blocks", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(
                               &transfer_kv_blocks)),
     METH_FASTCALL, "Checked per-call path of c_ext.transfer_kv_blocks (16 positional)."},
    {"transfer_kv_blocks_kv_ptrs", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(
                                       &transfer_kv_blocks_kv_ptrs)),
     METH_FASTCALL, "Checked per-call path of c_ext.transfer_kv_blocks_kv_ptrs (15 positional)."},
    {"bind", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(&bind)), METH_FASTCALL,
     "Hand over the C-ABI function addresses and mode values."},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_fkv_py", nullptr, -1, kMethods,
                       nullptr, nullptr, nullptr, nullptr};

}  // namespace

PyMODINIT_FUNC PyInit__fkv_py() { return PyModule_Create(&kModule); }
