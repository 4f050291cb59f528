// Native entry of the standalone cast: checks the tensors and calls sr_cast.
//
// A cast of up to a few million elements is bound by the host: the HIP
// launch itself costs about 2.2 us, and reaching it through a Python
// wrapper and ctypes added about 4 us (tensor checks, argument conversion,
// the foreign call).  This CPython extension takes the tensors directly,
// makes the output checks the wrapper made, and calls the C ABI's sr_cast
// through the address the Python side binds once, so the launch path costs
// little more than the launch.
//
// bind(address)
//   Keep the address of sr_cast (int (*)(const void*, void*, int64_t, int,
//   int, uint32_t, uint32_t, int, void*)), taken from the loaded library.
//
// cast(x, out, dtype_code, rule, seed, offset, threads, stream) -> int
//   x: contiguous FP32 tensor; out: contiguous tensor of x's shape and
//   device with the dtype of `dtype_code` (sr_dtype), sharing no byte with
//   x.  Raises ValueError when out breaks that, or when x is not a
//   contiguous FP32 GPU tensor, before anything is launched; otherwise
//   calls sr_cast with x's device current (set and restored only when it is
//   not) and returns its status (0 on success; nothing is launched for an
//   empty x).  seed and offset are taken modulo 2^32; `stream` is the raw
//   handle of a stream on x's device.

#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <c10/core/DeviceGuard.h>
#include <torch/csrc/autograd/python_variable.h>

#include <cstdint>
#include <exception>

namespace {

using CastFn = int (*)(const void*, void*, int64_t, int, int, uint32_t, uint32_t, int, void*);
CastFn g_cast = nullptr;

// sr_dtype codes of include/sr_states_hip.h.
bool dtype_matches(int code, c10::ScalarType type) {
  switch (code) {
    case 0: return type == c10::ScalarType::Float;
    case 1: return type == c10::ScalarType::BFloat16;
    case 2: return type == c10::ScalarType::Half;
    case 3: return type == c10::ScalarType::Float8_e4m3fn;
    case 4: return type == c10::ScalarType::Float8_e5m2;
    default: return false;
  }
}

PyObject* value_error(const char* message) {
  PyErr_SetString(PyExc_ValueError, message);
  return nullptr;
}

PyObject* bind(PyObject*, PyObject* args) {
  unsigned long long address = 0;
  if (!PyArg_ParseTuple(args, "K", &address)) return nullptr;
  if (address == 0) return value_error("null sr_cast address");
  g_cast = reinterpret_cast<CastFn>(static_cast<uintptr_t>(address));
  Py_RETURN_NONE;
}

PyObject* cast(PyObject*, PyObject* args) {
  PyObject *x_obj, *out_obj;
  int code, rule, threads;
  unsigned long long seed, offset, stream;
  if (!PyArg_ParseTuple(args, "OOiiKKiK", &x_obj, &out_obj, &code, &rule, &seed, &offset, &threads, &stream)) {
    return nullptr;
  }
  if (!THPVariable_Check(x_obj) || !THPVariable_Check(out_obj)) {
    PyErr_SetString(PyExc_TypeError, "x and out must be tensors");
    return nullptr;
  }
  const at::Tensor& x = THPVariable_Unpack(x_obj);
  const at::Tensor& out = THPVariable_Unpack(out_obj);
  // The output first: workgroups read x and write out concurrently, so any
  // shared byte would make the result depend on their timing.
  if (!dtype_matches(code, out.scalar_type()) || out.sizes() != x.sizes() || out.device() != x.device() ||
      !out.is_contiguous()) {
    return value_error("out must be a contiguous tensor of the requested dtype, shape and device");
  }
  const int64_t n = x.numel();
  if (n) {
    const auto x_start = reinterpret_cast<uintptr_t>(x.const_data_ptr());
    const auto out_start = reinterpret_cast<uintptr_t>(out.const_data_ptr());
    if (x_start < out_start + out.nbytes() && out_start < x_start + x.nbytes()) {
      return value_error("out must not overlap the input");
    }
  }
  if (!x.is_cuda() || x.scalar_type() != c10::ScalarType::Float || !x.is_contiguous()) {
    return value_error("the cast input must be a contiguous FP32 tensor on the GPU");
  }
  if (n == 0) return PyLong_FromLong(0);
  if (g_cast == nullptr) {
    PyErr_SetString(PyExc_RuntimeError, "the cast launcher is not bound to sr_cast");
    return nullptr;
  }
  int status = 0;
  try {
    const c10::DeviceGuard guard(x.device());
    status = g_cast(x.const_data_ptr(), out.data_ptr(), n, code, rule, static_cast<uint32_t>(seed),
                    static_cast<uint32_t>(offset), threads, reinterpret_cast<void*>(static_cast<uintptr_t>(stream)));
  } catch (const std::exception& error) {  // the device guard: no such device
    PyErr_SetString(PyExc_RuntimeError, error.what());
    return nullptr;
  }
  return PyLong_FromLong(status);
}

PyMethodDef methods[] = {
    {"bind", bind, METH_VARARGS, "Keep the address of the C ABI's sr_cast."},
    {"cast", cast, METH_VARARGS, "Check the tensors and call sr_cast; returns its status."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef module = {PyModuleDef_HEAD_INIT, "_cast_launch", "Native entry of the standalone cast.", -1, methods};

}  // namespace

PyMODINIT_FUNC PyInit__cast_launch(void) { return PyModule_Create(&module); }
