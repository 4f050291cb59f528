// Native entries of the single-tensor launches: the standalone cast and the
// functional AdamW and momentum-SGD updates.
//
// A launch over up to a few million elements is bound by the host: the HIP
// launch itself costs about 2.2 us, and reaching it through a Python wrapper
// and ctypes added about 4 us to a cast (tensor checks, argument conversion,
// the foreign call) and more to an update.  This CPython extension takes the
// tensors directly, makes the tensor checks the Python wrappers made, with
// their messages, and calls the C ABI's entry points through the addresses
// the Python side binds once.
//
// bind(cast, adamw_step, sgdm_step)
//   Keep the addresses of sr_cast, sr_adamw_step and sr_sgdm_step, taken
//   from the loaded library.
//
// cast(x, out, dtype_code, rule, seed, offset, threads, stream) -> int
//   x: contiguous FP32 tensor; out: contiguous tensor of x's shape and
//   device with the dtype of `dtype_code` (sr_dtype), sharing no byte with
//   x.  Raises ValueError when out breaks that, or when x is not a
//   contiguous FP32 GPU tensor, before anything is launched.
//
// adamw_step(p, g, m, v, m_code, m_rule, v_code, v_rule, scalars, key,
//            offset, block_size, stream) -> int
// sgdm_step(p, g, u, u_code, u_rule, scalars, key, offset, block_size,
//           stream) -> int
//   The tensor checks of the fused single-tensor updates
//   (sr_states/triton/_optimizer.py:24-60): GPU tensors on one device, of
//   one shape, contiguous; FP32 or BF16 parameter and gradient; no byte of
//   the parameter or a state shared with another operand (the gradient is
//   only read).  `scalars` is the tuple of the launch's FP32 scalars as the
//   host computed them (sr_adamw_hparams' eight fields in order, or
//   sr_sgdm_hparams' two), each rounded to FP32 here as ctypes rounds a
//   Python float.  Raises TypeError or ValueError before anything is
//   launched; nothing is launched for empty tensors.
//
// Each entry calls the C ABI with the first tensor's device current (set and
// restored only when it is not) and the GIL released, and returns its
// status.  Non-empty tensors without device memory (wrapper subclasses) are
// refused with ValueError.  seed, key and offset are taken modulo 2^32;
// `stream` is the raw handle of a stream on that device.

#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <c10/core/DeviceGuard.h>
#include <torch/csrc/autograd/python_variable.h>

#include <cstdint>
#include <exception>
#include <initializer_list>
#include <string>

#include "../../include/sr_states_hip.h"

namespace {

using CastFn = int (*)(const void*, void*, int64_t, int, int, uint32_t, uint32_t, int, void*);
using AdamWFn = int (*)(void*, const void*, void*, void*, int64_t, int, int, int, int, int, int,
                        const sr_adamw_hparams*, uint32_t, uint32_t, int, void*);
using SgdmFn = int (*)(void*, const void*, void*, int64_t, int, int, int, int, const sr_sgdm_hparams*, uint32_t,
                       uint32_t, int, void*);
CastFn g_cast = nullptr;
AdamWFn g_adamw = nullptr;
SgdmFn g_sgdm = nullptr;

// sr_dtype codes of include/sr_states_hip.h.
bool dtype_matches(int code, c10::ScalarType type) {
  switch (code) {
    case SR_F32: return type == c10::ScalarType::Float;
    case SR_BF16: return type == c10::ScalarType::BFloat16;
    case SR_F16: return type == c10::ScalarType::Half;
    case SR_E4M3: return type == c10::ScalarType::Float8_e4m3fn;
    case SR_E5M2: return type == c10::ScalarType::Float8_e5m2;
    default: return false;
  }
}

PyObject* fail(PyObject* type, const char* message) {
  PyErr_SetString(type, message);
  return nullptr;
}

void* address(unsigned long long value) { return reinterpret_cast<void*>(static_cast<uintptr_t>(value)); }

PyObject* bind(PyObject*, PyObject* args) {
  unsigned long long cast = 0, adamw = 0, sgdm = 0;
  if (!PyArg_ParseTuple(args, "KKK", &cast, &adamw, &sgdm)) return nullptr;
  if (!cast || !adamw || !sgdm) return fail(PyExc_ValueError, "null entry point address");
  g_cast = reinterpret_cast<CastFn>(address(cast));
  g_adamw = reinterpret_cast<AdamWFn>(address(adamw));
  g_sgdm = reinterpret_cast<SgdmFn>(address(sgdm));
  Py_RETURN_NONE;
}

bool tensors(std::initializer_list<PyObject*> objects) {
  for (PyObject* object : objects) {
    if (!THPVariable_Check(object)) return false;
  }
  return true;
}

// Calls `launch` with `device` current and the GIL released, as torch's
// own operators and a ctypes call do (a launch can wait for room in the
// device queue); a device the guard cannot select becomes a RuntimeError.
// The tensors stay alive through the caller's argument tuple.
template <class Launch>
PyObject* on_device(const c10::Device& device, Launch launch) {
  int status = 0;
  bool failed = false;
  std::string message;
  Py_BEGIN_ALLOW_THREADS
  try {
    const c10::DeviceGuard guard(device);
    status = launch();
  } catch (const std::exception& error) {
    failed = true;
    message = error.what();
  } catch (...) {
    failed = true;
    message = "unknown C++ exception in a native launch";
  }
  Py_END_ALLOW_THREADS
  if (failed) return fail(PyExc_RuntimeError, message.c_str());
  return PyLong_FromLong(status);
}

PyObject* cast(PyObject*, PyObject* args) {
  PyObject *x_obj, *out_obj;
  int code, rule, threads;
  unsigned long long seed, offset, stream;
  if (!PyArg_ParseTuple(args, "OOiiKKiK", &x_obj, &out_obj, &code, &rule, &seed, &offset, &threads, &stream)) {
    return nullptr;
  }
  if (!tensors({x_obj, out_obj})) return fail(PyExc_TypeError, "x and out must be tensors");
  const at::Tensor& x = THPVariable_Unpack(x_obj);
  const at::Tensor& out = THPVariable_Unpack(out_obj);
  // The output first: workgroups read x and write out concurrently, so any
  // shared byte would make the result depend on their timing.
  if (!dtype_matches(code, out.scalar_type()) || out.sizes() != x.sizes() || out.device() != x.device() ||
      !out.is_contiguous()) {
    return fail(PyExc_ValueError, "out must be a contiguous tensor of the requested dtype, shape and device");
  }
  const int64_t n = x.numel();
  if (n) {
    const auto x_start = reinterpret_cast<uintptr_t>(x.const_data_ptr());
    const auto out_start = reinterpret_cast<uintptr_t>(out.const_data_ptr());
    if (!x_start || !out_start) return fail(PyExc_ValueError, "tensors without device memory cannot be cast");
    if (x_start < out_start + out.nbytes() && out_start < x_start + x.nbytes()) {
      return fail(PyExc_ValueError, "out must not overlap the input");
    }
  }
  if (!x.is_cuda() || x.scalar_type() != c10::ScalarType::Float || !x.is_contiguous()) {
    return fail(PyExc_ValueError, "the cast input must be a contiguous FP32 tensor on the GPU");
  }
  if (n == 0) return PyLong_FromLong(0);
  if (g_cast == nullptr) return fail(PyExc_RuntimeError, "the native entries are not bound to the library");
  return on_device(x.device(), [&] {
    return g_cast(x.const_data_ptr(), out.data_ptr(), n, code, rule, static_cast<uint32_t>(seed),
                  static_cast<uint32_t>(offset), threads, address(stream));
  });
}

// The tensor checks of the fused updates, in the validating order of
// sr_states/triton/_optimizer.py:24-60; ts[0] is the parameter, ts[1] the
// gradient (only read).  Returns false with the Python error set.
bool check_update_tensors(std::initializer_list<const at::Tensor*> ts) {
  const at::Tensor& p = **ts.begin();
  const at::Tensor& g = **(ts.begin() + 1);
  if (!p.is_cuda()) {
    fail(PyExc_ValueError, "fused state updates require GPU tensors");
    return false;
  }
  for (const at::Tensor* t : ts) {
    if (t->device() != p.device()) {
      fail(PyExc_ValueError, "all tensors must be on the same GPU device");
      return false;
    }
    if (t->sizes() != p.sizes()) {
      fail(PyExc_ValueError, "all tensors must have identical shapes");
      return false;
    }
    if (!t->is_contiguous()) {
      fail(PyExc_ValueError, "fused state updates require contiguous tensors");
      return false;
    }
  }
  const auto float_or_bf16 = [](const at::Tensor& t) {
    return t.scalar_type() == c10::ScalarType::Float || t.scalar_type() == c10::ScalarType::BFloat16;
  };
  if (!float_or_bf16(p) || !float_or_bf16(g)) {
    fail(PyExc_TypeError, "parameter and gradient must be FP32 or BF16");
    return false;
  }
  if (p.numel() == 0) return true;
  for (const at::Tensor* t : ts) {
    if (t->const_data_ptr() == nullptr) {
      fail(PyExc_ValueError, "fused state updates require tensors that hold device memory");
      return false;
    }
  }
  // Every written span (all but the gradient) disjoint from every other
  // span: with one read-only tensor, every pair holds a written one.
  int i = 0;
  for (const at::Tensor* a : ts) {
    int j = 0;
    for (const at::Tensor* b : ts) {
      if (j > i) {
        const auto a0 = reinterpret_cast<uintptr_t>(a->const_data_ptr());
        const auto b0 = reinterpret_cast<uintptr_t>(b->const_data_ptr());
        if (a0 < b0 + b->nbytes() && b0 < a0 + a->nbytes()) {
          fail(PyExc_ValueError, "parameter, gradient, and state must not overlap optimizer writes");
          return false;
        }
      }
      ++j;
    }
    ++i;
  }
  return true;
}

int pg_code(const at::Tensor& t) { return t.scalar_type() == c10::ScalarType::Float ? SR_F32 : SR_BF16; }

bool state_matches(int code, const at::Tensor& t) {
  if (dtype_matches(code, t.scalar_type())) return true;
  fail(PyExc_ValueError, "state dtype does not match its state format");
  return false;
}

PyObject* adamw_step(PyObject*, PyObject* args) {
  PyObject *p_obj, *g_obj, *m_obj, *v_obj;
  int m_code, m_rule, v_code, v_rule, block;
  double s[8];
  unsigned long long key, offset, stream;
  if (!PyArg_ParseTuple(args, "OOOOiiii(dddddddd)KKiK", &p_obj, &g_obj, &m_obj, &v_obj, &m_code, &m_rule, &v_code,
                        &v_rule, &s[0], &s[1], &s[2], &s[3], &s[4], &s[5], &s[6], &s[7], &key, &offset, &block,
                        &stream)) {
    return nullptr;
  }
  if (!tensors({p_obj, g_obj, m_obj, v_obj})) return fail(PyExc_TypeError, "parameter, gradient and states must be tensors");
  const at::Tensor& p = THPVariable_Unpack(p_obj);
  const at::Tensor& g = THPVariable_Unpack(g_obj);
  const at::Tensor& m = THPVariable_Unpack(m_obj);
  const at::Tensor& v = THPVariable_Unpack(v_obj);
  if (!state_matches(m_code, m) || !state_matches(v_code, v) || !check_update_tensors({&p, &g, &m, &v})) {
    return nullptr;
  }
  if (p.numel() == 0) return PyLong_FromLong(0);
  if (g_adamw == nullptr) return fail(PyExc_RuntimeError, "the native entries are not bound to the library");
  const sr_adamw_hparams hp = {static_cast<float>(s[0]), static_cast<float>(s[1]), static_cast<float>(s[2]),
                               static_cast<float>(s[3]), static_cast<float>(s[4]), static_cast<float>(s[5]),
                               static_cast<float>(s[6]), static_cast<float>(s[7])};
  return on_device(p.device(), [&] {
    return g_adamw(p.data_ptr(), g.const_data_ptr(), m.data_ptr(), v.data_ptr(), p.numel(), pg_code(p), pg_code(g),
                   m_code, m_rule, v_code, v_rule, &hp, static_cast<uint32_t>(key), static_cast<uint32_t>(offset),
                   block, address(stream));
  });
}

PyObject* sgdm_step(PyObject*, PyObject* args) {
  PyObject *p_obj, *g_obj, *u_obj;
  int u_code, u_rule, block;
  double s[2];
  unsigned long long key, offset, stream;
  if (!PyArg_ParseTuple(args, "OOOii(dd)KKiK", &p_obj, &g_obj, &u_obj, &u_code, &u_rule, &s[0], &s[1], &key, &offset,
                        &block, &stream)) {
    return nullptr;
  }
  if (!tensors({p_obj, g_obj, u_obj})) return fail(PyExc_TypeError, "parameter, gradient and states must be tensors");
  const at::Tensor& p = THPVariable_Unpack(p_obj);
  const at::Tensor& g = THPVariable_Unpack(g_obj);
  const at::Tensor& u = THPVariable_Unpack(u_obj);
  if (!state_matches(u_code, u) || !check_update_tensors({&p, &g, &u})) return nullptr;
  if (p.numel() == 0) return PyLong_FromLong(0);
  if (g_sgdm == nullptr) return fail(PyExc_RuntimeError, "the native entries are not bound to the library");
  const sr_sgdm_hparams hp = {static_cast<float>(s[0]), static_cast<float>(s[1])};
  return on_device(p.device(), [&] {
    return g_sgdm(p.data_ptr(), g.const_data_ptr(), u.data_ptr(), p.numel(), pg_code(p), pg_code(g), u_code, u_rule,
                  &hp, static_cast<uint32_t>(key), static_cast<uint32_t>(offset), block, address(stream));
  });
}

// Every entry behind one guard: a C++ exception from torch (a tensor
// without storage refuses its data pointer) becomes a RuntimeError instead
// of escaping into the interpreter.
template <PyObject* (*Entry)(PyObject*, PyObject*)>
PyObject* guarded(PyObject* self, PyObject* args) {
  try {
    return Entry(self, args);
  } catch (const std::exception& error) {
    return fail(PyExc_RuntimeError, error.what());
  } catch (...) {
    return fail(PyExc_RuntimeError, "unknown C++ exception in a native entry");
  }
}

PyMethodDef methods[] = {
    {"bind", bind, METH_VARARGS, "Keep the addresses of the C ABI's single-tensor entry points."},
    {"cast", guarded<cast>, METH_VARARGS, "Check the tensors and call sr_cast; returns its status."},
    {"adamw_step", guarded<adamw_step>, METH_VARARGS,
     "Check the tensors and call sr_adamw_step; returns its status."},
    {"sgdm_step", guarded<sgdm_step>, METH_VARARGS, "Check the tensors and call sr_sgdm_step; returns its status."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef module = {PyModuleDef_HEAD_INIT, "_launch", "Native entries of the single-tensor launches.", -1, methods};

}  // namespace

PyMODINIT_FUNC PyInit__launch(void) { return PyModule_Create(&module); }
