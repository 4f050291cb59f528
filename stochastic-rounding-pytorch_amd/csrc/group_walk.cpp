// Native walk over one optimizer parameter group, for the fused multi-tensor
// step's host side.
//
// The reference validates and buckets every tensor of a group on every step
// (sr_states/triton/_multi_tensor.py:22-34 and :61-88).  The row tables only
// change when a layout, an address or the set of parameters with gradients
// changes, so this module condenses exactly those facts into one byte string
// per step.  The Python side runs the full validation and rebuilds the tables
// whenever the string differs from the one recorded at the last fully
// validated step; when it is equal, nothing the validation or the tables
// depend on has changed and the recorded launches are reused.
//
// group_signature(params, state, state_names, uses_step, first_index)
//     -> (bytes, step, steps, entries) or None
//   Each tensor contributes its Python type, so a validated step vouches only
//   for the types it saw.  None means "take the validating path": an object
//   that is not a tensor, a missing state, a non-strided tensor, one with
//   elements but no memory (wrapper subclasses), a stored step that is not a
//   non-negative int, or no parameter with a gradient.  Stored steps are not
//   part of the bytes.  When uses_step is true and every parameter with a
//   gradient stores the same step (0 when absent), ``step`` is that value and
//   ``steps`` is None; when they differ, ``step`` is None and ``steps`` lists
//   them in group order.  Both are None when uses_step is false.  ``entries``
//   lists the state dict of every parameter with a gradient, in group order.
//
// set_steps(entries, value)
//   entry["step"] = value for every dict in the list ``entries``.

#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <torch/csrc/autograd/python_variable.h>

#include <cstdint>
#include <vector>

namespace {

PyObject* g_grad = nullptr;  // interned "grad"
PyObject* g_step = nullptr;  // interned "step"

// Appends the words that fix one tensor's view: Python type, address, element
// count, dtype, device, contiguity, rank and sizes.  False when the object is
// not a tensor or has no strided memory to describe.
bool describe(PyObject* obj, std::vector<int64_t>& words) {
  if (!THPVariable_Check(obj)) return false;
  try {
    const at::Tensor& t = THPVariable_Unpack(obj);
    if (!t.defined() || t.layout() != at::kStrided || !t.has_storage()) return false;
    const auto sizes = t.sizes();
    const at::Device device = t.device();
    const auto address = reinterpret_cast<intptr_t>(t.data_ptr());
    if (address == 0 && t.numel() != 0) return false;
    words.push_back(static_cast<int64_t>(reinterpret_cast<intptr_t>(Py_TYPE(obj))));
    words.push_back(static_cast<int64_t>(address));
    words.push_back(t.numel());
    words.push_back(static_cast<int64_t>(t.scalar_type()) |
                    static_cast<int64_t>(device.type()) << 8 |
                    static_cast<int64_t>(static_cast<uint8_t>(device.index())) << 16 |
                    static_cast<int64_t>(t.is_contiguous()) << 24 |
                    static_cast<int64_t>(sizes.size()) << 32);
    for (int64_t s : sizes) words.push_back(s);
    return true;
  } catch (...) {
    return false;
  }
}

// Borrowed state dict of a parameter, or nullptr (without an exception set)
// when it is absent or not an exact dict.
PyObject* parameter_state(PyObject* state, PyObject* parameter) {
  PyObject* entry = PyDict_GetItemWithError(state, parameter);
  if (entry == nullptr || !PyDict_CheckExact(entry)) {
    PyErr_Clear();
    return nullptr;
  }
  return entry;
}

// Owned reference released at scope exit.
struct Ref {
  PyObject* obj;
  explicit Ref(PyObject* o) : obj(o) {}
  Ref(const Ref&) = delete;
  Ref& operator=(const Ref&) = delete;
  ~Ref() { Py_XDECREF(obj); }
};

// One parameter with a gradient: its words and its stored step.
bool walk_parameter(PyObject* parameter, PyObject* gradient, PyObject* state, PyObject* names,
                    bool uses_step, std::vector<int64_t>& words, int64_t& step, PyObject* entries) {
  PyObject* entry = parameter_state(state, parameter);
  if (entry == nullptr) return false;
  Ref hold_entry(entry);
  Py_INCREF(entry);
  if (PyList_Append(entries, entry) != 0) return false;
  words.push_back(2 + PyTuple_GET_SIZE(names));
  if (!describe(parameter, words) || !describe(gradient, words)) return false;
  for (Py_ssize_t k = 0; k < PyTuple_GET_SIZE(names); ++k) {
    PyObject* tensor = PyDict_GetItemWithError(entry, PyTuple_GET_ITEM(names, k));
    if (tensor == nullptr || !describe(tensor, words)) return false;
  }
  step = 0;
  if (!uses_step) return true;
  PyObject* value = PyDict_GetItemWithError(entry, g_step);
  if (value == nullptr) return !PyErr_Occurred();
  if (!PyLong_CheckExact(value)) return false;
  int overflow = 0;
  step = PyLong_AsLongLongAndOverflow(value, &overflow);
  return !overflow && !PyErr_Occurred() && step >= 0;
}

// The walk proper; returns false for "take the validating path".
bool walk(PyObject* params, PyObject* state, PyObject* names, bool uses_step,
          std::vector<int64_t>& words, std::vector<int64_t>& steps, PyObject* entries) {
  for (Py_ssize_t i = 0; i < PyList_GET_SIZE(params); ++i) {
    PyObject* parameter = PyList_GET_ITEM(params, i);
    Ref hold_parameter(parameter);
    Py_INCREF(parameter);
    if (!THPVariable_Check(parameter)) return false;
    Ref gradient(PyObject_GetAttr(parameter, g_grad));
    if (gradient.obj == nullptr) return false;
    if (gradient.obj == Py_None) {
      words.push_back(-1);
      continue;
    }
    int64_t step = 0;
    if (!walk_parameter(parameter, gradient.obj, state, names, uses_step, words, step, entries)) {
      return false;
    }
    steps.push_back(step);
  }
  return !steps.empty();
}

PyObject* group_signature(PyObject*, PyObject* args) {
  PyObject *params, *state, *names;
  int uses_step;
  long long first_index;
  if (!PyArg_ParseTuple(args, "O!O!O!pL", &PyList_Type, &params, &PyDict_Type, &state,
                        &PyTuple_Type, &names, &uses_step, &first_index)) {
    return nullptr;
  }
  std::vector<int64_t> words;
  words.reserve(4 + PyList_GET_SIZE(params) * (1 + 7 * (2 + PyTuple_GET_SIZE(names))));
  words.push_back(first_index);
  words.push_back(PyList_GET_SIZE(params));
  std::vector<int64_t> steps;
  bool found = false;
  Ref entries(PyList_New(0));
  if (entries.obj == nullptr) return nullptr;
  Py_INCREF(params);  // the walk may run Python code (Tensor.__hash__)
  try {
    found = walk(params, state, names, uses_step != 0, words, steps, entries.obj);
  } catch (...) {
    found = false;
  }
  Py_DECREF(params);
  if (!found) {
    PyErr_Clear();
    Py_RETURN_NONE;
  }
  bool uniform = true;
  for (int64_t s : steps) uniform = uniform && s == steps[0];
  Ref common(nullptr), listed(nullptr);
  if (!uses_step) {
    common.obj = Py_NewRef(Py_None);
    listed.obj = Py_NewRef(Py_None);
  } else if (uniform) {
    common.obj = PyLong_FromLongLong(steps[0]);
    listed.obj = Py_NewRef(Py_None);
  } else {
    common.obj = Py_NewRef(Py_None);
    listed.obj = PyList_New(static_cast<Py_ssize_t>(steps.size()));
    for (size_t k = 0; listed.obj != nullptr && k < steps.size(); ++k) {
      PyObject* value = PyLong_FromLongLong(steps[k]);
      if (value == nullptr) return nullptr;
      PyList_SET_ITEM(listed.obj, static_cast<Py_ssize_t>(k), value);
    }
  }
  if (common.obj == nullptr || listed.obj == nullptr) return nullptr;
  return Py_BuildValue("(y#OOO)", reinterpret_cast<const char*>(words.data()),
                       static_cast<Py_ssize_t>(words.size() * sizeof(int64_t)), common.obj,
                       listed.obj, entries.obj);
}

PyObject* set_steps(PyObject*, PyObject* args) {
  PyObject* entries;
  long long value;
  if (!PyArg_ParseTuple(args, "O!L", &PyList_Type, &entries, &value)) return nullptr;
  Ref step(PyLong_FromLongLong(value));
  if (step.obj == nullptr) return nullptr;
  for (Py_ssize_t i = 0; i < PyList_GET_SIZE(entries); ++i) {
    if (PyObject_SetItem(PyList_GET_ITEM(entries, i), g_step, step.obj) != 0) return nullptr;
  }
  Py_RETURN_NONE;
}

PyMethodDef kMethods[] = {
    {"group_signature", group_signature, METH_VARARGS,
     "group_signature(params, state, state_names, uses_step, first_index)"},
    {"set_steps", set_steps, METH_VARARGS, "set_steps(entries, value)"},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_group_walk",
                       "Per-step signature of an optimizer group's tensors.", -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__group_walk() {
  g_grad = PyUnicode_InternFromString("grad");
  g_step = PyUnicode_InternFromString("step");
  if (g_grad == nullptr || g_step == nullptr) return nullptr;
  return PyModule_Create(&kModule);
}
