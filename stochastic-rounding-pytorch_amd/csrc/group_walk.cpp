// Native walk over one optimizer parameter group, for the fused multi-tensor
// step's host side.
//
// The reference validates and buckets every tensor of a group on every step
// (sr_states/triton/_multi_tensor.py:22-34 and :61-88).  The row tables only
// change when a layout, an address or the set of parameters with gradients
// changes, so this module condenses exactly those facts for the Python side,
// which runs the full validation whenever they differ from those of an
// earlier fully validated step.  Gradients are reported apart from the rest:
// training loops free them every step and get them back at varying
// addresses, and a new gradient address only needs its table column patched
// and the overlap rule checked again (spans_disjoint).
//
// group_signature(params, state, state_names, uses_step, first_index)
//     -> (layout, step, steps, entries, gradients, spans) or None
//   ``layout`` (bytes) fixes every tensor's Python type, element count, dtype,
//   device, contiguity and sizes, every parameter's and state's address, and
//   which parameters have gradients; gradient addresses are left out.  A
//   DTensor is described by its spec's identity and its local shard.  A
//   validated step vouches only for the types it saw.  None means "take the
//   validating path": an object that is not a tensor, a missing state, a
//   non-strided tensor, one with elements but no memory (wrapper subclasses
//   other than DTensor), a stored step that is not a non-negative int, or
//   no parameter with a gradient.  When uses_step is true and every parameter
//   with a gradient stores the same step (0 when absent), ``step`` is that
//   value and ``steps`` is None; when they differ, ``step`` is None and
//   ``steps`` lists them in group order.  Both are None when uses_step is
//   false.  ``entries`` lists the state dict of every parameter with a
//   gradient, in group order; ``gradients`` (bytes) their gradients'
//   addresses as int64; ``spans`` (bytes) one (device, start, end, written)
//   int64 quadruple per tensor with elements.
//
// spans_disjoint(spans) -> bool
//   The overlap rule of the validating path (triton/_optimizer.py:38-49):
//   per device, every written span is disjoint from every other span;
//   gradients are only read and may share memory with each other.
//
// set_steps(entries, value)
//   entry["step"] = value for every dict in the list ``entries``.

#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <structmember.h>
#include <torch/csrc/autograd/python_variable.h>

#include <algorithm>
#include <array>
#include <climits>
#include <cstdint>
#include <vector>

namespace {

PyObject* g_grad = nullptr;   // interned "grad"
PyObject* g_step = nullptr;   // interned "step"
PyObject* g_local = nullptr;  // interned "_local_tensor"
PyObject* g_spec = nullptr;   // interned "_spec"
PyObject* g_hash = nullptr;   // interned "__hash__"
PyObject* g_mesh = nullptr;         // interned DTensorSpec field names
PyObject* g_placements = nullptr;
PyObject* g_shard_order = nullptr;
PyObject* g_tensor_meta = nullptr;
PyObject* g_tensor_hash = nullptr;  // torch.Tensor.__hash__ (returns id(self))
PyObject* g_spec_type = nullptr;    // DTensorSpec, once enable_spec_fast_path() vouched for its fields
// The exact DTensor type and the offsets of its `_local_tensor` and `_spec`
// slots, once enable_dtensor_slots() found them as object members.
PyTypeObject* g_dtensor_type = nullptr;
Py_ssize_t g_local_offset = -1, g_spec_offset = -1;

// Everything one walk collects.
struct Walk {
  std::vector<int64_t> words;      // the layout signature
  std::vector<int64_t> gradients;  // gradient address per parameter with a gradient
  std::vector<int64_t> spans;      // (device, start, end, written) per tensor with elements
  std::vector<int64_t> steps;      // stored step per parameter with a gradient
};

// Owned reference released at scope exit.
struct Ref {
  PyObject* obj;
  explicit Ref(PyObject* o) : obj(o) {}
  Ref(const Ref&) = delete;
  Ref& operator=(const Ref&) = delete;
  ~Ref() { Py_XDECREF(obj); }
};

bool describe(PyObject* obj, Walk& w, bool gradient, PyObject* parameter_spec = nullptr);

// A DTensor: a tensor subclass whose data is the `_local_tensor` it carries,
// laid out by its `_spec` (mesh, placements, global shape).
bool is_distributed(PyObject* obj) {
  if (Py_TYPE(obj) == g_dtensor_type) return true;
  return !THPVariable_CheckExact(obj) && PyObject_HasAttr(obj, g_local);
}

// New reference to a DTensor's `_local_tensor` or `_spec`, or nullptr (no
// error set).  The exact DTensor type's slots are read at their offsets.
PyObject* dtensor_part(PyObject* obj, PyObject* name, Py_ssize_t offset) {
  if (Py_TYPE(obj) == g_dtensor_type && offset >= 0) {
    PyObject* value = *reinterpret_cast<PyObject**>(reinterpret_cast<char*>(obj) + offset);
    Py_XINCREF(value);
    return value;
  }
  PyObject* value = PyObject_GetAttr(obj, name);
  if (value == nullptr) PyErr_Clear();
  return value;
}

// One attribute of a spec as a new reference, or nullptr (error cleared).
PyObject* field(PyObject* spec, PyObject* name) {
  PyObject* value = PyObject_GetAttr(spec, name);
  if (value == nullptr) PyErr_Clear();
  return value;
}

// Equal by PyObject_RichCompareBool, with no error left set.
bool same(PyObject* a, PyObject* b) {
  const int r = PyObject_RichCompareBool(a, b, Py_EQ);
  if (r < 0) PyErr_Clear();
  return r == 1;
}

// True only when DTensorSpec._check_equals(a, b) is certainly true, decided
// with C-level comparisons: the same mesh object; placements and shard order
// equal as tuples (their elements compare in C++); tensor metadata both
// absent, or the same shape, stride and dtype.  False means "undecided".
bool specs_certainly_equal(PyObject* a, PyObject* b) {
  if (g_spec_type == nullptr || Py_TYPE(a) != reinterpret_cast<PyTypeObject*>(g_spec_type) ||
      Py_TYPE(b) != Py_TYPE(a)) {
    return false;
  }
  Ref mesh_a(field(a, g_mesh)), mesh_b(field(b, g_mesh));
  if (mesh_a.obj == nullptr || mesh_a.obj != mesh_b.obj) return false;
  for (PyObject* name : {g_placements, g_shard_order}) {
    Ref x(field(a, name)), y(field(b, name));
    if (x.obj == nullptr || y.obj == nullptr) return false;
    if (x.obj != y.obj && !(PyTuple_CheckExact(x.obj) && PyTuple_CheckExact(y.obj) && same(x.obj, y.obj))) {
      return false;
    }
  }
  Ref meta_a(field(a, g_tensor_meta)), meta_b(field(b, g_tensor_meta));
  if (meta_a.obj == nullptr || meta_b.obj == nullptr) return false;
  if (meta_a.obj == Py_None || meta_b.obj == Py_None) return meta_a.obj == meta_b.obj;
  if (!PyTuple_Check(meta_a.obj) || !PyTuple_Check(meta_b.obj) || PyTuple_GET_SIZE(meta_a.obj) != 3 ||
      PyTuple_GET_SIZE(meta_b.obj) != 3) {
    return false;
  }
  for (Py_ssize_t k = 0; k < 3; ++k) {  // shape, stride, dtype
    PyObject* x = PyTuple_GET_ITEM(meta_a.obj, k);
    PyObject* y = PyTuple_GET_ITEM(meta_b.obj, k);
    if (x != y && !(PyTuple_Check(x) && PyTuple_Check(y) && same(x, y))) return false;
  }
  return true;
}

// A DTensor parameter's or state's words: its Python type, the identity of
// its spec, and its local shard's words.  The spec object is replaced
// whenever the mesh, placements or global shape change, and the optimizer
// keeps parameters and states (and so their specs) alive between steps, so
// an unchanged identity vouches for the shard start and the placement
// checks of the validated step.  A DTensor gradient is new every step: its
// spec must be the parameter's or equal to it, checked here, and only its
// type and local shard enter the words.
bool describe_distributed(PyObject* obj, Walk& w, bool gradient, PyObject* parameter_spec) {
  Ref local(dtensor_part(obj, g_local, g_local_offset));
  if (local.obj == nullptr || !THPVariable_Check(local.obj)) return false;
  Ref spec(dtensor_part(obj, g_spec, g_spec_offset));
  if (spec.obj == nullptr) return false;
  w.words.push_back(static_cast<int64_t>(reinterpret_cast<intptr_t>(Py_TYPE(obj))));
  if (gradient) {
    if (parameter_spec == nullptr) return false;
    if (spec.obj != parameter_spec && !specs_certainly_equal(spec.obj, parameter_spec) &&
        PyObject_RichCompareBool(spec.obj, parameter_spec, Py_EQ) != 1) {
      return false;
    }
  } else {
    w.words.push_back(static_cast<int64_t>(reinterpret_cast<intptr_t>(spec.obj)));
  }
  return describe(local.obj, w, gradient);
}

// Appends the words that fix one tensor's view: Python type, address (unless
// it is a gradient, whose address goes to w.gradients), element count, dtype,
// device, contiguity, rank and sizes; and the tensor's byte span.  A DTensor
// is described through its local shard.  False when the object is not a
// tensor or has no strided memory to describe.
bool describe(PyObject* obj, Walk& w, bool gradient, PyObject* parameter_spec) {
  if (!THPVariable_Check(obj)) return false;
  try {
    const at::Tensor& t = THPVariable_Unpack(obj);
    // Plain tensors and parameters skip the attribute lookup.
    if (is_distributed(obj)) return describe_distributed(obj, w, gradient, parameter_spec);
    if (!t.defined() || t.layout() != at::kStrided || !t.has_storage()) return false;
    const auto sizes = t.sizes();
    const at::Device device = t.device();
    const auto address = static_cast<int64_t>(reinterpret_cast<intptr_t>(t.data_ptr()));
    const int64_t numel = t.numel();
    if (address == 0 && numel != 0) return false;
    const int64_t device_key =
        static_cast<int64_t>(device.type()) << 8 | static_cast<uint8_t>(device.index());
    w.words.push_back(static_cast<int64_t>(reinterpret_cast<intptr_t>(Py_TYPE(obj))));
    if (gradient) {
      w.gradients.push_back(address);
    } else {
      w.words.push_back(address);
    }
    w.words.push_back(numel);
    w.words.push_back(static_cast<int64_t>(t.scalar_type()) | device_key << 8 |
                      static_cast<int64_t>(t.is_contiguous()) << 24 |
                      static_cast<int64_t>(sizes.size()) << 32);
    for (int64_t s : sizes) w.words.push_back(s);
    if (numel != 0) {
      const int64_t end = address + numel * static_cast<int64_t>(t.element_size());
      w.spans.insert(w.spans.end(), {device_key, address, end, gradient ? 0 : 1});
    }
    return true;
  } catch (...) {
    return false;
  }
}

// True when objects of `type` hash as torch.Tensor does, by id(self).  The
// last type seen is kept (with a reference, so its address cannot be reused).
bool hashes_by_id(PyTypeObject* type) {
  static PyTypeObject* last = nullptr;
  static bool last_result = false;
  if (type == last) return last_result;
  PyObject* method = _PyType_Lookup(type, g_hash);  // borrowed; sets no error
  Py_INCREF(type);
  Py_XDECREF(reinterpret_cast<PyObject*>(last));
  last = type;
  last_result = method != nullptr && method == g_tensor_hash;
  return last_result;
}

// Borrowed state dict of a parameter, or nullptr (without an exception set)
// when it is absent or not an exact dict.  A parameter whose type keeps
// torch.Tensor's id-based hash is looked up with that hash computed here,
// hash(id(parameter)), instead of calling the Python method.
PyObject* parameter_state(PyObject* state, PyObject* parameter) {
  PyObject* entry = nullptr;
  if (g_tensor_hash != nullptr && hashes_by_id(Py_TYPE(parameter))) {
    Ref id(PyLong_FromVoidPtr(parameter));
    const Py_hash_t hash = id.obj == nullptr ? -1 : PyObject_Hash(id.obj);
    entry = hash == -1 ? nullptr : _PyDict_GetItem_KnownHash(state, parameter, hash);
  } else {
    entry = PyDict_GetItemWithError(state, parameter);
  }
  if (entry == nullptr || !PyDict_CheckExact(entry)) {
    PyErr_Clear();
    return nullptr;
  }
  return entry;
}

// One parameter with a gradient: its words, spans and stored step.
bool walk_parameter(PyObject* parameter, PyObject* gradient, PyObject* state, PyObject* names,
                    bool uses_step, Walk& w, int64_t& step, PyObject* entries) {
  PyObject* entry = parameter_state(state, parameter);
  if (entry == nullptr) return false;
  Ref hold_entry(entry);
  Py_INCREF(entry);
  if (PyList_Append(entries, entry) != 0) return false;
  w.words.push_back(2 + PyTuple_GET_SIZE(names));
  Ref parameter_spec(is_distributed(parameter) ? dtensor_part(parameter, g_spec, g_spec_offset) : nullptr);
  if (!describe(parameter, w, false) || !describe(gradient, w, true, parameter_spec.obj)) return false;
  for (Py_ssize_t k = 0; k < PyTuple_GET_SIZE(names); ++k) {
    PyObject* tensor = PyDict_GetItemWithError(entry, PyTuple_GET_ITEM(names, k));
    if (tensor == nullptr || !describe(tensor, w, false)) return false;
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
bool walk(PyObject* params, PyObject* state, PyObject* names, bool uses_step, Walk& w,
          PyObject* entries) {
  for (Py_ssize_t i = 0; i < PyList_GET_SIZE(params); ++i) {
    PyObject* parameter = PyList_GET_ITEM(params, i);
    Ref hold_parameter(parameter);
    Py_INCREF(parameter);
    if (!THPVariable_Check(parameter)) return false;
    Ref gradient(PyObject_GetAttr(parameter, g_grad));
    if (gradient.obj == nullptr) return false;
    if (gradient.obj == Py_None) {
      w.words.push_back(-1);
      continue;
    }
    int64_t step = 0;
    if (!walk_parameter(parameter, gradient.obj, state, names, uses_step, w, step, entries)) {
      return false;
    }
    w.steps.push_back(step);
  }
  return !w.steps.empty();
}

PyObject* as_bytes(const std::vector<int64_t>& v) {
  return PyBytes_FromStringAndSize(reinterpret_cast<const char*>(v.data()),
                                   static_cast<Py_ssize_t>(v.size() * sizeof(int64_t)));
}

PyObject* group_signature(PyObject*, PyObject* args) {
  PyObject *params, *state, *names;
  int uses_step;
  long long first_index;
  if (!PyArg_ParseTuple(args, "O!O!O!pL", &PyList_Type, &params, &PyDict_Type, &state,
                        &PyTuple_Type, &names, &uses_step, &first_index)) {
    return nullptr;
  }
  Walk w;
  const Py_ssize_t tensors = PyList_GET_SIZE(params) * (2 + PyTuple_GET_SIZE(names));
  w.words.reserve(4 + PyList_GET_SIZE(params) + 7 * tensors);
  w.spans.reserve(4 * tensors);
  w.words.push_back(first_index);
  w.words.push_back(PyList_GET_SIZE(params));
  bool found = false;
  Ref entries(PyList_New(0));
  if (entries.obj == nullptr) return nullptr;
  Py_INCREF(params);  // the walk may run Python code (Tensor.__hash__)
  try {
    found = walk(params, state, names, uses_step != 0, w, entries.obj);
  } catch (...) {
    found = false;
  }
  Py_DECREF(params);
  if (!found) {
    PyErr_Clear();
    Py_RETURN_NONE;
  }
  const std::vector<int64_t>& steps = w.steps;
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
  Ref layout(as_bytes(w.words)), gradients(as_bytes(w.gradients)), spans(as_bytes(w.spans));
  if (layout.obj == nullptr || gradients.obj == nullptr || spans.obj == nullptr) return nullptr;
  return PyTuple_Pack(6, layout.obj, common.obj, listed.obj, entries.obj, gradients.obj,
                      spans.obj);
}

PyObject* spans_disjoint(PyObject*, PyObject* args) {
  const char* data;
  Py_ssize_t size;
  if (!PyArg_ParseTuple(args, "y#", &data, &size)) return nullptr;
  if (size % (4 * sizeof(int64_t)) != 0) {
    PyErr_SetString(PyExc_ValueError, "spans must hold (device, start, end, written) quadruples");
    return nullptr;
  }
  std::vector<std::array<int64_t, 4>> spans(static_cast<size_t>(size) / (4 * sizeof(int64_t)));
  std::copy_n(data, size, reinterpret_cast<char*>(spans.data()));
  // Sorted by device, then as the validating path sorts (start, end, written).
  std::sort(spans.begin(), spans.end());
  int64_t device = 0, max_end = 0, max_write_end = 0;
  for (size_t k = 0; k < spans.size(); ++k) {
    const auto& [dev, start, end, written] = spans[k];
    if (k == 0 || dev != device) {
      device = dev;
      max_end = max_write_end = INT64_MIN;
    }
    if (start < (written ? max_end : max_write_end)) Py_RETURN_FALSE;
    max_end = std::max(max_end, end);
    if (written) max_write_end = std::max(max_write_end, end);
  }
  Py_RETURN_TRUE;
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

// enable_spec_fast_path(spec_type): compare DTensor gradient specs of this
// exact type with specs_certainly_equal before falling back to __eq__.  The
// caller vouches that the type's equality is its mesh, placements, shard
// order and tensor metadata (shape, stride, dtype).
PyObject* enable_spec_fast_path(PyObject*, PyObject* args) {
  PyObject* type;
  if (!PyArg_ParseTuple(args, "O!", &PyType_Type, &type)) return nullptr;
  Py_INCREF(type);
  Py_XSETREF(g_spec_type, type);
  Py_RETURN_NONE;
}

// enable_dtensor_slots(dtensor_type): read `_local_tensor` and `_spec` of
// objects of exactly this type at their slot offsets.  Returns whether both
// are object members of the type (otherwise attribute lookups stay).
PyObject* enable_dtensor_slots(PyObject*, PyObject* args) {
  PyObject* type;
  if (!PyArg_ParseTuple(args, "O!", &PyType_Type, &type)) return nullptr;
  Py_ssize_t offsets[2] = {-1, -1};
  PyObject* names[2] = {g_local, g_spec};
  for (int k = 0; k < 2; ++k) {
    PyObject* descr = PyDict_GetItemWithError(reinterpret_cast<PyTypeObject*>(type)->tp_dict, names[k]);
    if (descr == nullptr || Py_TYPE(descr) != &PyMemberDescr_Type) {
      PyErr_Clear();
      Py_RETURN_FALSE;
    }
    const PyMemberDef* member = reinterpret_cast<PyMemberDescrObject*>(descr)->d_member;
    if (member->type != T_OBJECT_EX) Py_RETURN_FALSE;
    offsets[k] = member->offset;
  }
  Py_INCREF(type);
  Py_XDECREF(reinterpret_cast<PyObject*>(g_dtensor_type));
  g_dtensor_type = reinterpret_cast<PyTypeObject*>(type);
  g_local_offset = offsets[0];
  g_spec_offset = offsets[1];
  Py_RETURN_TRUE;
}

PyMethodDef kMethods[] = {
    {"enable_dtensor_slots", enable_dtensor_slots, METH_VARARGS, "enable_dtensor_slots(dtensor_type) -> bool"},
    {"enable_spec_fast_path", enable_spec_fast_path, METH_VARARGS, "enable_spec_fast_path(spec_type)"},
    {"group_signature", group_signature, METH_VARARGS,
     "group_signature(params, state, state_names, uses_step, first_index)"},
    {"spans_disjoint", spans_disjoint, METH_VARARGS, "spans_disjoint(spans) -> bool"},
    {"set_steps", set_steps, METH_VARARGS, "set_steps(entries, value)"},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_group_walk",
                       "Per-step signature of an optimizer group's tensors.", -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__group_walk() {
  g_grad = PyUnicode_InternFromString("grad");
  g_step = PyUnicode_InternFromString("step");
  g_local = PyUnicode_InternFromString("_local_tensor");
  g_spec = PyUnicode_InternFromString("_spec");
  g_hash = PyUnicode_InternFromString("__hash__");
  g_mesh = PyUnicode_InternFromString("mesh");
  g_placements = PyUnicode_InternFromString("placements");
  g_shard_order = PyUnicode_InternFromString("shard_order");
  g_tensor_meta = PyUnicode_InternFromString("tensor_meta");
  for (PyObject* name : {g_grad, g_step, g_local, g_spec, g_hash, g_mesh, g_placements, g_shard_order, g_tensor_meta}) {
    if (name == nullptr) return nullptr;
  }
  // torch.Tensor.__hash__, for the id-hash lookups; without it every
  // lookup calls the type's __hash__.
  PyObject* torch = PyImport_ImportModule("torch");
  PyObject* tensor = torch ? PyObject_GetAttrString(torch, "Tensor") : nullptr;
  g_tensor_hash = tensor ? PyObject_GetAttr(tensor, g_hash) : nullptr;
  Py_XDECREF(tensor);
  Py_XDECREF(torch);
  PyErr_Clear();
  return PyModule_Create(&kModule);
}
