// _region_guard: frozen-state guard for captured inference regions.
//
// A Guard snapshots, for every nn.Module of a region, what a captured graph
// silently depends on, and validate() re-checks it before each capture or
// replay.  The snapshot covers:
//   - the module's class and its __dict__ object;
//   - training == False and empty hook dicts;
//   - the child modules (by identity) and the forward binding (unless the
//     module is in `ignored`, whose forward the caller swaps itself);
//   - selected operator attributes (by identity or ==);
//   - every parameter and buffer: identity, version counter, data pointer,
//     sizes, strides, offset, dtype, device and requires_grad == False;
//   - each class's forward, and torch's global module hooks (none allowed).
// Any drift raises ValueError.  require_frozen_fp16() is the admission rule
// RegionContract applies before building a Guard.  Python API and messages follow the
// reference's region guard (region_guard.cpp:36-188, used through
// region_contract.py:5-28); the implementation is independent.
#include <pybind11/pybind11.h>
#include <torch/csrc/autograd/python_variable.h>

#include <string>
#include <utility>
#include <vector>

namespace py = pybind11;

namespace {

// Borrowed lookup in a dict; nullptr when absent (Python errors propagate).
PyObject* lookup(PyObject* dict, PyObject* key) {
  PyObject* v = PyDict_GetItemWithError(dict, key);
  if (!v && PyErr_Occurred()) throw py::error_already_set();
  return v;
}

PyObject* as_dict(PyObject* v) {
  if (!v || !PyDict_Check(v)) throw py::value_error("Expected a module state dictionary");
  return v;
}

Py_ssize_t size_of(PyObject* v) {
  const Py_ssize_t n = PyObject_Length(v);
  if (n < 0) throw py::error_already_set();
  return n;
}

py::str interned(const char* s) {
  PyObject* v = PyUnicode_InternFromString(s);
  if (!v) throw py::error_already_set();
  return py::reinterpret_steal<py::str>(v);
}

// Everything about a parameter/buffer tensor that a captured graph bakes in.
struct TensorState {
  bool defined = false;
  uint32_t version = 0;
  const void* data = nullptr;
  std::vector<int64_t> sizes, strides;
  int64_t offset = 0;
  c10::ScalarType dtype = c10::ScalarType::Undefined;
  c10::Device device{c10::DeviceType::CPU};

  static TensorState of(const at::Tensor& t) {
    TensorState s;
    if (!t.defined()) return s;
    s.defined = true;
    s.version = t.unsafeGetTensorImpl()->version_counter().current_version();
    s.data = t.const_data_ptr();
    s.sizes = t.sizes().vec();
    s.strides = t.strides().vec();
    s.offset = t.storage_offset();
    s.dtype = t.scalar_type();
    s.device = t.device();
    return s;
  }
  bool still(const at::Tensor& t) const {
    return !t.requires_grad() && t.unsafeGetTensorImpl()->version_counter().current_version() == version &&
           t.const_data_ptr() == data && t.scalar_type() == dtype && t.device() == device &&
           t.storage_offset() == offset && t.sizes() == at::IntArrayRef(sizes) &&
           t.strides() == at::IntArrayRef(strides);
  }
};

struct Slot {          // one entry of _parameters or _buffers
  py::str name;
  py::object value;    // the Tensor object (or None)
  TensorState state;
};

struct Collection {    // _parameters or _buffers
  py::str key;
  Py_ssize_t count = 0;
  std::vector<Slot> slots;
};

struct ModuleState {
  py::object module, cls, dict;
  bool guard_forward = true;
  bool instance_forward = false;      // forward stored in the instance dict
  py::object forward_func, forward_self;
  std::vector<std::pair<py::str, py::object>> children, attributes;
  std::vector<Collection> collections;
};

class Guard {
 public:
  Guard(py::iterable modules, py::set ignored, py::iterable attributes)
      : registry_(py::module_::import("torch.nn.modules.module")) {
    std::vector<py::str> attrs;
    for (auto a : attributes) attrs.push_back(py::reinterpret_borrow<py::str>(a));
    for (auto item : modules) snapshot(py::reinterpret_borrow<py::object>(item), ignored, attrs);
    validate();
  }

  void validate() const {
    for (const auto& name : global_hooks_) {
      py::object hooks = py::reinterpret_steal<py::object>(PyObject_GetAttr(registry_.ptr(), name.ptr()));
      if (!hooks) throw py::error_already_set();
      if (size_of(hooks.ptr())) throw py::value_error("Global module hooks are unsupported");
    }
    for (const auto& [cls, forward] : class_forwards_) {
      py::object now = py::reinterpret_steal<py::object>(PyObject_GetAttr(cls.ptr(), forward_.ptr()));
      if (!now) throw py::error_already_set();
      if (now.ptr() != forward.ptr()) throw py::value_error("Module class forward changed");
    }
    for (const auto& m : modules_) check(m);
  }

 private:
  void snapshot(py::object module, const py::set& ignored, const std::vector<py::str>& attrs) {
    ModuleState m;
    m.module = module;
    m.cls = py::type::of(module);
    m.dict = module.attr("__dict__");
    PyObject* d = as_dict(m.dict.ptr());
    m.guard_forward = !ignored.contains(module);
    m.instance_forward = lookup(d, forward_.ptr()) != nullptr;
    py::object bound = module.attr("forward");
    if (!PyMethod_Check(bound.ptr())) throw py::value_error("Expected a bound module forward");
    m.forward_func = py::reinterpret_borrow<py::object>(PyMethod_Function(bound.ptr()));
    m.forward_self = py::reinterpret_borrow<py::object>(PyMethod_Self(bound.ptr()));
    PyObject* children = as_dict(required(d, modules_key_));
    for (auto kv : py::reinterpret_borrow<py::dict>(children))
      m.children.emplace_back(py::reinterpret_borrow<py::str>(kv.first), py::reinterpret_borrow<py::object>(kv.second));
    for (const auto& a : attrs)
      if (PyObject* v = lookup(d, a.ptr())) m.attributes.emplace_back(a, py::reinterpret_borrow<py::object>(v));
    for (const auto& key : {params_key_, buffers_key_}) {
      Collection c;
      c.key = key;
      PyObject* values = as_dict(required(d, key));
      c.count = size_of(values);
      for (auto kv : py::reinterpret_borrow<py::dict>(values)) {
        py::object value = py::reinterpret_borrow<py::object>(kv.second);
        if (!value.is_none() && !THPVariable_Check(value.ptr()))
          throw py::type_error("Expected a Tensor or None in module parameters/buffers");
        Slot s{py::reinterpret_borrow<py::str>(kv.first), value,
               value.is_none() ? TensorState{} : TensorState::of(THPVariable_Unpack(value.ptr()))};
        c.slots.push_back(std::move(s));
      }
      m.collections.push_back(std::move(c));
    }
    bool seen = false;
    for (const auto& cf : class_forwards_) seen = seen || cf.first.ptr() == m.cls.ptr();
    if (!seen) class_forwards_.emplace_back(m.cls, m.cls.attr("forward"));
    modules_.push_back(std::move(m));
  }

  static PyObject* required(PyObject* dict, const py::str& key) {
    PyObject* v = lookup(dict, key.ptr());
    if (!v) throw py::value_error("Region attribute removed");
    return v;
  }

  void check(const ModuleState& m) const {
    if (reinterpret_cast<PyObject*>(Py_TYPE(m.module.ptr())) != m.cls.ptr())
      throw py::value_error("Region module class changed");
    {
      py::object now = py::reinterpret_steal<py::object>(PyObject_GenericGetDict(m.module.ptr(), nullptr));
      if (!now) throw py::error_already_set();
      if (now.ptr() != m.dict.ptr()) throw py::value_error("Region module dictionary changed");
    }
    PyObject* d = m.dict.ptr();
    if (required(d, training_) != Py_False) throw py::value_error("Region is inference-only");
    for (const auto& h : hook_keys_)
      if (size_of(required(d, h))) throw py::value_error("Region hooks changed");
    PyObject* children = as_dict(required(d, modules_key_));
    if (PyDict_Size(children) != (Py_ssize_t)m.children.size()) throw py::value_error("Region children changed");
    for (const auto& [name, child] : m.children)
      if (lookup(children, name.ptr()) != child.ptr()) throw py::value_error("Region child identity changed");
    if (m.guard_forward) {
      PyObject* f = lookup(d, forward_.ptr());
      if (f) {
        if (!PyMethod_Check(f) || PyMethod_Function(f) != m.forward_func.ptr() ||
            PyMethod_Self(f) != m.forward_self.ptr())
          throw py::value_error("Region forward changed");
      } else if (m.instance_forward) {
        throw py::value_error("Region forward changed");
      }
    }
    for (const auto& [name, value] : m.attributes) {
      PyObject* v = lookup(d, name.ptr());
      if (!v) throw py::value_error("Region operator configuration changed");
      if (v != value.ptr()) {
        const int eq = PyObject_RichCompareBool(v, value.ptr(), Py_EQ);
        if (eq < 0) throw py::error_already_set();
        if (eq != 1) throw py::value_error("Region operator configuration changed");
      }
    }
    for (const auto& c : m.collections) {
      PyObject* values = as_dict(required(d, c.key));
      if (size_of(values) != c.count) throw py::value_error("Region parameter/buffer set changed");
      for (const auto& s : c.slots) {
        if (lookup(values, s.name.ptr()) != s.value.ptr())
          throw py::value_error("Region parameter/prepack identity changed");
        if (!s.value.is_none() && !s.state.still(THPVariable_Unpack(s.value.ptr())))
          throw py::value_error("Region parameter/prepack version or gradient mode changed");
      }
    }
  }

  py::object registry_;
  std::vector<ModuleState> modules_;
  std::vector<std::pair<py::object, py::object>> class_forwards_;
  py::str training_ = interned("training"), modules_key_ = interned("_modules"), forward_ = interned("forward");
  py::str params_key_ = interned("_parameters"), buffers_key_ = interned("_buffers");
  std::vector<py::str> hook_keys_{interned("_forward_hooks"), interned("_forward_pre_hooks"),
                                  interned("_backward_hooks"), interned("_backward_pre_hooks")};
  std::vector<py::str> global_hooks_{interned("_global_forward_hooks"), interned("_global_forward_pre_hooks"),
                                     interned("_global_backward_hooks"), interned("_global_backward_pre_hooks")};
};

// Admission rule of a frozen fp16 region (RegionContract's constructor): every
// parameter and buffer of every module is a version-counted fp16 tensor on the
// npu device without gradient.  Tensors are visited module by module,
// parameters before buffers, and the first offender raises ValueError.  An
// inference-mode tensor has no version counter for the guard to snapshot.
void require_frozen_fp16(py::iterable modules) {
  const py::str keys[2] = {interned("_parameters"), interned("_buffers")};
  for (auto item : modules) {
    py::object state = py::reinterpret_borrow<py::object>(item).attr("__dict__");
    PyObject* d = as_dict(state.ptr());
    for (const auto& key : keys) {
      PyObject* values = lookup(d, key.ptr());
      if (!values) continue;
      for (auto kv : py::reinterpret_borrow<py::dict>(as_dict(values))) {
        if (kv.second.is_none()) continue;
        if (!THPVariable_Check(kv.second.ptr()))
          throw py::type_error("Expected a Tensor or None in module parameters/buffers");
        const at::Tensor& t = THPVariable_Unpack(kv.second.ptr());
        if (t.is_inference())
          throw py::value_error("Prepare versioned parameters under no_grad(), not inference_mode()");
        if (t.requires_grad() || t.scalar_type() != at::kHalf || t.device().type() != c10::DeviceType::PrivateUse1)
          throw py::value_error("Expected fixed FP16 NPU inference parameters");
      }
    }
  }
}

}  // namespace

PYBIND11_MODULE(_region_guard, m) {
  py::class_<Guard>(m, "Guard")
      .def(py::init<py::iterable, py::set, py::iterable>())
      .def("validate", &Guard::validate);
  m.def("require_frozen_fp16", &require_frozen_fp16);
}
