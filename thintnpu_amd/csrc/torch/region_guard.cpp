// _region_guard: frozen-state guard for captured inference regions.
//
// Python surface (the drop-in for the reference's region guard,
// region_guard.cpp:36-188, used through region_contract.py:5-28):
//   Guard(modules, ignored, attributes) and Guard.validate(), which raises
//   ValueError with the message of the first drift it finds;
//   require_frozen_fp16(modules), the admission rule RegionContract applies
//   before it builds a Guard.
//
// Design.  Building a Guard compiles the region into a check program: a flat
// list of Checks, each one comparison of a live object against what the
// snapshot saw, tagged with the ValueError message it raises.  validate()
// runs the program front to back and stops at the first failing check, so
// the list order is the order in which drifts are reported:
//   1. torch's global module hooks are empty;
//   2. every class's forward is the snapshot's function;
//   3. per module, in region order: its class, its __dict__ object, training
//      is False, the four hook dicts are empty, the children (count, then
//      identity), the forward binding (unless ignored), the operator
//      attributes, then _parameters and _buffers (count, then per slot the
//      object's identity and its tensor fingerprint).
// Reading a key that has disappeared from a module __dict__ raises
// "Region attribute removed".
#include <pybind11/pybind11.h>
#include <torch/csrc/autograd/python_variable.h>

#include <string>
#include <vector>

namespace py = pybind11;

namespace {

[[noreturn]] void python_error() { throw py::error_already_set(); }

// d[key] or nullptr (borrowed); lookup errors propagate.
PyObject* item(PyObject* d, PyObject* key) {
  PyObject* v = PyDict_GetItemWithError(d, key);
  if (!v && PyErr_Occurred()) python_error();
  return v;
}

PyObject* require_dict(PyObject* v) {
  if (!v || !PyDict_Check(v)) throw py::value_error("Expected a module state dictionary");
  return v;
}

Py_ssize_t length(PyObject* v) {
  const Py_ssize_t n = PyObject_Length(v);
  if (n < 0) python_error();
  return n;
}

py::str name(const char* s) {
  PyObject* v = PyUnicode_InternFromString(s);
  if (!v) python_error();
  return py::reinterpret_steal<py::str>(v);
}

// What a captured graph bakes in about a parameter or buffer.
struct Fingerprint {
  uint32_t version = 0;
  const void* data = nullptr;
  int64_t offset = 0;
  c10::ScalarType dtype = c10::ScalarType::Undefined;
  c10::Device device{c10::DeviceType::CPU};
  std::vector<int64_t> shape;  // sizes followed by strides
  bool grad = false;

  static Fingerprint of(PyObject* tensor) {
    const at::Tensor& t = THPVariable_Unpack(tensor);
    Fingerprint f;
    f.version = t.unsafeGetTensorImpl()->version_counter().current_version();
    f.data = t.const_data_ptr();
    f.offset = t.storage_offset();
    f.dtype = t.scalar_type();
    f.device = t.device();
    f.shape = t.sizes().vec();
    for (int64_t s : t.strides()) f.shape.push_back(s);
    f.grad = t.requires_grad();
    return f;
  }
  bool operator==(const Fingerprint& o) const {
    return version == o.version && data == o.data && offset == o.offset && dtype == o.dtype &&
           device == o.device && shape == o.shape && grad == o.grad;
  }
};

enum class Test {
  kEmptyAttr,     // len(getattr(subject, key)) == 0
  kAttrIs,        // getattr(subject, key) is expected
  kTypeIs,        // type(subject) is expected
  kDictIs,        // subject.__dict__ is expected
  kKeyIs,         // subject[key] is expected               (subject: a module __dict__)
  kKeyEmpty,      // len(subject[key]) == 0
  kKeyCount,      // len(subject[key]) == count, subject[key] a dict
  kEntryIs,       // subject[key].get(entry) is expected
  kForward,       // subject's instance forward, if any, binds expected (function) to bound (self)
  kKeyEquals,     // subject[key] is, or == , expected; a missing key fails the check
  kFingerprint,   // the tensor object `expected` still has fingerprint `print`
};

struct Check {
  Test test;
  const char* message;  // the ValueError raised when the check fails
  py::object subject, key, entry, expected, bound;
  Py_ssize_t count = 0;
  bool instance_forward = false;
  Fingerprint print;
};

// subject[key], which the snapshot saw: its disappearance is itself a drift.
PyObject* present(const py::object& subject, const py::object& key) {
  PyObject* v = item(subject.ptr(), key.ptr());
  if (!v) throw py::value_error("Region attribute removed");
  return v;
}

bool passes(const Check& c) {
  switch (c.test) {
    case Test::kEmptyAttr: {
      py::object v = py::reinterpret_steal<py::object>(PyObject_GetAttr(c.subject.ptr(), c.key.ptr()));
      if (!v) python_error();
      return length(v.ptr()) == 0;
    }
    case Test::kAttrIs: {
      py::object v = py::reinterpret_steal<py::object>(PyObject_GetAttr(c.subject.ptr(), c.key.ptr()));
      if (!v) python_error();
      return v.ptr() == c.expected.ptr();
    }
    case Test::kTypeIs:
      return reinterpret_cast<PyObject*>(Py_TYPE(c.subject.ptr())) == c.expected.ptr();
    case Test::kDictIs: {
      py::object v = py::reinterpret_steal<py::object>(PyObject_GenericGetDict(c.subject.ptr(), nullptr));
      if (!v) python_error();
      return v.ptr() == c.expected.ptr();
    }
    case Test::kKeyIs:
      return present(c.subject, c.key) == c.expected.ptr();
    case Test::kKeyEmpty:
      return length(present(c.subject, c.key)) == 0;
    case Test::kKeyCount:
      return length(require_dict(present(c.subject, c.key))) == c.count;
    case Test::kEntryIs:
      return item(require_dict(present(c.subject, c.key)), c.entry.ptr()) == c.expected.ptr();
    case Test::kForward: {
      PyObject* f = item(c.subject.ptr(), c.key.ptr());
      if (!f) return !c.instance_forward;  // the class forward serves, as at the snapshot
      return PyMethod_Check(f) && PyMethod_Function(f) == c.expected.ptr() && PyMethod_Self(f) == c.bound.ptr();
    }
    case Test::kKeyEquals: {
      PyObject* v = item(c.subject.ptr(), c.key.ptr());
      if (!v) return false;
      if (v == c.expected.ptr()) return true;
      const int eq = PyObject_RichCompareBool(v, c.expected.ptr(), Py_EQ);
      if (eq < 0) python_error();
      return eq == 1;
    }
    case Test::kFingerprint:
      return Fingerprint::of(c.expected.ptr()) == c.print;
  }
  return false;
}

class Guard {
 public:
  Guard(py::iterable modules, py::set ignored, py::iterable attributes) {
    std::vector<py::object> attrs;
    for (auto a : attributes) attrs.push_back(py::reinterpret_borrow<py::object>(a));

    py::object registry = py::module_::import("torch.nn.modules.module");
    for (const char* hooks : {"_global_forward_hooks", "_global_forward_pre_hooks", "_global_backward_hooks",
                              "_global_backward_pre_hooks"})
      add(head_, Test::kEmptyAttr, "Global module hooks are unsupported", registry, name(hooks));

    std::vector<Check> body;
    std::vector<PyObject*> classes;
    for (auto m : modules) {
      py::object module = py::reinterpret_borrow<py::object>(m);
      py::object cls = py::reinterpret_borrow<py::object>(reinterpret_cast<PyObject*>(Py_TYPE(module.ptr())));
      bool known = false;
      for (PyObject* c : classes) known = known || c == cls.ptr();
      if (!known) {
        classes.push_back(cls.ptr());
        add(head_, Test::kAttrIs, "Module class forward changed", cls, forward_, py::object(), cls.attr("forward"));
      }
      compile_module(body, module, cls, ignored.contains(module), attrs);
    }
    head_.insert(head_.end(), std::make_move_iterator(body.begin()), std::make_move_iterator(body.end()));
    validate();
  }

  void validate() const {
    for (const Check& c : head_)
      if (!passes(c)) throw py::value_error(c.message);
  }

 private:
  static Check& add(std::vector<Check>& program, Test test, const char* message, py::object subject,
                    py::object key = py::object(), py::object entry = py::object(),
                    py::object expected = py::object()) {
    Check c;
    c.test = test;
    c.message = message;
    c.subject = std::move(subject);
    c.key = std::move(key);
    c.entry = std::move(entry);
    c.expected = std::move(expected);
    program.push_back(std::move(c));
    return program.back();
  }

  void compile_module(std::vector<Check>& out, const py::object& module, const py::object& cls, bool ignored,
                      const std::vector<py::object>& attrs) {
    py::object state = module.attr("__dict__");
    PyObject* d = require_dict(state.ptr());
    py::object bound = module.attr("forward");
    if (!PyMethod_Check(bound.ptr())) throw py::value_error("Expected a bound module forward");

    add(out, Test::kTypeIs, "Region module class changed", module, {}, {}, cls);
    add(out, Test::kDictIs, "Region module dictionary changed", module, {}, {}, state);
    add(out, Test::kKeyIs, "Region is inference-only", state, training_, {},
        py::reinterpret_borrow<py::object>(Py_False));
    for (const char* hooks : {"_forward_hooks", "_forward_pre_hooks", "_backward_hooks", "_backward_pre_hooks"})
      add(out, Test::kKeyEmpty, "Region hooks changed", state, name(hooks));

    PyObject* children = require_dict(present(state, modules_));
    add(out, Test::kKeyCount, "Region children changed", state, modules_).count = PyDict_Size(children);
    for (auto kv : py::reinterpret_borrow<py::dict>(children))
      add(out, Test::kEntryIs, "Region child identity changed", state, modules_,
          py::reinterpret_borrow<py::object>(kv.first), py::reinterpret_borrow<py::object>(kv.second));

    if (!ignored) {
      Check& f = add(out, Test::kForward, "Region forward changed", state, forward_, {},
                     py::reinterpret_borrow<py::object>(PyMethod_Function(bound.ptr())));
      f.bound = py::reinterpret_borrow<py::object>(PyMethod_Self(bound.ptr()));
      f.instance_forward = item(d, forward_.ptr()) != nullptr;
    }

    for (const py::object& a : attrs)
      if (PyObject* v = item(d, a.ptr()))
        add(out, Test::kKeyEquals, "Region operator configuration changed", state, a, {},
            py::reinterpret_borrow<py::object>(v));

    for (const py::str* key : {&parameters_, &buffers_}) {
      PyObject* slots = require_dict(present(state, *key));
      add(out, Test::kKeyCount, "Region parameter/buffer set changed", state, *key).count = PyDict_Size(slots);
      for (auto kv : py::reinterpret_borrow<py::dict>(slots)) {
        py::object value = py::reinterpret_borrow<py::object>(kv.second);
        if (!value.is_none() && !THPVariable_Check(value.ptr()))
          throw py::type_error("Expected a Tensor or None in module parameters/buffers");
        add(out, Test::kEntryIs, "Region parameter/prepack identity changed", state, *key,
            py::reinterpret_borrow<py::object>(kv.first), value);
        if (value.is_none()) continue;
        Check& t = add(out, Test::kFingerprint, "Region parameter/prepack version or gradient mode changed", state,
                       {}, {}, value);
        t.print = Fingerprint::of(value.ptr());
        t.print.grad = false;  // a frozen region holds no tensor that requires grad
      }
    }
  }

  py::str training_ = name("training"), modules_ = name("_modules"), forward_ = name("forward");
  py::str parameters_ = name("_parameters"), buffers_ = name("_buffers");
  std::vector<Check> head_;  // the check program, in reporting order
};

// Admission rule of a frozen fp16 region (RegionContract's constructor,
// region_contract.py:15-24 in the reference): every parameter and buffer of
// every module is a version-counted fp16 tensor on the npu device without
// gradient.  Tensors are visited module by module, parameters before buffers,
// and the first offender raises ValueError.  An inference-mode tensor has no
// version counter for the guard to fingerprint.
void require_frozen_fp16(py::iterable modules) {
  const py::str keys[2] = {name("_parameters"), name("_buffers")};
  for (auto m : modules) {
    py::object state = py::reinterpret_borrow<py::object>(m).attr("__dict__");
    PyObject* d = require_dict(state.ptr());
    for (const auto& key : keys) {
      PyObject* slots = item(d, key.ptr());
      if (!slots) continue;
      for (auto kv : py::reinterpret_borrow<py::dict>(require_dict(slots))) {
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
