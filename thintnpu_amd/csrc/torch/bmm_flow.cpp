// libbmm_flow.so: the attention-bmm schemas of the reference library and its
// aten::bmm kernel for the device (bmm_flow.cpp:342-359), registered so that
// callers loading every flow library keep working; each raises -- the
// contraction is not part of this backend (the attention row-softmax that
// follows it is).
#include <ATen/ATen.h>
#include <torch/library.h>

namespace {
[[noreturn]] void unsupported(const char* name) {
  TORCH_CHECK(false, "thin_native_flow.", name, " is not provided by the MI355X tensor-library backend");
}
at::Tensor bmm(const at::Tensor&, const at::Tensor&) { unsupported("bmm"); }
at::Tensor aten_bmm(const at::Tensor&, const at::Tensor&) {
  TORCH_CHECK(false, "thin aten bmm is not provided by the MI355X tensor-library backend");
}
at::Tensor layout_bmm(const at::Tensor&, const at::Tensor&, bool, bool, bool, int64_t, int64_t, int64_t, int64_t,
                      int64_t) { unsupported("layout_bmm"); }
at::Tensor channel_select(const at::Tensor&, int64_t, int64_t, int64_t) { unsupported("channel_select"); }
}  // namespace

TORCH_LIBRARY_FRAGMENT(thin_native_flow, m) {
  m.def("bmm(Tensor a, Tensor b) -> Tensor");
  m.def("layout_bmm(Tensor a, Tensor b, bool transpose_a=False, bool transpose_b=False, bool blocked_output=False, "
        "int groups=0, int a_offset=0, int a_channels=-1, int b_offset=0, int b_channels=-1) -> Tensor");
  m.def("channel_select(Tensor x, int groups, int begin, int count) -> Tensor");
}
TORCH_LIBRARY_IMPL(thin_native_flow, PrivateUse1, m) {
  m.impl("bmm", TORCH_FN(bmm));
  m.impl("layout_bmm", TORCH_FN(layout_bmm));
  m.impl("channel_select", TORCH_FN(channel_select));
}
TORCH_LIBRARY_IMPL(thin_native_flow, AutogradPrivateUse1, m) {
  m.impl("bmm", torch::CppFunction::makeFallthrough());
  m.impl("layout_bmm", torch::CppFunction::makeFallthrough());
  m.impl("channel_select", torch::CppFunction::makeFallthrough());
}
TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("bmm", TORCH_FN(aten_bmm));
}
