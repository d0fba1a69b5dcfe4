// libconv_flow.so: thin_native_flow::pack_input (conv_flow.cpp:406-458 of the
// reference: NCHW -> NC1HWC0 with zero-filled channels beyond C; any N here)
// plus the convolution schemas of that library, which raise because the
// convolution family is not part of this backend.
#include "thin_runtime.h"

#include <torch/library.h>

namespace native_flow {
using namespace thin_rt;

at::Tensor pack_input(const at::Tensor& x) {
  TORCH_CHECK(x.device().type() == kDevice && x.dim() == 4 && x.size(1) > 0 && x.size(2) > 0 && x.size(3) > 0 &&
                  x.scalar_type() == at::kHalf && !x.requires_grad(),
              "expected FP16 NCHW input with positive C/H/W");
  select(x.device());
  auto y = at::empty({x.size(0), (x.size(1) + 15) / 16, x.size(2), x.size(3), 16}, x.options());
  if (!y.numel()) return y;
  thin_desc xd = desc(x), yd = desc(y);
  check(thin_pack_nc1hwc0(&xd, &yd, stream()), "thin_native_flow.pack_input");
  after_launch();
  return y;
}

std::vector<int64_t> plan_values(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t) {
  TORCH_CHECK(false, "thin_native_flow.plan is not provided by the MI355X tensor-library backend");
}
at::Tensor conv(const at::Tensor&, const at::Tensor&, const std::optional<at::Tensor>&, int64_t, int64_t, int64_t,
                bool, bool) {
  TORCH_CHECK(false, "thin_native_flow.conv is not provided by the MI355X tensor-library backend");
}
at::Tensor stem(const at::Tensor&, const at::Tensor&, const std::optional<at::Tensor>&) {
  TORCH_CHECK(false, "thin_native_flow.stem is not provided by the MI355X tensor-library backend");
}

}  // namespace native_flow

TORCH_LIBRARY_FRAGMENT(thin_native_flow, m) {
  m.def("plan(int ci, int co, int h, int w, int kernel, int stride) -> int[]", TORCH_FN(native_flow::plan_values));
  m.def("conv(Tensor x, Tensor packed, Tensor? bias, int co, int kernel, int stride, bool fused=True, bool "
        "nchw_output=False) -> Tensor");
  m.def("stem(Tensor x, Tensor w, Tensor? bias) -> Tensor");
  m.def("pack_input(Tensor x) -> Tensor");
}
TORCH_LIBRARY_IMPL(thin_native_flow, PrivateUse1, m) {
  m.impl("conv", TORCH_FN(native_flow::conv));
  m.impl("stem", TORCH_FN(native_flow::stem));
  m.impl("pack_input", TORCH_FN(native_flow::pack_input));
}
TORCH_LIBRARY_IMPL(thin_native_flow, AutogradPrivateUse1, m) {
  m.impl("conv", torch::CppFunction::makeFallthrough());
  m.impl("stem", torch::CppFunction::makeFallthrough());
  m.impl("pack_input", torch::CppFunction::makeFallthrough());
}
