// libdepthwise_flow.so: the depthwise schema of the reference library
// (depthwise_flow.cpp:218-233), registered for callers that load every flow
// library; it raises -- depthwise convolution is not part of this backend.
#include <ATen/ATen.h>
#include <torch/library.h>

namespace {
at::Tensor depthwise(const at::Tensor&, const at::Tensor&, const std::optional<at::Tensor>&, int64_t, int64_t, bool) {
  TORCH_CHECK(false, "thin_native_flow.depthwise is not provided by the MI355X tensor-library backend");
}
}  // namespace

TORCH_LIBRARY_FRAGMENT(thin_native_flow, m) {
  m.def("depthwise(Tensor x, Tensor packed, Tensor? bias, int kernel, int stride, bool fused=True) -> Tensor");
}
TORCH_LIBRARY_IMPL(thin_native_flow, PrivateUse1, m) { m.impl("depthwise", TORCH_FN(depthwise)); }
