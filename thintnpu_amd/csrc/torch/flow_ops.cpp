// thin_native_flow::upsample / maxpool (libflow_ops.so), mirroring
// flow_ops.cpp:201-266 of the reference.  Both take any N (the reference
// requires N=1, flow_ops.cpp:202); maxpool takes odd kernels up to 15.
#include "thin_runtime.h"

#include <torch/library.h>

namespace blocked_flow {
using namespace thin_rt;

void check_blocked(const at::Tensor& x) {
  TORCH_CHECK(x.device().type() == kDevice && x.dim() == 5 && x.size(4) == 16 &&
                  x.scalar_type() == at::kHalf && !x.requires_grad(),
              "expected inference-only FP16 NC1HWC0 input, C0=16");
}

at::Tensor upsample(const at::Tensor& x) {
  check_blocked(x);
  TORCH_CHECK(x.size(1) > 0 && x.size(2) > 0 && x.size(3) > 0, "blocked spatial operators require positive C1/H/W");
  select(x.device());
  auto y = at::empty({x.size(0), x.size(1), x.size(2) * 2, x.size(3) * 2, 16}, x.options());
  if (!y.numel()) return y;
  thin_desc xd = desc(x), yd = desc(y);
  check(thin_upsample2x_nc1hwc0(&xd, &yd, stream()), "thin_native_flow.upsample");
  after_launch();
  return y;
}

at::Tensor maxpool(const at::Tensor& x, int64_t kernel) {
  check_blocked(x);
  TORCH_CHECK(kernel >= 1 && kernel % 2 == 1, "maxpool kernel must be a positive odd integer");
  TORCH_CHECK(kernel <= 15, "maxpool kernel above 15 is not supported");
  TORCH_CHECK(x.size(1) > 0 && x.size(2) > 0 && x.size(3) > 0, "blocked spatial operators require positive C1/H/W");
  select(x.device());
  auto y = at::empty(x.sizes(), x.options().memory_format(c10::MemoryFormat::Contiguous));
  if (!y.numel()) return y;
  thin_desc xd = desc(x), yd = desc(y);
  check(thin_maxpool_nc1hwc0(&xd, (int32_t)kernel, &yd, stream()), "thin_native_flow.maxpool");
  after_launch();
  return y;
}

}  // namespace blocked_flow

TORCH_LIBRARY_FRAGMENT(thin_native_flow, m) {
  m.def("maxpool(Tensor x, int kernel) -> Tensor");
  m.def("upsample(Tensor x) -> Tensor");
}
TORCH_LIBRARY_IMPL(thin_native_flow, PrivateUse1, m) {
  m.impl("maxpool", TORCH_FN(blocked_flow::maxpool));
  m.impl("upsample", TORCH_FN(blocked_flow::upsample));
}
TORCH_LIBRARY_IMPL(thin_native_flow, AutogradPrivateUse1, m) {
  m.impl("maxpool", torch::CppFunction::makeFallthrough());
  m.impl("upsample", torch::CppFunction::makeFallthrough());
}
