// libthin_blocked.so: thin_blocked::pack / unpack (layout_blocked.h:43-69 of
// the reference, registered at conv_blocked.cpp:198-212) -- any N and any
// C / H*W here; thin_blocked::conv raises (convolution is not part of this
// backend).
#include "thin_runtime.h"

#include <torch/library.h>

namespace blocked_conv {
using namespace thin_rt;

at::Tensor pack(const at::Tensor& x) {
  TORCH_CHECK(x.dim() == 4 && x.numel() > 0 && !x.requires_grad() && x.scalar_type() == at::kHalf &&
                  x.device().type() == kDevice,
              "expected FP16 NCHW input");
  select(x.device());
  auto y = at::empty({x.size(0), (x.size(1) + 15) / 16, x.size(2), x.size(3), 16}, x.options());
  thin_desc xd = desc(x), yd = desc(y);
  check(thin_pack_nc1hwc0(&xd, &yd, stream()), "thin_blocked.pack");
  after_launch();
  return y;
}

at::Tensor unpack(const at::Tensor& x) {
  TORCH_CHECK(x.dim() == 5 && x.size(4) == 16 && x.numel() > 0 && !x.requires_grad() &&
                  x.scalar_type() == at::kHalf && x.device().type() == kDevice,
              "expected FP16 NC1HWC0 input");
  select(x.device());
  auto y = at::empty({x.size(0), x.size(1) * 16, x.size(2), x.size(3)}, x.options());
  thin_desc xd = desc(x), yd = desc(y);
  check(thin_unpack_nc1hwc0(&xd, &yd, stream()), "thin_blocked.unpack");
  after_launch();
  return y;
}

at::Tensor conv(const at::Tensor&, const at::Tensor&, const std::optional<at::Tensor>&, int64_t, int64_t, int64_t,
                bool, bool) {
  TORCH_CHECK(false, "thin_blocked.conv is not provided by the MI355X tensor-library backend");
}

}  // namespace blocked_conv

TORCH_LIBRARY(thin_blocked, m) {
  m.def("pack(Tensor x) -> Tensor");
  m.def("unpack(Tensor x) -> Tensor");
  m.def("conv(Tensor x, Tensor packed, Tensor? bias, int co, int kernel, int stride, bool fp32_output=False, bool "
        "fused=False) -> Tensor");
}
TORCH_LIBRARY_IMPL(thin_blocked, PrivateUse1, m) {
  m.impl("conv", TORCH_FN(blocked_conv::conv));
  m.impl("pack", TORCH_FN(blocked_conv::pack));
  m.impl("unpack", TORCH_FN(blocked_conv::unpack));
}
TORCH_LIBRARY_IMPL(thin_blocked, AutogradPrivateUse1, m) {
  m.impl("conv", torch::CppFunction::makeFallthrough());
  m.impl("pack", torch::CppFunction::makeFallthrough());
  m.impl("unpack", torch::CppFunction::makeFallthrough());
}
