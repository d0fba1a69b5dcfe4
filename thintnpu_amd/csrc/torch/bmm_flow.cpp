// libbmm_flow.so: thin_native_flow::bmm / layout_bmm / channel_select and the
// device's aten::bmm (bmm_flow.cpp:253-359 of the reference) over the
// thin_layout_bmm and thin_channel_select C entry points.  Unblocked results
// are the [.., :n] view of a [batch, m, round_up(n, 16)] buffer, as the
// reference returns them (bmm_flow.cpp:314,340).
#include "thin_runtime.h"

#include <torch/library.h>

namespace bmm_flow {
using namespace thin_rt;

at::Tensor layout_bmm(const at::Tensor& a, const at::Tensor& b, bool transpose_a, bool transpose_b,
                      bool blocked_output, int64_t groups, int64_t a_offset, int64_t a_channels, int64_t b_offset,
                      int64_t b_channels) {
  TORCH_CHECK(a.device().type() == kDevice && b.device() == a.device() && a.scalar_type() == at::kHalf &&
                  b.scalar_type() == at::kHalf && (a.dim() == 3 || a.dim() == 4) && (b.dim() == 3 || b.dim() == 4) &&
                  !a.requires_grad() && !b.requires_grad(),
              "bmm requires inference-only same-device FP16 rank-3 or channel-blocked rank-4 tensors");
  select(a.device());
  thin_bmm_layout L{transpose_a, transpose_b, blocked_output, 0, groups, a_offset, a_channels, b_offset, b_channels};
  thin_desc ad = desc(a), bd = desc(b);
  int32_t rank = 0;
  int64_t sizes[4] = {0, 0, 0, 0};
  check(thin_layout_bmm_shape(&ad, &bd, &L, &rank, sizes), "thin_native_flow.layout_bmm");
  at::Tensor result;
  if (blocked_output) {
    result = at::empty({sizes[0], sizes[1], sizes[2], sizes[3]}, a.options());
  } else {
    const int64_t pitch = (sizes[2] + 15) / 16 * 16;
    result = at::empty({sizes[0], sizes[1], pitch}, a.options());
    if (pitch != sizes[2]) result = result.slice(2, 0, sizes[2]);
  }
  thin_desc od = desc(result);
  check(thin_layout_bmm(&ad, &bd, &L, &od, stream()), "thin_native_flow.layout_bmm");
  after_launch();
  return result;
}

at::Tensor bmm(const at::Tensor& a, const at::Tensor& b) {
  TORCH_CHECK(a.dim() == 3 && b.dim() == 3, "bmm requires rank-3 operands");
  return layout_bmm(a, b, false, false, false, 0, 0, -1, 0, -1);
}

at::Tensor channel_select(const at::Tensor& x, int64_t groups, int64_t begin, int64_t count) {
  TORCH_CHECK(x.device().type() == kDevice && x.scalar_type() == at::kHalf && x.dim() == 4 && x.size(0) == 1 &&
                  x.size(3) == 16 && !x.requires_grad(),
              "channel_select expects aligned N=1 FP16 blocked input");
  select(x.device());
  thin_desc xd = desc(x);
  int64_t sizes[4] = {0, 0, 0, 0};
  check(thin_channel_select_shape(&xd, groups, begin, count, sizes), "thin_native_flow.channel_select");
  auto out = at::empty({sizes[0], sizes[1], sizes[2], sizes[3]}, x.options());
  if (!out.numel()) return out;
  thin_desc od = desc(out);
  check(thin_channel_select(&xd, groups, begin, count, &od, stream()), "thin_native_flow.channel_select");
  after_launch();
  return out;
}

// The blocked attention chain of whole_blocked.py:91-103 in one launch: from
// the grouped QKV tensor [1, C1, T, 16] to the mixed values
// [1, heads * head_dim / 16, T, 16], with the bits of channel_select -> mul ->
// layout_bmm -> softmax -> layout_bmm (or layout_bmm -> mul -> ... when
// prescale is false).  `scale` is rounded as a 0-d operand of the chain's mul.
// Shapes outside the fused kernel's range run that chain op by op.
at::Tensor attention(const at::Tensor& qkv, int64_t heads, int64_t key_dim, int64_t head_dim, double scale,
                     bool prescale) {
  TORCH_CHECK(qkv.device().type() == kDevice && qkv.scalar_type() == at::kHalf && qkv.dim() == 4 &&
                  qkv.size(0) == 1 && qkv.size(3) == 16 && !qkv.requires_grad(),
              "attention expects an inference-only N=1 FP16 blocked qkv tensor");
  TORCH_CHECK(heads > 0 && head_dim > 0 && heads * head_dim % 16 == 0,
              "attention requires C0-aligned value channels");
  select(qkv.device());
  const double sv = scalar_operand(at::scalar_tensor(scale, at::kDouble), at::kHalf);
  auto out = at::empty({1, heads * head_dim / 16, qkv.size(2), 16}, qkv.options());
  thin_desc xd = desc(qkv), od = desc(out);
  const thin_status st = thin_attention(&xd, heads, key_dim, head_dim, (float)sv, prescale ? 1 : 0, &od, stream());
  if (st == THIN_OK) {
    after_launch();
    return out;
  }
  if (st != THIN_ERR_UNSUPPORTED) check(st, "thin_native_flow.attention");
  at::Tensor scores;
  if (prescale) {
    scores = layout_bmm(channel_select(qkv, heads, 0, key_dim) * scale, qkv, true, false, false, heads, 0, key_dim,
                        key_dim, key_dim);
  } else {
    scores = layout_bmm(qkv, qkv, true, false, false, heads, 0, key_dim, key_dim, key_dim) * scale;
  }
  return layout_bmm(qkv, scores.softmax(-1), false, true, true, heads, 2 * key_dim, head_dim, 0, -1);
}

}  // namespace bmm_flow

TORCH_LIBRARY_FRAGMENT(thin_native_flow, m) {
  m.def("bmm(Tensor a, Tensor b) -> Tensor");
  m.def("layout_bmm(Tensor a, Tensor b, bool transpose_a=False, bool transpose_b=False, bool blocked_output=False, "
        "int groups=0, int a_offset=0, int a_channels=-1, int b_offset=0, int b_channels=-1) -> Tensor");
  m.def("channel_select(Tensor x, int groups, int begin, int count) -> Tensor");
  m.def("attention(Tensor qkv, int heads, int key_dim, int head_dim, float scale, bool prescale=True) -> Tensor");
}
TORCH_LIBRARY_IMPL(thin_native_flow, PrivateUse1, m) {
  m.impl("bmm", TORCH_FN(bmm_flow::bmm));
  m.impl("layout_bmm", TORCH_FN(bmm_flow::layout_bmm));
  m.impl("channel_select", TORCH_FN(bmm_flow::channel_select));
  m.impl("attention", TORCH_FN(bmm_flow::attention));
}
TORCH_LIBRARY_IMPL(thin_native_flow, AutogradPrivateUse1, m) {
  m.impl("bmm", torch::CppFunction::makeFallthrough());
  m.impl("layout_bmm", torch::CppFunction::makeFallthrough());
  m.impl("channel_select", torch::CppFunction::makeFallthrough());
  m.impl("attention", torch::CppFunction::makeFallthrough());
}
TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("bmm", TORCH_FN(bmm_flow::bmm));
}
