// aten / thin_backend / thin_fused kernels of the PrivateUse1 backend, each a
// thin host wrapper over the thin_hip C ABI.
//
// Reference interfaces served (names, argument meaning, error messages):
//   ops.cpp:419-524        cat, binary add/sub/mul/div, silu_
//   aten_adapter.cpp:25-112 sigmoid, silu, upsample_nearest2d, conv/pool rejects
//   softmax_host.cpp:51-92 _softmax
//   backend.cpp:207-356    thin_backend::add/sigmoid/upsample_nearest2d + Meta
#include "thin_runtime.h"

#include <ATen/ExpandUtils.h>
#include <ATen/MemoryOverlap.h>
#include <ATen/WrapDimUtils.h>
#include <c10/core/GradMode.h>
#include <torch/library.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

namespace thin_ops {

using namespace thin_rt;

void trace(const char* aten, const char* target) {
  const char* enabled = std::getenv("THIN_ATEN_TRACE");
  if (enabled && std::string(enabled) == "1") std::fprintf(stderr, "THIN_ATEN %s -> %s device=npu:0\n", aten, target);
}

bool float_type(const at::Tensor& t) { return t.scalar_type() == at::kFloat || t.scalar_type() == at::kHalf; }

// ------------------------------------------------------------------ binary
// ops.cpp:464-497.  A 0-d CPU operand is converted to the tensor's dtype
// first, as the reference converts it (ops.cpp:466-467), so x * (1/sqrt(32))
// multiplies by the fp16 value of 1/sqrt(32) for every op (scalar_operand).

at::Tensor binary(const at::Tensor& input, const at::Tensor& other, int op, const at::Scalar& alpha = 1) {
  const bool x_scalar = input.is_cpu() && input.dim() == 0;
  const bool y_scalar = other.is_cpu() && other.dim() == 0;
  TORCH_CHECK(!(x_scalar && y_scalar), "binary requires an NPU tensor operand");
  if (x_scalar || y_scalar) {
    const at::Tensor& t = x_scalar ? other : input;
    const at::Tensor& s = x_scalar ? input : other;
    inference(t, "thin ops");
    TORCH_CHECK(float_type(t), "binary supports float32/float16");
    select(t.device());
    auto out = at::empty(t.sizes(), t.options().memory_format(c10::MemoryFormat::Contiguous));
    if (!t.numel()) return out;
    thin_desc td = desc(t), od = desc(out);
    check(thin_binary_scalar(op, &td, scalar_operand(s, t.scalar_type()), x_scalar ? 1 : 0, &od,
                             alpha.toFloat(), stream()),
          "thin binary");
    after_launch();
    return out;
  }
  auto sizes = at::infer_size(input.sizes(), other.sizes());
  at::Tensor x = input.sizes() == sizes ? input : input.expand(sizes);
  at::Tensor y = other.sizes() == sizes ? other : other.expand(sizes);
  inference(x, "thin ops");
  inference(y, "thin ops");
  TORCH_CHECK(x.device() == y.device() && x.scalar_type() == y.scalar_type(),
              "binary requires matching device, shape and dtype");
  TORCH_CHECK(float_type(x), "binary supports float32/float16");
  select(x.device());
  auto out = at::empty(sizes, x.options().memory_format(c10::MemoryFormat::Contiguous));
  if (!out.numel()) return out;
  thin_desc xd = desc(x), yd = desc(y), od = desc(out);
  check(thin_binary(op, &xd, &yd, &od, alpha.toFloat(), stream()), "thin binary");
  after_launch();
  return out;
}
at::Tensor sub(const at::Tensor& x, const at::Tensor& y, const at::Scalar& alpha) { return binary(x, y, THIN_SUB, alpha); }
at::Tensor add(const at::Tensor& x, const at::Tensor& y, const at::Scalar& alpha) { return binary(x, y, THIN_ADD, alpha); }
at::Tensor mul(const at::Tensor& x, const at::Tensor& y) { return binary(x, y, THIN_MUL); }
at::Tensor div(const at::Tensor& x, const at::Tensor& y) { return binary(x, y, THIN_DIV); }

// ------------------------------------------------------------------ unary
at::Tensor unary_out(const at::Tensor& x, int op, const char* what) {
  inference(x, what);
  TORCH_CHECK(float_type(x), what, " supports float32 and float16");
  select(x.device());
  auto out = at::empty(x.sizes(), x.options().memory_format(c10::MemoryFormat::Contiguous));
  if (!x.numel()) return out;
  thin_desc xd = desc(x), od = desc(out);
  check(thin_unary(op, &xd, &od, stream()), what);
  after_launch();
  return out;
}

// ops.cpp:498-512: in place on any strided view (no pack / copy back needed).
at::Tensor& silu_(at::Tensor& x) {
  inference(x, "thin ops");
  TORCH_CHECK(float_type(x), "silu_ supports float32/float16");
  at::assert_no_internal_overlap(x);
  if (!x.numel()) return x;
  select(x.device());
  thin_desc d = desc(x);
  check(thin_unary(THIN_SILU, &d, &d, stream()), "thin silu_");
  after_launch();
  return x;
}

// aten_adapter.cpp:94-105
at::Tensor sigmoid(const at::Tensor& x) {
  TORCH_CHECK(!x.requires_grad() || !c10::GradMode::is_enabled(),
              "thin aten sigmoid is inference-only; use no_grad/inference_mode");
  trace("aten::sigmoid", "thin_unary(SIGMOID)");
  return unary_out(x.detach(), THIN_SIGMOID, "sigmoid");
}
at::Tensor silu(const at::Tensor& x) {
  TORCH_CHECK(!x.requires_grad() || !c10::GradMode::is_enabled(),
              "thin aten silu is inference-only; use no_grad/inference_mode");
  trace("aten::silu", "thin_unary(SILU)");
  return unary_out(x.detach(), THIN_SILU, "silu");
}

// ------------------------------------------------------------------ cat
// aten::cat with torch.cat semantics (the reference's thin_ops::cat,
// ops.cpp:419-462).  Legacy 1-D empty tensors are accepted anywhere in the list
// and contribute nothing; the first contributing input fixes the output's
// rank, dtype, device and the sizes outside `dim`.  Inputs are launched in
// groups of THIN_MAX_CAT_INPUTS, each into its slice of the output.
namespace {

bool legacy_empty(const at::Tensor& t) { return t.dim() == 1 && t.numel() == 0; }

struct CatShape {
  std::vector<at::Tensor> parts;  // contributing inputs, in list order
  std::vector<int64_t> sizes;     // output sizes
  int64_t dim = 0;
};

CatShape cat_shape(const at::ITensorListRef& inputs, int64_t dim) {
  const std::vector<at::Tensor> all(inputs.begin(), inputs.end());
  TORCH_CHECK(!all.empty(), "cat expects a nonempty tensor list");
  for (const auto& t : all) {
    inference(t, "thin ops");
    TORCH_CHECK(t.dim() > 0, "cat cannot concatenate scalar tensors");
  }
  const auto first = std::find_if(all.begin(), all.end(), [](const at::Tensor& t) { return !legacy_empty(t); });
  const at::Tensor& shape = first == all.end() ? all.front() : *first;
  CatShape c;
  c.dim = at::maybe_wrap_dim(dim, shape.dim());
  c.sizes = shape.sizes().vec();
  c.sizes[c.dim] = 0;
  for (const auto& t : all) {
    TORCH_CHECK(t.device() == shape.device() && t.scalar_type() == shape.scalar_type(),
                "cat requires matching device and dtype");
    if (legacy_empty(t)) continue;
    TORCH_CHECK(t.dim() == shape.dim(), "cat rank mismatch");
    const auto same_outside = [&](int64_t d) { return d == c.dim || t.size(d) == shape.size(d); };
    for (int64_t d = 0; d < t.dim(); ++d)
      TORCH_CHECK(same_outside(d), "cat shape mismatch outside concatenation dimension");
    c.sizes[c.dim] += t.size(c.dim);
    c.parts.push_back(t);
  }
  return c;
}

}  // namespace

at::Tensor cat(const at::ITensorListRef& inputs, int64_t dim) {
  const CatShape c = cat_shape(inputs, dim);
  const at::Tensor& like = c.parts.empty() ? *inputs.begin() : c.parts.front();
  select(like.device());
  auto out = at::empty(c.sizes, like.options().memory_format(c10::MemoryFormat::Contiguous));
  if (!out.numel()) return out;
  int64_t start = 0;
  for (size_t g = 0; g < c.parts.size(); g += THIN_MAX_CAT_INPUTS) {
    const size_t n = std::min<size_t>(THIN_MAX_CAT_INPUTS, c.parts.size() - g);
    std::vector<thin_desc> ds;
    int64_t width = 0;
    for (size_t k = 0; k < n; ++k) {
      ds.push_back(desc(c.parts[g + k]));
      width += c.parts[g + k].size(c.dim);
    }
    at::Tensor slice = c.parts.size() <= THIN_MAX_CAT_INPUTS ? out : out.narrow(c.dim, start, width);
    thin_desc od = desc(slice);
    check(thin_cat(ds.data(), (int32_t)n, (int32_t)c.dim, &od, stream()), "thin cat");
    start += width;
  }
  after_launch();
  return out;
}

// ------------------------------------------------------------------ softmax
at::Tensor softmax(const at::Tensor& x, int64_t dim, bool half_to_float) {
  TORCH_CHECK(x.device().type() == kDevice && !x.requires_grad(), "softmax requires inference-only NPU input");
  TORCH_CHECK(float_type(x), "softmax supports float32/float16");
  TORCH_CHECK(!half_to_float || x.scalar_type() == at::kHalf, "half_to_float requires float16 input");
  dim = at::maybe_wrap_dim(dim, x.dim());
  select(x.device());
  auto dtype = half_to_float ? at::kFloat : x.scalar_type();
  auto out = at::empty(x.sizes(), x.options().dtype(dtype).memory_format(c10::MemoryFormat::Contiguous));
  if (!x.numel()) return out;
  thin_desc xd = desc(x), od = desc(out);
  check(thin_softmax(&xd, (int32_t)dim, &od, stream()), "thin softmax");
  after_launch();
  return out;
}

// ------------------------------------------------------------------ upsample
at::Tensor upsample_nchw(const at::Tensor& x, const char* what) {
  TORCH_CHECK(!x.requires_grad() || !c10::GradMode::is_enabled(), what, " is inference-only");
  TORCH_CHECK(x.device().type() == kDevice, what, " requires an NPU tensor");
  TORCH_CHECK(x.dim() == 4, what, " requires NCHW");
  TORCH_CHECK(float_type(x), what, " supports float32/float16");
  TORCH_CHECK(x.size(1) > 0 && x.size(2) > 0 && x.size(3) > 0, "C, H, W must be positive");
  select(x.device());
  auto y = at::empty({x.size(0), x.size(1), x.size(2) * 2, x.size(3) * 2}, x.options());
  if (!y.numel()) return y;
  thin_desc xd = desc(x), yd = desc(y);
  check(thin_upsample2x_nchw(&xd, &yd, stream()), what);
  after_launch();
  return y;
}

void validate_scale(std::optional<double> scale) {
  TORCH_CHECK(!scale || *scale == 2.0, "thin aten nearest2d supports scale=2 only");
}

// aten_adapter.cpp:85-93
at::Tensor aten_upsample_nearest2d(const at::Tensor& input, at::IntArrayRef output_size,
                                   std::optional<double> scales_h, std::optional<double> scales_w) {
  TORCH_CHECK(input.dim() == 4 && output_size.size() == 2 && output_size[0] == input.size(2) * 2 &&
                  output_size[1] == input.size(3) * 2,
              "thin aten nearest2d requires a 2x output size");
  validate_scale(scales_h);
  validate_scale(scales_w);
  trace("aten::upsample_nearest2d", "thin_upsample2x_nchw");
  return upsample_nchw(input.detach(), "upsample_nearest2d");
}

// ------------------------------------------------------------------ max pool
// NCHW stride-1 max pool (backend.cpp:245-266, k5) through thin_maxpool2d_nchw.
at::Tensor maxpool_nchw(const at::Tensor& x, int64_t kernel, const char* what) {
  TORCH_CHECK(!x.requires_grad() || !c10::GradMode::is_enabled(), what, " is inference-only");
  TORCH_CHECK(x.device().type() == kDevice, what, " requires an NPU tensor");
  TORCH_CHECK(x.dim() == 4 && x.size(1) > 0 && x.size(2) > 0 && x.size(3) > 0, what,
              " requires NCHW with positive C/H/W");
  TORCH_CHECK(float_type(x), what, " supports float32 and float16");
  select(x.device());
  auto y = at::empty(x.sizes(), x.options().memory_format(c10::MemoryFormat::Contiguous));
  if (!y.numel()) return y;
  thin_desc xd = desc(x), yd = desc(y);
  check(thin_maxpool2d_nchw(&xd, (int32_t)kernel, &yd, stream()), what);
  after_launch();
  return y;
}

int64_t square(at::IntArrayRef values, const char* name) {
  TORCH_CHECK(values.size() == 1 || values.size() == 2, "thin aten: ", name, " must have one or two elements");
  TORCH_CHECK(values.size() == 1 || values[0] == values[1], "thin aten: asymmetric ", name, " is unsupported");
  return values[0];
}

// aten_adapter.cpp:61-80: k5/s1/p2/d1 only; indices are a zero placeholder.
std::tuple<at::Tensor, at::Tensor> max_pool2d_with_indices(const at::Tensor& input, at::IntArrayRef kernel,
                                                           at::IntArrayRef stride, at::IntArrayRef padding,
                                                           at::IntArrayRef dilation, bool ceil_mode) {
  TORCH_CHECK(square(kernel, "kernel_size") == 5 && (stride.empty() ? 5 : square(stride, "stride")) == 1 &&
                  square(padding, "padding") == 2 && square(dilation, "dilation") == 1 && !ceil_mode,
              "thin aten maxpool supports only k5/s1/p2/d1, ceil_mode=False");
  trace("aten::max_pool2d_with_indices", "thin_maxpool2d_nchw (indices=zeros placeholder)");
  auto values = maxpool_nchw(input.detach(), 5, "max_pool2d");
  auto indices = at::empty(values.sizes(), values.options().dtype(at::kLong));
  if (indices.numel()) {
    thin_desc id = desc(indices);
    check(thin_fill(&id, 0.0, 0, stream()), "zero placeholder indices");
    after_launch();
  }
  return {values, indices};
}

// ------------------------------------------------------------------ rejects
// The convolution / bmm family is not part of this backend: callers get the
// reference's "thin aten" style error rather than a CPU fallback.
at::Tensor convolution(const at::Tensor&, const at::Tensor&, const std::optional<at::Tensor>&, at::IntArrayRef,
                       at::IntArrayRef, at::IntArrayRef, bool, at::IntArrayRef, int64_t) {
  TORCH_CHECK(false, "thin aten convolution is not provided by the MI355X tensor-library backend");
}

// ------------------------------------------------------------------ thin_backend::
// backend.cpp:207-244,269-286
at::Tensor tb_add(const at::Tensor& x, const at::Tensor& y) {
  TORCH_CHECK(!x.requires_grad() && !y.requires_grad(), "thin_backend.add is inference-only");
  TORCH_CHECK(x.device() == y.device() && x.device().type() == kDevice, "add requires tensors on the same NPU");
  TORCH_CHECK(x.scalar_type() == at::kFloat && y.scalar_type() == at::kFloat && x.sizes() == y.sizes(),
              "add requires matching float32 tensors");
  return binary(x, y, THIN_ADD);
}
at::Tensor tb_sigmoid(const at::Tensor& x) {
  TORCH_CHECK(!x.requires_grad(), "thin_backend.sigmoid is inference-only");
  TORCH_CHECK(x.device().type() == kDevice, "sigmoid requires an NPU tensor");
  TORCH_CHECK(float_type(x), "sigmoid supports float32 and float16");
  return unary_out(x, THIN_SIGMOID, "sigmoid");
}
at::Tensor tb_upsample(const at::Tensor& x) { return upsample_nchw(x, "upsample_nearest2d"); }
at::Tensor tb_maxpool2d(const at::Tensor& x) { return maxpool_nchw(x, 5, "maxpool2d"); }
at::Tensor tb_unsupported1(const at::Tensor&) {
  TORCH_CHECK(false, "thin_backend: this operator is not provided by the MI355X tensor-library backend");
}
at::Tensor tb_conv_unsupported(const at::Tensor&, const at::Tensor&, const std::optional<at::Tensor>&, int64_t,
                               int64_t, bool) {
  TORCH_CHECK(false, "thin_backend.conv2d is not provided by the MI355X tensor-library backend");
}
at::Tensor tb_conv_prepared(const at::Tensor&, const at::Tensor&, const at::Tensor&, const std::optional<at::Tensor>&,
                            int64_t, int64_t, bool, bool) {
  TORCH_CHECK(false, "thin_backend.conv2d_prepared is not provided by the MI355X tensor-library backend");
}
at::Tensor tb_conv_fused(const at::Tensor&, const at::Tensor&, const std::optional<at::Tensor>&, int64_t, int64_t,
                         bool, bool) {
  TORCH_CHECK(false, "thin_backend.conv2d_fused is not provided by the MI355X tensor-library backend");
}
at::Tensor tb_nms(const at::Tensor&, const at::Tensor&, double) {
  TORCH_CHECK(false, "thin_backend.nms is not provided by the MI355X tensor-library backend");
}

// Meta kernels (backend.cpp:287-311)
at::Tensor add_meta(const at::Tensor& x, const at::Tensor& y) {
  TORCH_CHECK(x.sizes() == y.sizes() && x.scalar_type() == at::kFloat && y.scalar_type() == at::kFloat,
              "add requires matching float32 tensors");
  return at::empty(x.sizes(), x.options());
}
at::Tensor sigmoid_meta(const at::Tensor& x) {
  TORCH_CHECK(float_type(x), "sigmoid supports float32 and float16");
  return at::empty(x.sizes(), x.options());
}
at::Tensor maxpool2d_meta(const at::Tensor& x) { return at::empty(x.sizes(), x.options()); }
at::Tensor upsample_meta(const at::Tensor& x) {
  TORCH_CHECK(x.dim() == 4, "upsample_nearest2d requires contiguous NCHW");
  TORCH_CHECK(float_type(x), "upsample_nearest2d supports float32/float16");
  TORCH_CHECK(x.size(1) > 0 && x.size(2) > 0 && x.size(3) > 0, "C, H, W must be positive");
  return at::empty({x.size(0), x.size(1), x.size(2) * 2, x.size(3) * 2}, x.options());
}
at::Tensor conv2d_meta(const at::Tensor& x, const at::Tensor& w, const std::optional<at::Tensor>&, int64_t stride,
                       int64_t pad, bool fp32_output) {
  TORCH_CHECK(x.dim() == 4 && w.dim() == 4 && w.size(1) == x.size(1), "expected NCHW / OIHW convolution");
  return at::empty({x.size(0), w.size(0), (x.size(2) + 2 * pad - w.size(2)) / stride + 1,
                    (x.size(3) + 2 * pad - w.size(3)) / stride + 1},
                   x.options().dtype(fp32_output ? at::kFloat : x.scalar_type()));
}

// ------------------------------------------------------------------ thin_fused::
// Fused chains of the path (no single reference op; each replaces the
// reference's unfused sequence named in include/thin_hip.h).
at::Tensor silu_add(const at::Tensor& x, const at::Tensor& y) {
  inference(x, "thin_fused.silu_add");
  inference(y, "thin_fused.silu_add");
  TORCH_CHECK(float_type(x) && x.scalar_type() == y.scalar_type(), "silu_add requires matching float16/float32");
  auto sizes = at::infer_size(x.sizes(), y.sizes());
  select(x.device());
  auto out = at::empty(sizes, x.options().memory_format(c10::MemoryFormat::Contiguous));
  if (!out.numel()) return out;
  thin_desc xd = desc(x.expand(sizes)), yd = desc(y.expand(sizes)), od = desc(out);
  check(thin_silu_add(&xd, &yd, &od, stream()), "thin silu_add");
  after_launch();
  return out;
}
at::Tensor affine_silu(const at::Tensor& x, const at::Tensor& s, const at::Tensor& b) {
  inference(x, "thin_fused.affine_silu");
  inference(s, "thin_fused.affine_silu");
  inference(b, "thin_fused.affine_silu");
  TORCH_CHECK(float_type(x) && s.scalar_type() == x.scalar_type() && b.scalar_type() == x.scalar_type(),
              "affine_silu requires matching float16/float32");
  select(x.device());
  auto out = at::empty(x.sizes(), x.options().memory_format(c10::MemoryFormat::Contiguous));
  if (!out.numel()) return out;
  thin_desc xd = desc(x), sd = desc(s.expand(x.sizes())), bd = desc(b.expand(x.sizes())), od = desc(out);
  check(thin_affine_silu(&xd, &sd, &bd, &od, stream()), "thin affine_silu");
  after_launch();
  return out;
}
// Output sizes of upsample_cat: H, W of the first input taken as is, or twice
// those of the first input when every input is upsampled.
std::vector<int64_t> upsample_cat_sizes(at::TensorList xs, at::IntArrayRef upsample) {
  TORCH_CHECK(!xs.empty() && xs.size() == upsample.size(), "upsample_cat expects matching tensor and flag lists");
  const at::Tensor* ref = nullptr;
  int64_t c1 = 0;
  for (size_t i = 0; i < xs.size(); ++i) {
    TORCH_CHECK(xs[i].dim() == 5, "upsample_cat expects NC1HWC0 tensors");
    if (!ref && !upsample[i]) ref = &xs[i];
    c1 += xs[i].size(1);
  }
  const int64_t scale = ref ? 1 : 2;
  if (!ref) ref = &xs[0];
  return {ref->size(0), c1, ref->size(2) * scale, ref->size(3) * scale, ref->size(4)};
}
at::Tensor upsample_cat(at::TensorList xs, at::IntArrayRef upsample) {
  for (const auto& t : xs) inference(t, "thin_fused.upsample_cat");
  auto sizes = upsample_cat_sizes(xs, upsample);
  select(xs[0].device());
  auto out = at::empty(sizes, xs[0].options());
  if (!out.numel()) return out;
  std::vector<thin_desc> ds;
  std::vector<int32_t> up;
  for (size_t i = 0; i < xs.size(); ++i) {
    ds.push_back(desc(xs[i]));
    up.push_back(upsample[i] ? 1 : 0);
  }
  thin_desc od = desc(out);
  check(thin_upsample_cat_nc1hwc0(ds.data(), up.data(), (int32_t)ds.size(), &od, stream()), "thin upsample_cat");
  after_launch();
  return out;
}
at::Tensor dfl_expect(const at::Tensor& x, bool fp32_output) {
  inference(x, "thin_fused.dfl_expect");
  TORCH_CHECK(x.scalar_type() == at::kHalf && x.dim() == 3 && x.size(1) == 64,
              "dfl_expect expects float16 box logits [N,64,A]");
  select(x.device());
  auto out = at::empty({x.size(0), 4, x.size(2)}, x.options().dtype(fp32_output ? at::kFloat : at::kHalf));
  if (!out.numel()) return out;
  thin_desc xd = desc(x), od = desc(out);
  check(thin_dfl_expect(&xd, &od, stream()), "thin dfl_expect");
  after_launch();
  return out;
}

// Anchor-free head decode (whole_blocked.py:118-146): shapes = flattened
// per-level (h, w), strides = per-level strides; boxes are DFL logits
// [B,64,A] or, for reg_max = 1 heads, the distances [B,4,A].
void decode_check(const at::Tensor& boxes, const at::Tensor& scores, at::IntArrayRef shapes,
                  at::ArrayRef<double> strides) {
  TORCH_CHECK(boxes.scalar_type() == at::kHalf && scores.scalar_type() == at::kHalf && boxes.dim() == 3 &&
                  scores.dim() == 3 && (boxes.size(1) == 64 || boxes.size(1) == 4) &&
                  scores.size(0) == boxes.size(0) && scores.size(2) == boxes.size(2),
              "detect_decode expects float16 boxes [B,64,A] (DFL logits) or [B,4,A] (distances) and scores [B,nc,A]");
  TORCH_CHECK(shapes.size() % 2 == 0 && shapes.size() / 2 == strides.size() && !strides.empty() &&
                  strides.size() <= 8,
              "detect_decode expects (h, w) per level and one stride per level (1..8 levels)");
}
at::Tensor detect_decode(const at::Tensor& boxes, const at::Tensor& scores, at::IntArrayRef shapes,
                         at::ArrayRef<double> strides, bool xywh) {
  inference(boxes, "thin_fused.detect_decode");
  inference(scores, "thin_fused.detect_decode");
  decode_check(boxes, scores, shapes, strides);
  select(boxes.device());
  auto out = at::empty({boxes.size(0), 4 + scores.size(1), boxes.size(2)}, boxes.options());
  std::vector<int32_t> hw(shapes.begin(), shapes.end());
  std::vector<double> st(strides.begin(), strides.end());
  thin_desc bd = desc(boxes), sd = desc(scores), od = desc(out);
  check(thin_detect_decode(&bd, &sd, hw.data(), st.data(), (int32_t)st.size(), xywh ? 1 : 0, &od, stream()),
        "thin detect_decode");
  after_launch();
  return out;
}

// SPPF pooling and concat: cat([x, p(x), p(p(x)), ...], 1), p the stride-1
// k x k max pool, NC1HWC0 fp16.
std::vector<int64_t> sppf_sizes(const at::Tensor& x, int64_t kernel, int64_t repeats) {
  TORCH_CHECK(x.scalar_type() == at::kHalf && x.dim() == 5 && x.size(4) == 16,
              "sppf expects float16 NC1HWC0 [N,C1,H,W,16]");
  TORCH_CHECK(kernel >= 1 && kernel <= 15 && kernel % 2 == 1 && repeats >= 1 && repeats <= 8,
              "sppf takes an odd kernel in [1, 15] and 1..8 repeats");
  return {x.size(0), (repeats + 1) * x.size(1), x.size(2), x.size(3), 16};
}
at::Tensor sppf(const at::Tensor& x, int64_t kernel, int64_t repeats) {
  inference(x, "thin_fused.sppf");
  auto sizes = sppf_sizes(x, kernel, repeats);
  select(x.device());
  auto out = at::empty(sizes, x.options());
  if (!out.numel()) return out;
  thin_desc xd = desc(x), od = desc(out);
  check(thin_sppf_nc1hwc0(&xd, (int32_t)kernel, (int32_t)repeats, &od, stream()), "thin sppf");
  after_launch();
  return out;
}

// Meta kernels of thin_fused: the shapes and dtypes of the device kernels.
at::Tensor silu_add_meta(const at::Tensor& x, const at::Tensor& y) {
  TORCH_CHECK(float_type(x) && x.scalar_type() == y.scalar_type(), "silu_add requires matching float16/float32");
  return at::empty(at::infer_size(x.sizes(), y.sizes()), x.options());
}
at::Tensor affine_silu_meta(const at::Tensor& x, const at::Tensor& s, const at::Tensor& b) {
  TORCH_CHECK(float_type(x) && s.scalar_type() == x.scalar_type() && b.scalar_type() == x.scalar_type(),
              "affine_silu requires matching float16/float32");
  return at::empty(x.sizes(), x.options());
}
at::Tensor upsample_cat_meta(at::TensorList xs, at::IntArrayRef upsample) {
  return at::empty(upsample_cat_sizes(xs, upsample), xs[0].options());
}
at::Tensor detect_decode_meta(const at::Tensor& boxes, const at::Tensor& scores, at::IntArrayRef shapes,
                              at::ArrayRef<double> strides, bool) {
  decode_check(boxes, scores, shapes, strides);
  return at::empty({boxes.size(0), 4 + scores.size(1), boxes.size(2)}, boxes.options());
}
at::Tensor sppf_meta(const at::Tensor& x, int64_t kernel, int64_t repeats) {
  return at::empty(sppf_sizes(x, kernel, repeats), x.options());
}
at::Tensor dfl_expect_meta(const at::Tensor& x, bool fp32_output) {
  TORCH_CHECK(x.scalar_type() == at::kHalf && x.dim() == 3 && x.size(1) == 64,
              "dfl_expect expects float16 box logits [N,64,A]");
  return at::empty({x.size(0), 4, x.size(2)}, x.options().dtype(fp32_output ? at::kFloat : at::kHalf));
}

}  // namespace thin_ops

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("cat", TORCH_FN(thin_ops::cat));
  m.impl("silu_", TORCH_FN(thin_ops::silu_));
  m.impl("sub.Tensor", TORCH_FN(thin_ops::sub));
  m.impl("mul.Tensor", TORCH_FN(thin_ops::mul));
  m.impl("div.Tensor", TORCH_FN(thin_ops::div));
  m.impl("add.Tensor", TORCH_FN(thin_ops::add));
  m.impl("sigmoid", TORCH_FN(thin_ops::sigmoid));
  m.impl("silu", TORCH_FN(thin_ops::silu));
  m.impl("_softmax", TORCH_FN(thin_ops::softmax));
  m.impl("upsample_nearest2d", TORCH_FN(thin_ops::aten_upsample_nearest2d));
  m.impl("convolution", TORCH_FN(thin_ops::convolution));
  m.impl("max_pool2d_with_indices", TORCH_FN(thin_ops::max_pool2d_with_indices));
}

TORCH_LIBRARY_IMPL(thin_backend, PrivateUse1, m) {
  m.impl("conv2d_prepare", TORCH_FN(thin_ops::tb_unsupported1));
  m.impl("conv2d_prepared", TORCH_FN(thin_ops::tb_conv_prepared));
  m.impl("conv2d_fused", TORCH_FN(thin_ops::tb_conv_fused));
  m.impl("add", TORCH_FN(thin_ops::tb_add));
  m.impl("sigmoid", TORCH_FN(thin_ops::tb_sigmoid));
  m.impl("maxpool2d", TORCH_FN(thin_ops::tb_maxpool2d));
  m.impl("upsample_nearest2d", TORCH_FN(thin_ops::tb_upsample));
  m.impl("conv2d", TORCH_FN(thin_ops::tb_conv_unsupported));
  m.impl("nms", TORCH_FN(thin_ops::tb_nms));
}

TORCH_LIBRARY_IMPL(thin_backend, AutogradPrivateUse1, m) {
  for (const char* name : {"conv2d_prepare", "conv2d_prepared", "conv2d_fused", "add", "sigmoid", "maxpool2d",
                           "upsample_nearest2d", "conv2d", "nms"})
    m.impl(name, torch::CppFunction::makeFallthrough());
}

TORCH_LIBRARY_IMPL(thin_backend, Meta, m) {
  m.impl("add", TORCH_FN(thin_ops::add_meta));
  m.impl("sigmoid", TORCH_FN(thin_ops::sigmoid_meta));
  m.impl("maxpool2d", TORCH_FN(thin_ops::maxpool2d_meta));
  m.impl("upsample_nearest2d", TORCH_FN(thin_ops::upsample_meta));
  m.impl("conv2d", TORCH_FN(thin_ops::conv2d_meta));
}

TORCH_LIBRARY(thin_fused, m) {
  m.def("silu_add(Tensor x, Tensor y) -> Tensor");
  m.def("affine_silu(Tensor x, Tensor scale, Tensor bias) -> Tensor");
  m.def("upsample_cat(Tensor[] tensors, int[] upsample) -> Tensor");
  m.def("dfl_expect(Tensor x, bool fp32_output=False) -> Tensor");
  m.def("detect_decode(Tensor boxes, Tensor scores, int[] shapes, float[] strides, bool xywh=False) -> Tensor");
  m.def("sppf(Tensor x, int kernel=5, int repeats=3) -> Tensor");
}

TORCH_LIBRARY_IMPL(thin_fused, PrivateUse1, m) {
  m.impl("silu_add", TORCH_FN(thin_ops::silu_add));
  m.impl("affine_silu", TORCH_FN(thin_ops::affine_silu));
  m.impl("upsample_cat", TORCH_FN(thin_ops::upsample_cat));
  m.impl("dfl_expect", TORCH_FN(thin_ops::dfl_expect));
  m.impl("detect_decode", TORCH_FN(thin_ops::detect_decode));
  m.impl("sppf", TORCH_FN(thin_ops::sppf));
}

TORCH_LIBRARY_IMPL(thin_fused, AutogradPrivateUse1, m) {
  for (const char* name : {"silu_add", "affine_silu", "upsample_cat", "dfl_expect", "detect_decode", "sppf"})
    m.impl(name, torch::CppFunction::makeFallthrough());
}

TORCH_LIBRARY_IMPL(thin_fused, Meta, m) {
  m.impl("silu_add", TORCH_FN(thin_ops::silu_add_meta));
  m.impl("affine_silu", TORCH_FN(thin_ops::affine_silu_meta));
  m.impl("upsample_cat", TORCH_FN(thin_ops::upsample_cat_meta));
  m.impl("dfl_expect", TORCH_FN(thin_ops::dfl_expect_meta));
  m.impl("detect_decode", TORCH_FN(thin_ops::detect_decode_meta));
  m.impl("sppf", TORCH_FN(thin_ops::sppf_meta));
}
