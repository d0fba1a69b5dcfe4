// libselection_flow.so: thin_native_flow::detection_select(_trace), mirroring
// selection_flow.cpp:429-514 of the reference (same schema, checks, output
// shapes and trace order) over thin_detection_select.
#include "thin_runtime.h"

#include <torch/library.h>

namespace detection_selection {
using namespace thin_rt;

std::vector<at::Tensor> run(const at::Tensor& decoded, int64_t max_det, bool agnostic, bool trace) {
  TORCH_CHECK(decoded.device().type() == kDevice && decoded.scalar_type() == at::kHalf && decoded.dim() == 3 &&
                  !decoded.requires_grad(),
              "detection_select expects inference-only device FP16 [B,A,4+nc]");
  TORCH_CHECK(decoded.size(2) > 4 && max_det >= 0, "detection_select requires nc > 0 and max_det >= 0");
  const int64_t batches = decoded.size(0), anchors = decoded.size(1), classes = decoded.size(2) - 4;
  const int64_t k = std::min(max_det, anchors);
  select(decoded.device());
  auto output = at::empty({batches, k, 6}, decoded.options().dtype(at::kFloat));
  if (!trace && (!batches || !k)) return {output};
  at::Tensor maxima, gathered, stage1, top, stage2, anchor_idx, labels;
  if (trace) {
    maxima = at::empty({batches, anchors}, decoded.options());
    stage1 = at::empty({batches, k}, decoded.options().dtype(at::kLong));
    gathered = at::empty({batches, agnostic ? 0 : k, classes}, decoded.options());
    top = at::empty({batches, k}, decoded.options());
    stage2 = at::empty({batches, agnostic ? 0 : k}, decoded.options().dtype(at::kLong));
    anchor_idx = at::empty({batches, k}, decoded.options().dtype(at::kLong));
    labels = at::empty({batches, k}, decoded.options().dtype(at::kLong));
  }
  if (batches && anchors) {
    const size_t ws_bytes = thin_detection_select_workspace(batches, anchors, classes, max_det, agnostic ? 1 : 0);
    at::Tensor ws = empty_bytes((int64_t)ws_bytes);
    thin_select_trace tr{};
    auto ptr = [](const at::Tensor& t) -> void* { return t.defined() && t.numel() ? t.data_ptr() : nullptr; };
    if (trace) {
      tr.class_max = ptr(maxima);
      tr.stage1 = ptr(stage1);
      tr.gathered = ptr(gathered);
      tr.top_values = ptr(top);
      tr.stage2 = ptr(stage2);
      tr.anchors = ptr(anchor_idx);
      tr.labels = ptr(labels);
    }
    thin_desc d = desc(decoded);
    check(thin_detection_select(&d, max_det, agnostic ? 1 : 0, output.numel() ? output.data_ptr() : nullptr,
                                ws.data_ptr(), (size_t)ws.numel(), trace ? &tr : nullptr, stream()),
          "thin_native_flow.detection_select");
    after_launch();
  }
  if (!trace) return {output};
  return {output, maxima, stage1, gathered, top, stage2, anchor_idx, labels};
}

at::Tensor detection_select(const at::Tensor& decoded, int64_t max_det, bool agnostic) {
  return run(decoded, max_det, agnostic, false)[0];
}
std::vector<at::Tensor> detection_select_trace(const at::Tensor& decoded, int64_t max_det, bool agnostic) {
  return run(decoded, max_det, agnostic, true);
}

}  // namespace detection_selection

TORCH_LIBRARY_FRAGMENT(thin_native_flow, m) {
  m.def("detection_select(Tensor decoded, int max_det, bool agnostic=False) -> Tensor");
  m.def("detection_select_trace(Tensor decoded, int max_det, bool agnostic=False) -> Tensor[]");
}
TORCH_LIBRARY_IMPL(thin_native_flow, PrivateUse1, m) {
  m.impl("detection_select", TORCH_FN(detection_selection::detection_select));
  m.impl("detection_select_trace", TORCH_FN(detection_selection::detection_select_trace));
}
TORCH_LIBRARY_IMPL(thin_native_flow, AutogradPrivateUse1, m) {
  m.impl("detection_select", torch::CppFunction::makeFallthrough());
  m.impl("detection_select_trace", torch::CppFunction::makeFallthrough());
}
