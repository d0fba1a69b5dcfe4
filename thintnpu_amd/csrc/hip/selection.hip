// YOLO26 NMS-free detection selection: class max per anchor, stable top-K
// over anchors, score gather, stable top-K over the K x nc pairs, index
// mapping and FP32 packing -- bit-exact by construction.
//
// Ordering.  score_key(bits) maps an fp16 encoding to a 16-bit key whose
// ascending order is: NaN first, then descending value, with +0 and -0 equal
// (selection_flow.cpp:30-35).  Candidates are ordered by (key, index); the
// 64-bit record (key << 32) | index is unique, so any correct sort gives the
// stable order, ties resolved by the lower index.
//
// Top-K (K <= kLdsSort): one block per batch.  An exact two-level radix select
// over the 16-bit keys (two 256-bin LDS histograms) finds the threshold key T
// and how many T-keyed candidates to keep; a compaction pass in index order
// (wave ballots give each T-keyed candidate its rank) collects exactly K
// records in LDS, which a bitonic sort orders.  Larger K sorts every record in
// the caller's workspace with a multi-launch bitonic network.
#include "common.h"

#include <string.h>

namespace thin {
namespace {

constexpr uint32_t kSelThreads = 1024;
constexpr uint32_t kLdsSort = 8192;  // records sorted in LDS (64 KiB)
constexpr uint32_t kThreads = 256;

__device__ __forceinline__ uint32_t score_key(uint32_t bits) {
  const uint32_t mag = bits & 0x7fffu;
  if (mag > 0x7c00u) return 0u;       // NaN: best
  if (mag == 0u) return 0x7fffu;      // +0 and -0 compare equal
  return (bits & 0x8000u) ? bits : ((~(bits ^ 0x8000u)) & 0xffffu);
}

// Exact fp16 -> fp32 bit expansion; NaNs keep sign and payload and are quieted
// (selection_flow.cpp:37-51).
__device__ __forceinline__ uint32_t float_bits(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  uint32_t exponent = (h >> 10) & 31u;
  uint32_t mantissa = h & 1023u;
  if (exponent == 31u) return sign | 0x7f800000u | (mantissa << 13) | (mantissa ? 0x00400000u : 0u);
  if (exponent) return sign | ((exponent + 112u) << 23) | (mantissa << 13);
  if (!mantissa) return sign;
  exponent = 113u;
  while (!(mantissa & 1024u)) {
    mantissa <<= 1;
    --exponent;
  }
  return sign | (exponent << 23) | ((mantissa & 1023u) << 13);
}

struct Layout {
  const uint16_t* x;  // fp16 bits of decoded [B, A, 4+nc]
  int64_t sb, sa, sc; // element strides
};

// ---------------------------------------------------------------- stage 1
// bits1[b,a], cls1[b,a]: the first class with the smallest key.
__global__ __launch_bounds__(kThreads) void class_max_kernel(Layout L, int64_t batches, int64_t anchors,
                                                              int64_t classes, uint16_t* bits1, int32_t* cls1,
                                                              uint16_t* trace_max) {
  const int64_t total = batches * anchors;
  for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (int64_t)gridDim.x * kThreads) {
    const int64_t b = t / anchors, a = t - b * anchors;
    const uint16_t* row = L.x + b * L.sb + a * L.sa + 4 * L.sc;
    uint32_t best = 0x10000u, best_bits = 0, best_cls = 0;
    for (int64_t c = 0; c < classes; ++c) {
      const uint32_t bits = row[c * L.sc];
      const uint32_t k = score_key(bits);
      if (k < best) {
        best = k;
        best_bits = bits;
        best_cls = (uint32_t)c;
      }
    }
    bits1[t] = (uint16_t)best_bits;
    cls1[t] = (int32_t)best_cls;
    if (trace_max) trace_max[t] = (uint16_t)best_bits;
  }
}

// ---------------------------------------------------------------- top-K
struct TopkPlan {
  const uint16_t* bits;  // keys are score_key(bits[b * n + i])
  uint32_t n;            // candidates per batch
  uint32_t k;            // selected per batch (<= n)
  int32_t* sel;          // [B, k] selected candidate indices in (key, index) order
};

__global__ __launch_bounds__(kSelThreads) void topk_block_kernel(TopkPlan p) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t wave_eq[kSelThreads / 64];
  __shared__ uint32_t shared_u[4];
  __shared__ uint64_t recs[kLdsSort];
  const uint32_t b = blockIdx.x;
  const uint16_t* bits = p.bits + (size_t)b * p.n;
  const uint32_t n = p.n, K = p.k, tid = threadIdx.x;
  const uint32_t lane = tid & 63u, wave = tid >> 6;

  // level 1: histogram of key >> 8
  for (uint32_t i = tid; i < 256; i += kSelThreads) hist[i] = 0;
  __syncthreads();
  for (uint32_t i = tid; i < n; i += kSelThreads) atomicAdd(&hist[score_key(bits[i]) >> 8], 1u);
  __syncthreads();
  if (tid == 0) {
    uint32_t cum = 0, b1 = 255;
    for (uint32_t q = 0; q < 256; ++q) {
      if (cum + hist[q] >= K) { b1 = q; break; }
      cum += hist[q];
    }
    shared_u[0] = b1;
    shared_u[1] = cum;
  }
  __syncthreads();
  const uint32_t b1 = shared_u[0], below1 = shared_u[1];
  // level 2: histogram of the low byte inside bucket b1
  for (uint32_t i = tid; i < 256; i += kSelThreads) hist[i] = 0;
  __syncthreads();
  for (uint32_t i = tid; i < n; i += kSelThreads) {
    const uint32_t k = score_key(bits[i]);
    if ((k >> 8) == b1) atomicAdd(&hist[k & 0xffu], 1u);
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t cum = below1, t = 255;
    for (uint32_t q = 0; q < 256; ++q) {
      if (cum + hist[q] >= K) { t = q; break; }
      cum += hist[q];
    }
    shared_u[0] = (b1 << 8) | t;   // threshold key T
    shared_u[1] = cum;             // candidates with key < T
    shared_u[2] = 0;               // compaction counter
  }
  __syncthreads();
  const uint32_t T = shared_u[0];
  const uint32_t need = K - shared_u[1];  // T-keyed candidates to keep, lowest index first
  // compaction in index order
  uint32_t eq_base = 0;
  for (uint32_t base = 0; base < n; base += kSelThreads) {
    const uint32_t i = base + tid;
    const uint32_t k = i < n ? score_key(bits[i]) : 0xffffffffu;
    const bool eq = k == T;
    const uint64_t ballot = __ballot(eq);
    const uint32_t in_wave = (uint32_t)__popcll(ballot & ((1ull << lane) - 1ull));
    if (lane == 0) wave_eq[wave] = (uint32_t)__popcll(ballot);
    __syncthreads();
    uint32_t before = 0, chunk_eq = 0;
    for (uint32_t w = 0; w < kSelThreads / 64; ++w) {
      if (w < wave) before += wave_eq[w];
      chunk_eq += wave_eq[w];
    }
    const uint32_t rank = eq_base + before + in_wave;
    if (k < T || (eq && rank < need)) {
      const uint32_t pos = atomicAdd(&shared_u[2], 1u);
      recs[pos] = ((uint64_t)k << 32) | i;
    }
    eq_base += chunk_eq;
    __syncthreads();
  }
  // bitonic sort of the K records (padded to a power of two)
  uint32_t P = 1;
  while (P < K) P <<= 1;
  for (uint32_t i = K + tid; i < P; i += kSelThreads) recs[i] = ~0ull;
  __syncthreads();
  for (uint32_t size = 2; size <= P; size <<= 1) {
    for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
      for (uint32_t i = tid; i < P; i += kSelThreads) {
        const uint32_t l = i ^ stride;
        if (l > i) {
          const uint64_t a = recs[i], c = recs[l];
          const bool up = (i & size) == 0;
          if ((a > c) == up) {
            recs[i] = c;
            recs[l] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  for (uint32_t r = tid; r < K; r += kSelThreads) p.sel[(size_t)b * K + r] = (int32_t)(uint32_t)recs[r];
}

// Large K: records for every candidate, padded to P (power of two) per batch.
__global__ __launch_bounds__(kThreads) void records_kernel(const uint16_t* bits, uint32_t n, uint32_t P,
                                                           uint64_t total, uint64_t* recs) {
  for (uint64_t t = (uint64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (uint64_t)gridDim.x * kThreads) {
    const uint64_t b = t / P;
    const uint32_t i = (uint32_t)(t - b * P);
    recs[t] = i < n ? (((uint64_t)score_key(bits[b * n + i]) << 32) | i) : ~0ull;
  }
}

__global__ __launch_bounds__(kThreads) void bitonic_step_kernel(uint64_t* recs, uint32_t P, uint64_t total,
                                                                uint32_t size, uint32_t stride) {
  for (uint64_t t = (uint64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (uint64_t)gridDim.x * kThreads) {
    const uint64_t b = t / P;
    const uint32_t i = (uint32_t)(t - b * P);
    const uint32_t l = i ^ stride;
    if (l > i) {
      uint64_t* r = recs + b * P;
      const uint64_t a = r[i], c = r[l];
      const bool up = (i & size) == 0;
      if ((a > c) == up) {
        r[i] = c;
        r[l] = a;
      }
    }
  }
}

__global__ __launch_bounds__(kThreads) void take_kernel(const uint64_t* recs, uint32_t P, uint32_t K,
                                                        uint64_t total, int32_t* sel) {
  for (uint64_t t = (uint64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (uint64_t)gridDim.x * kThreads) {
    const uint64_t b = t / K;
    const uint32_t r = (uint32_t)(t - b * K);
    sel[t] = (int32_t)(uint32_t)recs[b * P + r];
  }
}

// ---------------------------------------------------------------- stage 3
// gathered[b, r*nc + c] = bits of x[b, stage1[b,r], 4+c]
__global__ __launch_bounds__(kThreads) void gather_kernel(Layout L, int64_t batches, int64_t K, int64_t classes,
                                                          const int32_t* stage1, uint16_t* gathered,
                                                          uint16_t* trace_gathered) {
  const int64_t per = K * classes, total = batches * per;
  for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (int64_t)gridDim.x * kThreads) {
    const int64_t b = t / per, f = t - b * per;
    const int64_t r = f / classes, c = f - r * classes;
    const int64_t a = stage1[b * K + r];
    const uint16_t v = L.x[b * L.sb + a * L.sa + (4 + c) * L.sc];
    gathered[t] = v;
    if (trace_gathered) trace_gathered[t] = v;
  }
}

// ---------------------------------------------------------------- pack
struct PackArgs {
  Layout L;
  int64_t batches, K, classes;
  int32_t agnostic;
  const int32_t* stage1;
  const int32_t* stage2;
  const uint16_t* bits1;
  const int32_t* cls1;
  const uint16_t* gathered;
  int64_t anchors;
  uint32_t* out;
  thin_select_trace tr;
};

__global__ __launch_bounds__(kThreads) void pack_kernel(PackArgs p) {
  const int64_t total = p.batches * p.K;
  for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (int64_t)gridDim.x * kThreads) {
    const int64_t b = t / p.K;
    int64_t a, label, flat = 0;
    uint32_t sbits;
    if (p.agnostic) {
      a = p.stage1[t];
      label = p.cls1[b * p.anchors + a];
      sbits = p.bits1[b * p.anchors + a];
    } else {
      flat = p.stage2[t];
      const int64_t rank = flat / p.classes;
      label = flat - rank * p.classes;
      a = p.stage1[b * p.K + rank];
      sbits = p.gathered[b * p.K * p.classes + flat];
    }
    const uint16_t* box = p.L.x + b * p.L.sb + a * p.L.sa;
    uint32_t* o = p.out + t * 6;
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = float_bits(box[c * p.L.sc]);
    o[4] = float_bits(sbits);
    o[5] = __float_as_uint((float)label);
    if (p.tr.stage1) static_cast<int64_t*>(p.tr.stage1)[t] = p.stage1[t];
    if (p.tr.stage2 && !p.agnostic) static_cast<int64_t*>(p.tr.stage2)[t] = flat;
    if (p.tr.anchors) static_cast<int64_t*>(p.tr.anchors)[t] = a;
    if (p.tr.labels) static_cast<int64_t*>(p.tr.labels)[t] = label;
    if (p.tr.top_values) static_cast<uint16_t*>(p.tr.top_values)[t] = (uint16_t)sbits;
  }
}

// ---------------------------------------------------------------- host

struct WsLayout {
  size_t bits1, cls1, stage1, gathered, stage2, recs, total;
  uint32_t recs_pitch;  // P for the large-K path (0 = not needed)
};

size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

WsLayout ws_layout(int64_t B, int64_t A, int64_t nc, int64_t max_det, bool agnostic) {
  WsLayout w;
  memset(&w, 0, sizeof w);
  const int64_t K = max_det < A ? max_det : A;
  size_t off = 0;
  w.bits1 = off; off += up256((size_t)(B * A) * 2);
  w.cls1 = off; off += up256((size_t)(B * A) * 4);
  w.stage1 = off; off += up256((size_t)(B * K) * 4);
  if (!agnostic) {
    w.gathered = off; off += up256((size_t)(B * K * nc) * 2);
    w.stage2 = off; off += up256((size_t)(B * K) * 4);
  }
  if (K > (int64_t)kLdsSort) {
    const int64_t n = agnostic ? A : (A > K * nc ? A : K * nc);
    uint64_t P = 1;
    while ((int64_t)P < n) P <<= 1;
    w.recs_pitch = (uint32_t)P;
    w.recs = off; off += up256((size_t)(B * (int64_t)P) * 8);
  }
  w.total = off;
  return w;
}

uint32_t blocks_for(uint64_t total) {
  uint64_t g = (total + kThreads - 1) / kThreads;
  if (g < 1) g = 1;
  if (g > 8192) g = 8192;
  return (uint32_t)g;
}

thin_status topk(const uint16_t* bits, int64_t B, int64_t n, int64_t K, int32_t* sel, uint64_t* recs, uint32_t P,
                 hipStream_t stream) {
  if (K <= (int64_t)kLdsSort) {
    TopkPlan p{bits, (uint32_t)n, (uint32_t)K, sel};
    hipLaunchKernelGGL(topk_block_kernel, dim3((uint32_t)B), dim3(kSelThreads), 0, stream, p);
    THIN_LAUNCH_CHECK("topk_block");
    return THIN_OK;
  }
  THIN_REQUIRE(recs && P >= (uint32_t)n, THIN_ERR_WORKSPACE, "selection: record workspace missing");
  const uint64_t total = (uint64_t)B * P;
  hipLaunchKernelGGL(records_kernel, dim3(blocks_for(total)), dim3(kThreads), 0, stream, bits, (uint32_t)n, P, total,
                     recs);
  for (uint32_t size = 2; size <= P; size <<= 1)
    for (uint32_t stride = size >> 1; stride > 0; stride >>= 1)
      hipLaunchKernelGGL(bitonic_step_kernel, dim3(blocks_for(total)), dim3(kThreads), 0, stream, recs, P, total,
                         size, stride);
  const uint64_t kt = (uint64_t)B * K;
  hipLaunchKernelGGL(take_kernel, dim3(blocks_for(kt)), dim3(kThreads), 0, stream, recs, P, (uint32_t)K, kt, sel);
  THIN_LAUNCH_CHECK("topk_global");
  return THIN_OK;
}

}  // namespace
}  // namespace thin

using namespace thin;

extern "C" size_t thin_detection_select_workspace(int64_t batches, int64_t anchors, int64_t classes,
                                                  int64_t max_det, int32_t agnostic) {
  if (batches < 0 || anchors < 0 || classes < 1 || max_det < 0) return 0;
  return ws_layout(batches, anchors, classes, max_det, agnostic != 0).total;
}

extern "C" thin_status thin_detection_select(const thin_desc* decoded, int64_t max_det, int32_t agnostic, void* out,
                                             void* workspace, size_t workspace_bytes,
                                             const thin_select_trace* trace, hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(desc_valid(decoded), THIN_ERR_INVALID, "detection_select: invalid descriptor");
  THIN_REQUIRE(decoded->dtype == THIN_F16 && decoded->rank == 3, THIN_ERR_INVALID,
               "detection_select expects float16 [B,A,4+nc]");
  THIN_REQUIRE(decoded->sizes[2] > 4 && max_det >= 0, THIN_ERR_INVALID,
               "detection_select requires nc > 0 and max_det >= 0");
  const int64_t B = decoded->sizes[0], A = decoded->sizes[1], nc = decoded->sizes[2] - 4;
  const int64_t K = max_det < A ? max_det : A;
  // With K == 0 only a requested class_max trace has work (selection_flow.cpp:439).
  if (B == 0 || A == 0 || (K == 0 && !(trace && trace->class_max))) return THIN_OK;
  THIN_REQUIRE(out != nullptr || K == 0, THIN_ERR_INVALID, "detection_select: null output");
  THIN_REQUIRE(A < ((int64_t)1 << 31) && K * nc < ((int64_t)1 << 31), THIN_ERR_UNSUPPORTED,
               "detection_select: candidate count exceeds 2^31");
  const bool agn = agnostic != 0;
  const WsLayout w = ws_layout(B, A, nc, max_det, agn);
  THIN_REQUIRE(workspace != nullptr && workspace_bytes >= w.total, THIN_ERR_WORKSPACE,
               "detection_select: workspace of %zu bytes needed, %zu given", w.total, workspace_bytes);
  THIN_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, THIN_ERR_WORKSPACE,
               "detection_select: workspace must be 256-byte aligned");
  char* ws = static_cast<char*>(workspace);
  uint16_t* bits1 = reinterpret_cast<uint16_t*>(ws + w.bits1);
  int32_t* cls1 = reinterpret_cast<int32_t*>(ws + w.cls1);
  int32_t* stage1 = reinterpret_cast<int32_t*>(ws + w.stage1);
  uint16_t* gathered = agn ? nullptr : reinterpret_cast<uint16_t*>(ws + w.gathered);
  int32_t* stage2 = agn ? nullptr : reinterpret_cast<int32_t*>(ws + w.stage2);
  uint64_t* recs = w.recs_pitch ? reinterpret_cast<uint64_t*>(ws + w.recs) : nullptr;
  thin_select_trace tr;
  memset(&tr, 0, sizeof tr);
  if (trace) tr = *trace;

  Layout L{static_cast<const uint16_t*>(decoded->data), decoded->strides[0], decoded->strides[1],
           decoded->strides[2]};
  hipLaunchKernelGGL(class_max_kernel, dim3(blocks_for((uint64_t)(B * A))), dim3(kThreads), 0, stream, L, B, A, nc,
                     bits1, cls1, static_cast<uint16_t*>(tr.class_max));
  THIN_LAUNCH_CHECK("class_max");
  if (K == 0) return THIN_OK;
  thin_status s = topk(bits1, B, A, K, stage1, recs, w.recs_pitch, stream);
  if (s) return s;
  if (!agn) {
    hipLaunchKernelGGL(gather_kernel, dim3(blocks_for((uint64_t)(B * K * nc))), dim3(kThreads), 0, stream, L, B, K,
                       nc, stage1, gathered, static_cast<uint16_t*>(tr.gathered));
    THIN_LAUNCH_CHECK("gather");
    s = topk(gathered, B, K * nc, K, stage2, recs, w.recs_pitch, stream);
    if (s) return s;
  }
  PackArgs pa;
  pa.L = L;
  pa.batches = B;
  pa.K = K;
  pa.classes = nc;
  pa.agnostic = agn ? 1 : 0;
  pa.stage1 = stage1;
  pa.stage2 = stage2;
  pa.bits1 = bits1;
  pa.cls1 = cls1;
  pa.gathered = gathered;
  pa.anchors = A;
  pa.out = static_cast<uint32_t*>(out);
  pa.tr = tr;
  hipLaunchKernelGGL(pack_kernel, dim3(blocks_for((uint64_t)(B * K))), dim3(kThreads), 0, stream, pa);
  THIN_LAUNCH_CHECK("pack");
  return THIN_OK;
}
