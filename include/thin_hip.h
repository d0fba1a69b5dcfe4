/*
 * thin_hip.h -- C ABI of the MI355X (gfx950) FP16 blocked-layout tensor library.
 *
 * Every entry point takes plain pointers, sizes and a hipStream_t; no torch
 * types cross this boundary.  Tensors are described by `thin_desc`: a data
 * pointer that already includes the storage offset, a dtype, a rank and
 * per-dimension sizes/strides counted in elements (stride 0 = broadcast).
 *
 * Rules shared by every entry point:
 *   - the library never allocates device memory and never synchronizes; work
 *     is enqueued on the given stream, so every call is safe to record into a
 *     HIP graph (hipStreamBeginCapture .. hipStreamEndCapture);
 *   - a call that cannot run returns a non-zero thin_status and leaves a
 *     message in thin_last_error() (thread-local); nothing is launched then;
 *   - calls are thread-safe; the library keeps no per-call state.
 *
 * Reference interfaces are cited as file:line of the ThinTNPU sources
 * (AscendC kernels + libtorch host code) whose behaviour each entry replaces.
 */
#ifndef THIN_HIP_H
#define THIN_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define THIN_MAX_DIMS 8
#define THIN_MAX_CAT_INPUTS 64

typedef enum thin_status {
  THIN_OK = 0,
  THIN_ERR_INVALID = 1,     /* argument / shape / dtype contract violated */
  THIN_ERR_UNSUPPORTED = 2, /* well-formed but outside what the library implements */
  THIN_ERR_HIP = 3,         /* a HIP runtime call failed (launch error etc.) */
  THIN_ERR_WORKSPACE = 4    /* caller-provided workspace too small */
} thin_status;

typedef enum thin_dtype {
  THIN_F16 = 0,
  THIN_F32 = 1,
  THIN_I64 = 2,
  THIN_I32 = 3,
  THIN_I16 = 4,
  THIN_U8 = 5,
  THIN_F64 = 6,
  THIN_BF16 = 7
} thin_dtype;

typedef struct thin_desc {
  void* data;                       /* address of element [0,...,0] */
  int32_t dtype;                    /* thin_dtype */
  int32_t rank;                     /* 0..THIN_MAX_DIMS */
  int64_t sizes[THIN_MAX_DIMS];
  int64_t strides[THIN_MAX_DIMS];   /* in elements, >= 0 */
} thin_desc;

/* Binary operation codes; the numbering follows the reference's
 * elementwise.cpp:104-115 entries (sub=0, mul=1, div=2, add=3). */
typedef enum thin_binary_op { THIN_SUB = 0, THIN_MUL = 1, THIN_DIV = 2, THIN_ADD = 3 } thin_binary_op;

typedef enum thin_unary_op { THIN_SIGMOID = 0, THIN_SILU = 1 } thin_unary_op;

/* Last error message of the calling thread ("" after a successful call). */
const char* thin_last_error(void);

/* Library version string, e.g. "thin-hip 0.1 gfx950". */
const char* thin_version(void);

/* ------------------------------------------------------------------ */
/* Elementwise                                                         */
/* ------------------------------------------------------------------ */

/* out = x op (alpha * y) for add/sub, x*y, x/y; fp16 or fp32.
 * x, y and out share out's sizes (broadcast operands carry stride 0); any
 * strides.  fp16 math runs in fp32 with one round-to-nearest-even cast, so
 * add/sub/mul/div with alpha == 1 are correctly rounded fp16 results.
 * Replaces thin_ops::binary + sub/add/mul/div (ops.cpp:464-497), the packed
 * binary_impl kernels (elementwise.cpp:6-45) and strided_binary::launch
 * (strided_binary.h:192-222). */
thin_status thin_binary(int32_t op, const thin_desc* x, const thin_desc* y,
                        const thin_desc* out, float alpha, hipStream_t stream);

/* out = x op scalar (scalar_first == 0) or scalar op x (scalar_first != 0),
 * with the scalar held at fp32 precision, as PyTorch CPU holds a wrapped
 * Python number.  Replaces the 0-d CPU operand branch of thin_ops::binary
 * (ops.cpp:466-467). */
thin_status thin_binary_scalar(int32_t op, const thin_desc* x, double scalar,
                               int32_t scalar_first, const thin_desc* out,
                               float alpha, hipStream_t stream);

/* out = sigmoid(x) or silu(x), computed in fp32, one cast; fp16 or fp32; any
 * strides (out may alias x exactly, for in-place use).
 * Replaces thin::sigmoid (backend.cpp:226-244; sigmoid.cpp:6-51),
 * thin_ops::silu_ (ops.cpp:498-512; elementwise.cpp:47-102) and
 * thin_aten::sigmoid/silu (aten_adapter.cpp:94-105). */
thin_status thin_unary(int32_t op, const thin_desc* x, const thin_desc* out,
                       hipStream_t stream);

/* Fused residual: out = y + silu(x) in fp32 with a single rounding (fp16).
 * No reference counterpart as one op: replaces the chain silu_ (ops.cpp:498)
 * followed by add.Tensor (ops.cpp:495) of the C2f Bottleneck residual. */
thin_status thin_silu_add(const thin_desc* x, const thin_desc* y,
                          const thin_desc* out, hipStream_t stream);

/* Fused per-channel affine + SiLU: out = silu(round16(round16(x*s) + b)),
 * fp16, reproducing the fp16 roundings of the unfused mul -> add -> silu
 * chain (ops.cpp:464-497 twice, then elementwise.cpp:47-102) in registers.
 * s and b carry out's sizes with broadcast strides (e.g. [1,C1,1,1,16] over
 * an NC1HWC0 x). */
thin_status thin_affine_silu(const thin_desc* x, const thin_desc* s,
                             const thin_desc* b, const thin_desc* out,
                             hipStream_t stream);

/* ------------------------------------------------------------------ */
/* Data movement (bit-exact)                                           */
/* ------------------------------------------------------------------ */

/* dst = src elementwise bit copy, equal sizes and dtype, any strides.
 * Replaces materialize::copy / gather_kernel / transpose_kernel
 * (ops.cpp:85-295) and the device-to-device leg of thin_ops::copy_strided
 * (ops.cpp:32-78). */
thin_status thin_copy(const thin_desc* src, const thin_desc* dst, hipStream_t stream);

/* out = cat(inputs, dim) with PyTorch semantics: every input has out's rank,
 * and out's sizes outside `dim`; inputs may have any strides (0-sized inputs
 * contribute nothing).  n <= THIN_MAX_CAT_INPUTS.
 * Replaces thin_ops::cat (ops.cpp:419-462) with concatenate::concat_kernel
 * (ops.cpp:309-417) and strided_concat::launch (strided_concat.h:1-247). */
thin_status thin_cat(const thin_desc* inputs, int32_t n, int32_t dim,
                     const thin_desc* out, hipStream_t stream);

/* Nearest 2x upsample of an NC1HWC0 fp16/fp32 tensor [N,C1,H,W,C0] into
 * [N,C1,2H,2W,C0] (any N; any strides on N and C1, H/W/C0 dense).
 * Replaces blocked_flow::upsample (flow_ops.cpp:129-199,233-252). */
thin_status thin_upsample2x_nc1hwc0(const thin_desc* x, const thin_desc* y,
                                    hipStream_t stream);

/* Nearest 2x upsample of NCHW [N,C,H,W] into [N,C,2H,2W] (any strides).
 * Replaces thin::upsample_nearest2d (backend.cpp:269-286; upsample.cpp:5-132). */
thin_status thin_upsample2x_nchw(const thin_desc* x, const thin_desc* y,
                                 hipStream_t stream);

/* Fused neck op: out = cat([up2x(x_i) if upsample[i] else x_i ...], dim=1) on
 * NC1HWC0 tensors, one launch.  No single reference counterpart: replaces
 * thin_native_flow::upsample (flow_ops.cpp:233-252) followed by aten::cat
 * (ops.cpp:419-462). */
thin_status thin_upsample_cat_nc1hwc0(const thin_desc* inputs, const int32_t* upsample,
                                      int32_t n, const thin_desc* out, hipStream_t stream);

/* NCHW [N,C,H,W] -> NC1HWC0 [N,ceil(C/16),H,W,16]; channels >= C are zero.
 * Replaces native_flow::pack_input (conv_flow.cpp:406-458) and
 * thin_blocked::pack (layout_blocked.h:2-55); any N. */
thin_status thin_pack_nc1hwc0(const thin_desc* x, const thin_desc* y, hipStream_t stream);

/* NC1HWC0 [N,C1,H,W,16] -> NCHW [N,C,H,W] with C <= 16*C1 (drops padding).
 * Replaces thin_blocked::unpack (layout_blocked.h:57-69); any N. */
thin_status thin_unpack_nc1hwc0(const thin_desc* x, const thin_desc* y, hipStream_t stream);

/* Stride-1 max pool, odd kernel k in [1, 15], "same" padding (taps outside
 * the plane skipped): out[n,c1,y,x,:] = max over the k x k window of x.  The
 * first maximum in row-major window order is kept (PyTorch CPU's choice for
 * +0/-0 ties); a NaN in the window gives NaN.  fp16 NC1HWC0, any N, N/C1/H
 * strides free, pixels 16-byte aligned.  Replaces blocked_flow::maxpool and
 * maxpool_tiles (flow_ops.cpp:82-127,208-231; SPPF k5). */
thin_status thin_maxpool_nc1hwc0(const thin_desc* x, int32_t kernel, const thin_desc* out, hipStream_t stream);

/* SPPF pooling and concat in one pass: out = cat([x, p(x), p(p(x)), ...], dim 1)
 * with p the max pool above (odd kernel in [1, 15]) applied `repeats` times
 * (1..8), each repeat pooling the previous one's output, so +0/-0 ties and
 * NaNs come out as from chained thin_maxpool_nc1hwc0 calls.  fp16 NC1HWC0:
 * x [N,C1,H,W,16], out [N,(repeats+1)*C1,H,W,16], strides as for the pool.
 * Replaces the SPPF block's three k5 pools (whole_blocked.py:63-64,259-262,
 * flow_ops.cpp:82-127) and the cat of their outputs (ops.cpp:419-462). */
thin_status thin_sppf_nc1hwc0(const thin_desc* x, int32_t kernel, int32_t repeats, const thin_desc* out,
                              hipStream_t stream);

/* The same pool over NCHW fp16/fp32, any strides.  Replaces thin::maxpool2d
 * (backend.cpp:245-266; maxpool.cpp:1-60, k5 s1 p2) and serves aten
 * max_pool2d_with_indices (aten_adapter.cpp:61-80). */
thin_status thin_maxpool2d_nchw(const thin_desc* x, int32_t kernel, const thin_desc* out, hipStream_t stream);

/* out[...] = value (float dtypes) or ivalue (integer dtypes), any strides.
 * Replaces the device side of aten fill_.Scalar / zero_ (decode.cpp:29-34)
 * and the zero placeholder indices of max_pool2d_with_indices
 * (aten_adapter.cpp:71-78); a kernel, so safe inside graph capture. */
thin_status thin_fill(const thin_desc* out, double value, int64_t ivalue, hipStream_t stream);

/* ------------------------------------------------------------------ */
/* Reductions                                                          */
/* ------------------------------------------------------------------ */

/* out = softmax(x, dim): fp32 max / exp / sum, out = e * (1/sum) (last dim)
 * or e / sum (other dims); NaN/inf follow PyTorch CPU.  x fp16 or fp32, out
 * fp16/fp32 (fp16 -> fp32 = half_to_float).  x any strides; out any strides.
 * Replaces thin_softmax::softmax (softmax_host.cpp:51-89), Softmax<T,U,Last>
 * (softmax.cpp:6-173) and the DFL fast path DflSoftmax (softmax.cpp:175-271;
 * softmax_host.cpp:29-50). */
thin_status thin_softmax(const thin_desc* x, int32_t dim, const thin_desc* out,
                         hipStream_t stream);

/* Fused DFL: x = box logits [N,4*16,A] (fp16, any strides, bins of side s at
 * channels 16s..16s+15) -> out [N,4,A] (fp16 or fp32) where
 * out[n,s,a] = sum_i i * softmax_i(x[n,16s+i,a]).  fp32 throughout, one cast.
 * Replaces DflSoftmax (softmax.cpp:175-271) followed by the 1x1 arange(16)
 * convolution of the DFL head (model_optimization.py:20-31,
 * conv_img.cpp:590-597). */
thin_status thin_dfl_expect(const thin_desc* x, const thin_desc* out, hipStream_t stream);

/* ------------------------------------------------------------------ */
/* Detection selection (YOLO26 NMS-free top-K)                         */
/* ------------------------------------------------------------------ */

/* Optional trace outputs; any pointer may be NULL.  Sizes follow
 * SELECTION_FLOW.md's stage list: class_max fp16 [B,A], stage1 int64 [B,K],
 * gathered fp16 [B,K,nc] (class-aware only), top_values fp16 [B,K],
 * stage2 int64 [B,K] (class-aware only), anchors int64 [B,K],
 * labels int64 [B,K]; all contiguous. */
typedef struct thin_select_trace {
  void* class_max;
  void* stage1;
  void* gathered;
  void* top_values;
  void* stage2;
  void* anchors;
  void* labels;
} thin_select_trace;

/* Anchor-free detect-head decode in one launch: the DFL expectation of
 * boxes [B,64,A] (bit-identical to thin_dfl_expect with fp16 output), or
 * boxes [B,4,A] taken as the distances themselves (reg_max = 1 heads such as
 * YOLO26's, whose module.dfl is the identity), the
 * distances applied to the per-level grid cell centres (x + 0.5, y + 0.5) as
 * lower = centre - d[0:2], upper = centre + d[2:4], scaled by the level stride
 * as xyxy (lower, upper) or xywh ((lower+upper)/2, upper-lower), each step one
 * correctly rounded fp16 operation; then sigmoid(scores [B,nc,A])
 * (bit-identical to thin_unary SIGMOID).  out [B,4+nc,A] fp16 is the
 * detection-selection input.  level_hw holds `levels` (h, w) pairs in anchor
 * order (sum h*w = A), level_stride their strides (rounded to fp16).  Replaces
 * the decode chain of anchorfree_predictions (whole_blocked.py:118-146;
 * YOLO26.md:30-38). */
thin_status thin_detect_decode(const thin_desc* boxes, const thin_desc* scores, const int32_t* level_hw,
                               const double* level_stride, int32_t levels, int32_t xywh, const thin_desc* out,
                               hipStream_t stream);

/* Bytes of device workspace thin_detection_select needs for these sizes.
 * Replaces the intermediate tensors the reference allocates per call
 * (selection_flow.cpp:445-466: maxima, gathered, indices, values, records). */
size_t thin_detection_select_workspace(int64_t batches, int64_t anchors, int64_t classes,
                                       int64_t max_det, int32_t agnostic);

/* decoded: fp16 [B,A,4+nc], any non-negative strides.  out: fp32 [B,K,6]
 * contiguous, K = min(max_det, A); rows (box0..3, score, class).  Order:
 * ascending (score_key(bits), index) -- NaN first, +-0 equal, lower index
 * wins ties; class max keeps the first best class.  Bit-exact by contract.
 * workspace: >= thin_detection_select_workspace(...) bytes, 256-B aligned.
 * Replaces detection_selection::run / detection_select /
 * detection_select_trace (selection_flow.cpp:429-499). */
thin_status thin_detection_select(const thin_desc* decoded, int64_t max_det, int32_t agnostic,
                                  void* out, void* workspace, size_t workspace_bytes,
                                  const thin_select_trace* trace, hipStream_t stream);

/* Capacity of the static device scratch behind thin_detection_select_noalloc
 * (8 MiB per GPU the library runs on, held until the process ends; the C5
 * shape [1,8400,84] with K = 300 needs about 100 KB per image). */
#define THIN_SELECT_SCRATCH_BYTES (8u << 20)

/* thin_detection_select without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference: the
 * reference allocates its intermediates per call.  Same arguments, results
 * and errors as thin_detection_select; the intermediates live in a static
 * device array of the library, one per GPU, whose device address is taken
 * once per device on the first call with that device current.  Calls whose
 * thin_detection_select_workspace(...) exceeds THIN_SELECT_SCRATCH_BYTES fail
 * with THIN_ERR_WORKSPACE.  Allocates nothing (no hipMalloc, hipFree or
 * allocating library call).  Every call on one GPU shares that GPU's scratch:
 * calls that overlap on one GPU (two streams, or two host threads) race and
 * must be ordered by the caller. */
thin_status thin_detection_select_noalloc(const thin_desc* decoded, int64_t max_det, int32_t agnostic,
                                          void* out, const thin_select_trace* trace, hipStream_t stream);

/* ------------------------------------------------------------------ */
/* Attention contractions                                              */
/* ------------------------------------------------------------------ */

/* Operand interpretation of thin_layout_bmm, the arguments of the reference's
 * layout_bmm after its two tensors (bmm_flow.cpp:276-278,347).  An operand is
 * a rank-3 [batch, rows, cols] tensor or a channel-blocked rank-4
 * [N, C1, T, 16] tensor whose logical matrix has the C1*16 channels as rows
 * and the T tokens as columns.  groups > 0 splits the channels of an N=1
 * blocked operand into `groups` heads (the batch); a/b_offset and
 * a/b_channels select a channel (row) range inside each head, -1 = to the end.
 * transpose_a/b transpose the logical matrices; blocked_output packs the
 * [batch, m, n] result as NC1HWC0 [batch, m/16, n, 16], or [1, batch*m/16, n,
 * 16] when groups > 0. */
typedef struct thin_bmm_layout {
  int32_t transpose_a;
  int32_t transpose_b;
  int32_t blocked_output;
  int32_t reserved;
  int64_t groups;
  int64_t a_offset;
  int64_t a_channels;
  int64_t b_offset;
  int64_t b_channels;
} thin_bmm_layout;

/* Validates a layout_bmm call and writes the output's rank and sizes:
 * [batch, m, n] (the reference allocates n rounded up to 16 columns and
 * returns the [.., :n] view), or the blocked shape.  Same checks and messages
 * as dynamic_bmm::run (bmm_flow.cpp:279-312). */
thin_status thin_layout_bmm_shape(const thin_desc* a, const thin_desc* b, const thin_bmm_layout* layout,
                                  int32_t* out_rank, int64_t* out_sizes);

/* out = a @ b over the logical fp16 matrices described above; out any
 * strides, of the shape thin_layout_bmm_shape gives.  Each output is the fp32
 * sum of its products in reduction order k = 0..K-1 from zero, cast once to
 * fp16 (round to nearest even): bit-equal to the reference's sequential
 * accumulation.  Replaces dynamic_bmm::multiply and pack_channels
 * (bmm_flow.cpp:35-191) behind layout_bmm / bmm / aten::bmm
 * (bmm_flow.cpp:276-359). */
thin_status thin_layout_bmm(const thin_desc* a, const thin_desc* b, const thin_bmm_layout* layout,
                            const thin_desc* out, hipStream_t stream);

/* Output sizes [1, groups*count/16, T, 16] of thin_channel_select, after its
 * checks (bmm_flow.cpp:255-262). */
thin_status thin_channel_select_shape(const thin_desc* x, int64_t groups, int64_t begin, int64_t count,
                                      int64_t* out_sizes);

/* x: fp16 [1, C1, T, 16] (any strides).  Output channel c is input channel
 * (c / count) * (C1*16 / groups) + begin + c % count: channels
 * [begin, begin + count) of every one of the `groups` equal channel groups,
 * packed back to back.  Bit copy.  Replaces channel_select /
 * channel_select_kernel (bmm_flow.cpp:217-266). */
thin_status thin_channel_select(const thin_desc* x, int64_t groups, int64_t begin, int64_t count,
                                const thin_desc* out, hipStream_t stream);

/* Fused blocked attention of one C2PSA block, from the head-grouped QKV
 * tensor to the mixed values, in one launch.  It has no single counterpart in
 * the reference: it replaces the chain that attention_forward runs
 * (whole_blocked.py:91-103) through channel_select, the scalar mul,
 * layout_bmm (bmm_flow.cpp:35-191), the row softmax (softmax.cpp:6-173) and
 * layout_bmm again, and returns that chain's bits:
 *   prescale != 0:  s = layout_bmm(channel_select(qkv, heads, 0, key_dim) * scale,
 *                                  qkv, T, F, F, heads, 0, key_dim, key_dim, key_dim)
 *   prescale == 0:  s = layout_bmm(qkv, qkv, T, F, F, heads, 0, key_dim, key_dim, key_dim) * scale
 *   out = layout_bmm(qkv, softmax(s, -1), F, T, T, heads, 2 * key_dim, head_dim)
 * qkv: fp16 [1, C1, T, 16] with heads equal channel groups (q, k, v at
 * offsets 0, key_dim, 2 * key_dim of each); out: fp16 [1, heads * head_dim /
 * 16, T, 16].  `scale` multiplies in fp32 as the chain's mul does (pass the
 * fp16-rounded scalar for the reference's 0-d operand rule).  Covered: packed
 * 16-channel blocks (token stride 16) with a 16-byte aligned qkv, key_dim 16,
 * 32 or 64, head_dim a multiple of 16 up to 128, T a multiple of 8 in (128,
 * 512] with T * head_dim * 2 bytes of v fitting the kernel's LDS; other
 * shapes return THIN_ERR_UNSUPPORTED (run the chain op by op). */
thin_status thin_attention(const thin_desc* qkv, int64_t heads, int64_t key_dim, int64_t head_dim, float scale,
                           int32_t prescale, const thin_desc* out, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* THIN_HIP_H */
