// Shared host/device helpers of libthin_hip.so (gfx950).
//
// Host side: thread-local error text, descriptor validation, coalescing of
// dimensions shared by several operands, and magic-number division tables.
// Device side: fp16 vector types, fp32 math helpers, wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "thin_hip.h"

namespace thin {

constexpr int kMaxDims = THIN_MAX_DIMS;

// ---------------------------------------------------------------- errors
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define THIN_REQUIRE(cond, status, ...)          \
  do {                                           \
    if (!(cond)) {                               \
      ::thin::set_error(__VA_ARGS__);            \
      return (status);                           \
    }                                            \
  } while (0)

#define THIN_HIP_CHECK(call)                                                     \
  do {                                                                           \
    hipError_t thin_e_ = (call);                                                 \
    if (thin_e_ != hipSuccess) {                                                 \
      ::thin::set_error("%s failed: %s", #call, hipGetErrorString(thin_e_));     \
      return THIN_ERR_HIP;                                                       \
    }                                                                            \
  } while (0)

// Checks the launch that was just enqueued (hipGetLastError).
#define THIN_LAUNCH_CHECK(name) THIN_HIP_CHECK(hipGetLastError())

// ---------------------------------------------------------------- descriptors
int dtype_size(int32_t dtype);  // 0 for an unknown dtype
const char* dtype_name(int32_t dtype);
bool desc_valid(const thin_desc* d);  // rank/sizes/strides sane, non-null data if non-empty
int64_t numel(const thin_desc* d);
bool same_sizes(const thin_desc* a, const thin_desc* b);
bool is_contiguous(const thin_desc* d);

// Magic-number unsigned division, exact for n < 2^31 and any 1 <= d < 2^31
// (round-up multiplier method: q = umulhi(n, mul) >> shr).
struct FastDiv {
  uint32_t d;
  uint32_t mul;
  uint32_t shr;
  static FastDiv make(uint32_t divisor) {
    FastDiv f;
    f.d = divisor;
    if (divisor <= 1) {
      f.mul = 0;
      f.shr = 0;
    } else {
      uint32_t l = 32u - (uint32_t)__builtin_clz(divisor - 1u);  // ceil(log2(d))
      uint64_t p = 31u + l;
      f.mul = (uint32_t)(((1ull << p) + divisor - 1u) / divisor);
      f.shr = (uint32_t)(p - 32u);
    }
    return f;
  }
  __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    return d == 1u ? n : (__umulhi(n, mul) >> shr);
#else
    return d == 1u ? n : (uint32_t)((((uint64_t)n * mul) >> 32) >> shr);
#endif
  }
};

// Dimensions shared by up to kMaxOps operands after dropping size-1 dims and
// merging neighbours that are contiguous relative to each other in every
// operand.  dim 0 is outermost.
constexpr int kMaxOps = 4;
struct Coalesced {
  int nd;
  int64_t size[kMaxDims];
  int64_t stride[kMaxOps][kMaxDims];
};
// All descriptors must have equal sizes.  Returns the coalesced layout.
Coalesced coalesce(const thin_desc* const* ops, int nops);

// Number of workgroups for a grid-stride kernel over `units` work items with
// `threads` threads each handling `per_thread` items per iteration.
uint32_t grid_for(uint64_t units, uint32_t threads, uint32_t per_thread = 1,
                  uint32_t max_blocks = 256u * 16u);

}  // namespace thin

// ---------------------------------------------------------------- device
#if defined(__HIPCC__)
namespace thin {
namespace dev {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// NaN-propagating maximum (fmaxf would drop a NaN operand).
__device__ __forceinline__ float max_nan(float a, float b) {
  return (a > b || a != a) ? a : b;
}

// exp(-x) through the hardware exp2; the fp32 argument rounding error is far
// below one fp16 ulp, so fp16 outputs built on it stay within the fp16
// tolerance of a correctly rounded fp32 evaluation.
__device__ __forceinline__ float fast_exp_neg(float x) {
  return __builtin_amdgcn_exp2f(x * -1.4426950408889634f);
}
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// Sum / max across the 64 lanes of a wavefront (all lanes get the result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max_nan(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max_nan(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace dev
}  // namespace thin
#endif
