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

// Magic-number unsigned division, exact for n < 2^31 and any 1 <= d < 2^31,
// with no branch: q = (umulhi(n, mul) + n) >> shr, shr = ceil(log2 d),
// mul = floor(2^32 (2^shr - d) / d) + 1 (Granlund and Montgomery's round-up
// multiplier, its 33rd bit carried by the add of n; n < 2^31 keeps the sum in
// 32 bits).  d = 1 is mul = 1, shr = 0.  Being branch-free, a kernel reads all
// three fields in one round of scalar loads (a `d == 1` test put the loads of
// mul and shr behind a wait).
struct FastDiv {
  uint32_t d;
  uint32_t mul;
  uint32_t shr;
  static FastDiv make(uint32_t divisor) {
    FastDiv f;
    f.d = divisor;
    if (divisor == 0 || divisor > (1u << 31)) {  // no quotient to give (d = 0), or 0 for every n < 2^31
      f.mul = 0;
      f.shr = 31;
    } else {
      const uint32_t l = divisor == 1u ? 0u : 32u - (uint32_t)__builtin_clz(divisor - 1u);  // ceil(log2(d))
      f.mul = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << l) - divisor)) / divisor + 1u);
      f.shr = l;
    }
    return f;
  }
  __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    return (__umulhi(n, mul) + n) >> shr;
#else
    return (uint32_t)(((((uint64_t)n * mul) >> 32) + n) >> shr);
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

// Launches whose operand reaches this many bytes use non-temporal (streaming)
// loads and stores.  Measured on MI355X (affine+SiLU over NC1HWC0 fp16): with
// cold inputs streaming is 25-40% faster from 6 MB up; when a producer and a
// consumer ping-pong two buffers that stay in the caches it is equal up to
// 13 MB and faster at 26 MB.  Below a few MB the launch latency dominates.
constexpr int64_t kStreamingBytes = (int64_t)4 << 20;

// Number of workgroups for a grid-stride kernel over `units` work items with
// `threads` threads each handling `per_thread` items per iteration.
uint32_t grid_for(uint64_t units, uint32_t threads, uint32_t per_thread = 1,
                  uint32_t max_blocks = 256u * 16u);

// Reduction tree of the fp16/fp32 row softmax: `lanes` lanes share a row and
// lane g holds chunks g, g + lanes, ... (`chunks_per_lane` of them).  The row
// sum is each lane's chunks in order, then an xor butterfly over the lanes.
struct RowTree {
  int lanes, chunks_per_lane;
};
RowTree row_tree(int64_t chunks, uint64_t rows);

}  // namespace thin

// ---------------------------------------------------------------- device
#if defined(__HIPCC__)
namespace thin {
namespace dev {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// Holds v in a scalar register at this point of the kernel: a kernel
// argument passed here is loaded before the branches that follow, in the same
// round of scalar loads as the ones they test, instead of after them.
template <typename T>
__device__ __forceinline__ void scalar_here(T v) {
  __asm__ volatile("" ::"s"(v));
}

// Dispatch deals the workgroups of a launch to the 8 XCDs round robin (block
// b runs on XCD b % 8, each XCD with its own L2).  xcd_grouped<RUN>(b, nb) is
// the logical block that b runs as when each XCD is to take runs of RUN
// consecutive logical blocks (neighbours that read the same lines then share
// an L2), the 8 runs of each window of 8 * RUN logical blocks side by side
// (so that the launch still sweeps memory as one front).  Blocks past the
// last whole window keep their index; the map is a bijection on [0, nb).
template <uint32_t RUN>
__device__ __forceinline__ uint32_t xcd_grouped(uint32_t b, uint32_t nb) {
  constexpr uint32_t kSpan = 8 * RUN;
  if (b >= nb / kSpan * kSpan) return b;
  return b / kSpan * kSpan + (b & 7u) * RUN + b % kSpan / 8u;
}

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

// Sigmoid for fp16 outputs (shared by the elementwise and detect-decode
// kernels so that both produce the same bits).
__device__ __forceinline__ float sigmoid_fast(float x) { return fast_rcp(1.0f + fast_exp_neg(x)); }

// DFL expectation of V adjacent anchors: sum_i i * softmax_i(bins[i][j]) over
// the 16 bins of one box side.  The bin max only stabilises the exponentials
// (NaN-propagating packed maximum: a NaN bin, a +inf bin or an all -inf side
// makes the sum NaN either way, as the CPU softmax then expectation does).
// FAST (fp16 results): e = exp2(x*log2e - m*log2e) as one fma (an error in the
// common term scales every e_i alike and cancels in w/s) and w * 1/s;
// otherwise expf and an IEEE division.  w accumulates with fma.
template <int V, bool FAST>
__device__ __forceinline__ void dfl_side(const _Float16 (&bins)[16][V], float (&r)[V]) {
  typedef _Float16 hv __attribute__((ext_vector_type(2)));
  float m[V];
  if constexpr (V == 2) {
    hv mv = {bins[0][0], bins[0][1]};
#pragma unroll
    for (int i = 1; i < 16; ++i) mv = __builtin_elementwise_maximum(mv, (hv){bins[i][0], bins[i][1]});
    m[0] = (float)mv[0];
    m[1] = (float)mv[1];
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      m[j] = (float)bins[0][j];
#pragma unroll
      for (int i = 1; i < 16; ++i) m[j] = fmaxf(m[j], (float)bins[i][j]);
    }
  }
  constexpr float kLog2e = 1.4426950408889634f;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const float ml = m[j] * kLog2e;
    float s = 0.f, w = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float x = (float)bins[i][j];
      const float e = FAST ? __builtin_amdgcn_exp2f(__builtin_fmaf(x, kLog2e, -ml)) : expf(x - m[j]);
      s += e;
      if (i > 0) w = __builtin_fmaf(e, (float)i, w);
    }
    if (FAST) {
      // Materialise the fp32 quotient: otherwise the backend may fold the
      // later fp16 conversion into a single-rounding v_fma_mixlo_f16 in one
      // kernel and not in another, and the kernels sharing this function
      // would disagree by an ulp on halfway cases.
      float q = w * fast_rcp(s);
      __asm__ volatile("" : "+v"(q));
      r[j] = q;
    } else {
      r[j] = w / s;
    }
  }
}

// Loads the 16 bins of V adjacent anchors: bin i sits at byte offset
// off + i * stride from base.
template <int V>
__device__ __forceinline__ void dfl_load(const char* base, uint64_t off, uint64_t stride, _Float16 (&bins)[16][V]) {
  typedef _Float16 hv __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const char* ptr = base + (off + i * stride);
    if constexpr (V == 2) {
      const hv b = *reinterpret_cast<const hv*>(ptr);
      bins[i][0] = b[0];
      bins[i][1] = b[1];
    } else {
      bins[i][0] = *reinterpret_cast<const _Float16*>(ptr);
    }
  }
}

// Raw buffer resource over `bytes` bytes from base (gfx9 descriptor word 3);
// loads at offsets >= bytes return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// The same 16 bins through a buffer resource: the per-bin offset i * stride is
// uniform, so it travels as the scalar offset and a load needs no vector
// address arithmetic.  NT: non-temporal (streaming) loads.
template <int V, bool NT>
__device__ __forceinline__ void dfl_load_buffer(__amdgpu_buffer_rsrc_t rsrc, uint32_t off, uint32_t stride,
                                                _Float16 (&bins)[16][V]) {
  typedef _Float16 hv __attribute__((ext_vector_type(2)));
  constexpr int kAux = NT ? 2 : 0;  // cache-policy operand: 2 = nt
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if constexpr (V == 2) {
      const hv b = __builtin_bit_cast(hv, __builtin_amdgcn_raw_buffer_load_b32(rsrc, off, i * stride, kAux));
      bins[i][0] = b[0];
      bins[i][1] = b[1];
    } else {
      bins[i][0] = __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(rsrc, off, i * stride, kAux));
    }
  }
}

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


// fp32 -> fp16 of the fp32 value as computed.  Without the register barrier
// the compiler folds a producing fma or mul into v_fma_mixlo_f16, which
// rounds the exact result to fp16 once (and forms a product as fma(a, b, +0),
// turning -0 into +0), instead of rounding to fp32 first as the source says.
__device__ __forceinline__ _Float16 to_half(float x) {
  asm("" : "+v"(x));
  return (_Float16)x;
}

// Max / sum over the G lanes of a row group (G a power of two <= 64): an xor
// butterfly, so every lane of the group ends with the same bits.  fmaxf drops
// a NaN operand; the row softmax relies on the sum, not the max, to carry
// NaN through.
//
// Lane l ^ o is fetched by DPP for o <= 8 (quad_perm for 1 and 2, row
// rotates for 4 and 8) and by the gfx950 permlane swaps for 16 and 32: a few
// cycles per step where a ds_bpermute shuffle costs ~150.  The pairs, and so
// the bits, are those of __shfl_xor.
template <int O>
__device__ __forceinline__ uint32_t lane_xor_bits(uint32_t v) {
  const int x = (int)v;
  int r;
  if constexpr (O == 1) {
    r = __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if constexpr (O == 2) {
    r = __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else if constexpr (O == 4) {
    // lane i of a row reads lane (i - n) mod 16 under row_ror:n: row_ror:4
    // into lanes 4-7 and 12-15 (banks 1, 3), row_ror:12 into 0-3 and 8-11
    r = __builtin_amdgcn_update_dpp(x, x, 0x124, 0xF, 0xA, false);
    r = __builtin_amdgcn_update_dpp(r, x, 0x12C, 0xF, 0x5, false);
  } else if constexpr (O == 8) {
    r = __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (O == 16) {
    const auto s = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
    r = (int)((threadIdx.x & 16u) ? s[0] : s[1]);
  } else {
    static_assert(O == 32, "lane_xor: offset must be a power of two below 64");
    const auto s = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
    r = (int)((threadIdx.x & 32u) ? s[0] : s[1]);
  }
  return (uint32_t)r;
}
template <int O>
__device__ __forceinline__ float lane_xor(float v) {
  return __builtin_bit_cast(float, lane_xor_bits<O>(__builtin_bit_cast(uint32_t, v)));
}

template <int G, int O = G / 2>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (O == 0) {
    return v;
  } else {
    v = fmaxf(v, lane_xor<O>(v));
    return group_max<G, O / 2>(v);
  }
}
template <int G, int O = G / 2>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (O == 0) {
    return v;
  } else {
    v += lane_xor<O>(v);
    return group_sum<G, O / 2>(v);
  }
}

// fp16 row softmax over a row held by G lanes, KPT chunks of eight elements
// per lane (lane g holds chunks g, g + G, ...; `have[k]` says chunk k exists):
// m = max, e = exp2(x * log2e - m * log2e) as one fma, s = the lane's e in
// order then the group butterfly, out = fp16(e * (1 / s)).  Shared by the row
// softmax kernel and the fused attention kernel so both give the same bits.
template <int G, int KPT>
__device__ __forceinline__ void softmax_row_h8(const h8 (&x)[KPT], const bool (&have)[KPT], h8 (&out)[KPT]) {
  float m = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < KPT; ++k)
    if (have[k]) {
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, (float)x[k][j]);
    }
  m = group_max<G>(m);
  constexpr float kLog2e = 1.4426950408889634f;
  const float ml = m * kLog2e;
  float e[KPT][8];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < KPT; ++k)
    if (have[k]) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        e[k][j] = __builtin_amdgcn_exp2f(__builtin_fmaf((float)x[k][j], kLog2e, -ml));
        s += e[k][j];
      }
    }
  s = group_sum<G>(s);
  const float inv = 1.0f / s;
#pragma unroll
  for (int k = 0; k < KPT; ++k)
    if (have[k]) {
#pragma unroll
      for (int j = 0; j < 8; ++j) out[k][j] = to_half(e[k][j] * inv);
    }
}

}  // namespace dev
}  // namespace thin
#endif
