// Elementwise kernels: binary (add/sub/mul/div with alpha), scalar binary,
// sigmoid, SiLU, the fused silu_add / affine_silu chains and strided bit
// copies.  One grid-stride kernel family serves all of them:
//
//   * dimensions of all operands are coalesced on the host (dim 0 innermost
//     in the kernel plan) and passed by value -- no metadata upload;
//   * when the innermost coalesced dimension is a multiple of the vector
//     width V (16 bytes of elements), each thread handles V consecutive
//     outputs; every operand then loads in one of three modes, chosen per
//     operand on the host: 16-byte vector (stride 1, aligned), broadcast
//     (stride 0: one scalar load) or gather (V strided scalar loads);
//   * otherwise a one-element-per-thread path handles any layout.
//
// Arithmetic for fp16 tensors runs in fp32 and rounds once to nearest-even;
// see the per-op notes for the reference behaviour each one matches.
#include "common.h"

#include <string.h>

#include <type_traits>

namespace thin {
namespace {

using dev::fast_exp_neg;
using dev::fast_rcp;

constexpr uint32_t kThreads = 256;

enum LoadMode : uint32_t { kVec = 0, kBcast = 1, kGather = 2 };

// Offsets are 32-bit: the host splits a launch into slabs whose element
// spans fit in int32 for every operand.
template <int NIN>
struct MapPlan {
  int32_t nd;                       // coalesced dims, index 0 innermost
  uint32_t size[kMaxDims];
  FastDiv div[kMaxDims];
  int32_t ostride[kMaxDims];
  int32_t istride[NIN][kMaxDims];
  void* out;
  const void* in[NIN];
  uint32_t units;                   // vectors (V > 1) or elements (V == 1)
  uint32_t in_mode[NIN];            // LoadMode per input (V > 1 only)
  uint32_t out_mode;                // kVec or kGather (V > 1 only)
  float pa, pb;                     // op parameters (alpha, scalar)
};

// ------------------------------------------------------------ op functors
// Each functor maps NIN storage values of type T to one T.

template <typename T> __device__ __forceinline__ float to_f(T v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f(float v) { return (T)v; }

// Sigmoid / SiLU.  fp16: fp32 evaluation through the hardware exp2 and
// reciprocal (a few fp32 ulps, far below one fp16 ulp); fp32: library expf and
// IEEE division, as PyTorch CPU's 1/(1+exp(-x)) and x/(1+exp(-x))
// (sigmoid.cpp:30-36 and elementwise.cpp:76-86 compute the same formulas).
template <typename T> __device__ __forceinline__ float sigmoid_f(float x);
template <> __device__ __forceinline__ float sigmoid_f<_Float16>(float x) {
  return dev::sigmoid_fast(x);
}
template <> __device__ __forceinline__ float sigmoid_f<float>(float x) {
  return 1.0f / (1.0f + expf(-x));
}
template <typename T> __device__ __forceinline__ float silu_f(float x);
template <> __device__ __forceinline__ float silu_f<_Float16>(float x) {
  return x * fast_rcp(1.0f + fast_exp_neg(x));
}
template <> __device__ __forceinline__ float silu_f<float>(float x) {
  return x / (1.0f + expf(-x));
}

struct OpCopy {
  template <typename T, int NIN>
  __device__ __forceinline__ T operator()(const T (&v)[NIN], float, float) const { return v[0]; }
};
// x + alpha*y as one fp32 fused multiply-add: with alpha == 1 this is the
// correctly rounded sum, and fp32 -> fp16 double rounding is innocuous for
// fp16 operands (24 >= 2*11 + 2).
struct OpAdd {
  template <typename T, int NIN>
  __device__ __forceinline__ T operator()(const T (&v)[NIN], float alpha, float) const {
    return from_f<T>(fmaf(alpha, to_f(v[1]), to_f(v[0])));
  }
};
struct OpSub {
  template <typename T, int NIN>
  __device__ __forceinline__ T operator()(const T (&v)[NIN], float alpha, float) const {
    return from_f<T>(fmaf(-alpha, to_f(v[1]), to_f(v[0])));
  }
};
struct OpMul {
  template <typename T, int NIN>
  __device__ __forceinline__ T operator()(const T (&v)[NIN], float, float) const {
    return from_f<T>(to_f(v[0]) * to_f(v[1]));
  }
};
struct OpDiv {  // IEEE fp32 division (hipcc's default correctly rounded divide)
  template <typename T, int NIN>
  __device__ __forceinline__ T operator()(const T (&v)[NIN], float, float) const {
    return from_f<T>(to_f(v[0]) / to_f(v[1]));
  }
};
// Tensor (op) fp32 scalar; `pb` holds the scalar.  SUB/ADD use alpha on the
// scalar operand exactly as the Tensor-Tensor forms do.
template <int OP, bool SCALAR_FIRST>
struct OpScalar {
  template <typename T, int NIN>
  __device__ __forceinline__ T operator()(const T (&v)[NIN], float alpha, float s) const {
    float x = to_f(v[0]);
    float a = SCALAR_FIRST ? s : x;
    float b = SCALAR_FIRST ? x : s;
    float r;
    if (OP == THIN_ADD) r = fmaf(alpha, b, a);
    else if (OP == THIN_SUB) r = fmaf(-alpha, b, a);
    else if (OP == THIN_MUL) r = a * b;
    else r = a / b;
    return from_f<T>(r);
  }
};
struct OpSigmoid {
  template <typename T, int NIN>
  __device__ __forceinline__ T operator()(const T (&v)[NIN], float, float) const {
    return from_f<T>(sigmoid_f<T>(to_f(v[0])));
  }
};
struct OpSilu {
  template <typename T, int NIN>
  __device__ __forceinline__ T operator()(const T (&v)[NIN], float, float) const {
    return from_f<T>(silu_f<T>(to_f(v[0])));
  }
};
// x / (1 + exp(-x)) in fp32 for an fp16 x, to the accuracy of the library expf
// and an IEEE division, in about half their instructions:
//   * exp(-x) = 2^n * 2^f.  t = x * -log2(e)_hi is exact (13 significant bits
//     of log2(e) times the 11 of x), n = rint(t), f = (t - n) - x * log2(e)_lo
//     (one rounding; |f| <= 0.51 wherever e is finite), 2^f by the hardware
//     exp2, scaled by ldexp.
//     x is first clamped to [-65504, 64]: exp(-64) already leaves 1 + e == 1,
//     a NaN clamps to a number (the NaN comes back through x below), and n
//     stays finite.
//   * x / d, d = 1 + e: q0 = x * rcp(d), one Newton step q0 + rcp(d)(x - q0 d)
//     (the residual exact through fma), then v_div_fixup_f32 for the special
//     operands: d = inf gives a zero of x's sign (x <= -88.7, as x / inf), or
//     NaN for x = -inf; x = +inf gives +inf; a NaN x stays NaN.
__device__ __forceinline__ float silu_f16_accurate(float x) {
  constexpr float kL2eHi = 1.442626953125f;       // log2(e) truncated to 13 significant bits
  constexpr float kL2eLo = 6.8087763963387e-05f;  // log2(e) - kL2eHi
  const float xe = fmaxf(fminf(x, 64.0f), -65504.0f);
  const float t = xe * -kL2eHi;
  const float n = __builtin_rintf(t);
  const float e = __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f(__builtin_fmaf(xe, -kL2eLo, t - n)), (int)n);
  const float d = 1.0f + e;
  const float r = __builtin_amdgcn_rcpf(d);
  const float q0 = x * r;
  return __builtin_amdgcn_div_fixupf(__builtin_fmaf(__builtin_fmaf(-q0, d, x), r, q0), d, x);
}

// y + silu(x), one rounding.  The residual add can cancel (y ~ -silu(x)), which
// magnifies any fp32 error of silu(x) relative to the small result, so silu
// is evaluated to the accuracy class of PyTorch CPU's fp32 x / (1 + exp(-x)):
// library expf and IEEE division for fp32 tensors, silu_f16_accurate (the
// same steps, specialised to an fp16 operand) for fp16 ones.
struct OpSiluAdd {
  template <typename T, int NIN>
  __device__ __forceinline__ T operator()(const T (&v)[NIN], float, float) const {
    const float x = to_f(v[0]);
    if constexpr (std::is_same<T, _Float16>::value) return from_f<T>(to_f(v[1]) + silu_f16_accurate(x));
    else return from_f<T>(to_f(v[1]) + x / (1.0f + expf(-x)));
  }
};
// silu(round(round(x*s) + b)): the fp16 roundings of the unfused chain.
struct OpAffineSilu {
  template <typename T, int NIN>
  __device__ __forceinline__ T operator()(const T (&v)[NIN], float, float) const {
    T t1 = from_f<T>(to_f(v[0]) * to_f(v[1]));
    T t2 = from_f<T>(to_f(t1) + to_f(v[2]));
    return from_f<T>(silu_f<T>(to_f(t2)));
  }
};

// ------------------------------------------------------------ kernels

template <typename T, int V>
struct alignas(16) VecT {
  T v[V];
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte store; NT selects a streaming (non-temporal) store for outputs too
// large to stay cache-resident for their consumer.  Measured on gfx950 over a
// 1 GB rotation (Infinity Cache defeated), a 52 MB copy moves 5.5 TB/s with
// cached loads and stores, 5.5-5.7 with streaming stores and 5.7-6.0 with
// streaming loads and stores.
template <bool NT, typename W>
__device__ __forceinline__ void store16(void* dst, const W& w) {
  static_assert(sizeof(W) == 16, "16-byte store");
  u32x4 bits = __builtin_bit_cast(u32x4, w);
  if (NT) __builtin_nontemporal_store(bits, reinterpret_cast<u32x4*>(dst));
  else *reinterpret_cast<u32x4*>(dst) = bits;
}

template <bool NT, typename W>
__device__ __forceinline__ W load16(const void* src) {
  static_assert(sizeof(W) == 16, "16-byte load");
  u32x4 bits = NT ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src))
                  : *reinterpret_cast<const u32x4*>(src);
  return __builtin_bit_cast(W, bits);
}

// Outputs of at least kStreamingBytes are written with streaming
// (non-temporal) stores, and inputs read once in full at that size are read
// with streaming loads.  Operands re-read across the grid (broadcast
// scale/bias) always use cached loads.  On gfx950, 256-thread blocks with two
// 16-byte vectors per thread and one tile per block measured best for every
// kernel here (1024-thread blocks and 4-8 vectors per thread were slower).

// Unit offsets for the vector kernel; ND == 1 means every operand is flat
// (one coalesced dim), so the unit index is the element offset times stride.
template <int NIN, int ND>
__device__ __forceinline__ void unit_offsets(const MapPlan<NIN>& p, uint32_t e, int32_t& oo,
                                             int32_t (&io)[NIN]) {
  oo = 0;
#pragma unroll
  for (int k = 0; k < NIN; ++k) io[k] = 0;
  if (ND == 1) {
    oo = (int32_t)e * p.ostride[0];
#pragma unroll
    for (int k = 0; k < NIN; ++k) io[k] = (int32_t)e * p.istride[k][0];
    return;
  }
#pragma unroll
  for (int d = 0; d < ND; ++d) {
    if (d >= p.nd) break;
    uint32_t q = p.div[d].div(e);
    int32_t c = (int32_t)(e - q * p.size[d]);
    e = q;
    oo += c * p.ostride[d];
#pragma unroll
    for (int k = 0; k < NIN; ++k) io[k] += c * p.istride[k][d];
  }
}

// Each block handles tiles of kThreads*U units; lane t of the block takes
// units tile + u*kThreads + t, so every load/store instruction of a wave
// covers 64 consecutive 16-byte vectors when the operand is dense.  All U
// loads are issued before any math to keep several vectors in flight.
template <typename T, int V, int NIN, int ND, int U, bool NT, class Op, uint32_t BS>
__global__ __launch_bounds__(BS) void map_vec_kernel(MapPlan<NIN> p) {
  const uint32_t tile_units = BS * U;
  for (uint32_t tile = blockIdx.x * tile_units; tile < p.units; tile += gridDim.x * tile_units) {
    // raw 16-byte vectors only: unpacking is deferred to the compute phase so
    // that U * NIN vectors in flight cost 4 VGPRs each
    VecT<T, V> raw[U][NIN];
    int32_t oo[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t unit = tile + u * BS + threadIdx.x;
      if (unit >= p.units) break;
      int32_t io[NIN];
      unit_offsets<NIN, ND>(p, unit * (uint32_t)V, oo[u], io);
#pragma unroll
      for (int k = 0; k < NIN; ++k) {
        const T* src = static_cast<const T*>(p.in[k]) + io[k];
        if (p.in_mode[k] == kVec) {
          raw[u][k] = load16<false, VecT<T, V>>(src);
        } else if (p.in_mode[k] == kBcast) {
          const T sv = *src;
#pragma unroll
          for (int j = 0; j < V; ++j) raw[u][k].v[j] = sv;
        } else {
          const int32_t st = p.istride[k][0];
#pragma unroll
          for (int j = 0; j < V; ++j) raw[u][k].v[j] = src[j * st];
        }
      }
    }
    const Op op;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t unit = tile + u * BS + threadIdx.x;
      if (unit >= p.units) break;
      if constexpr (std::is_same<Op, OpCopy>::value) {
        // bit copy: move the 16-byte word as is
        T* dst = static_cast<T*>(p.out) + oo[u];
        if (p.out_mode == kVec) {
          store16<NT>(dst, raw[u][0]);
        } else {
          const int32_t st = p.ostride[0];
#pragma unroll
          for (int j = 0; j < V; ++j) dst[j * st] = raw[u][0].v[j];
        }
        continue;
      }
      VecT<T, V> r;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        T lane[NIN];
#pragma unroll
        for (int k = 0; k < NIN; ++k) lane[k] = raw[u][k].v[j];
        r.v[j] = op.template operator()<T, NIN>(lane, p.pa, p.pb);
      }
      T* dst = static_cast<T*>(p.out) + oo[u];
      if (p.out_mode == kVec) {
        store16<NT>(dst, r);
      } else {
        const int32_t st = p.ostride[0];
#pragma unroll
        for (int j = 0; j < V; ++j) dst[j * st] = r.v[j];
      }
    }
  }
}

// Two coalesced dims with every operand contiguous along the inner one (rows
// of equal length, each operand with its own row stride: channel slices of
// NC1HWC0 tensors, narrowed halves): one division per vector and no
// per-operand load modes, one tile of kThreads * U vectors per block.  NTL,
// NT: streaming loads, stores.  Against map_vec_kernel on the narrowed
// [32,4,80,80,16] half of [32,8,80,80,16]: SiLU into a dense tensor 11.6 ->
// 10.5 us, a + b of two halves 11.8 -> 10.6 us.
template <typename T, int V, int NIN, int U, bool NTL, bool NT, class Op>
__global__ __launch_bounds__(kThreads) void map_rows_kernel(MapPlan<NIN> p) {
  const uint32_t tile = blockIdx.x * (kThreads * U);
  const FastDiv& rows = p.div[0];  // vectors per row: size[0] / V
  // the plan fields the loads need, in registers before the bounds test: one
  // round of scalar loads (one asm statement: each is a scheduling boundary)
  if constexpr (NIN == 1)
    __asm__ volatile("" ::"s"(p.out), "s"(p.in[0]), "s"(rows.d), "s"(rows.mul), "s"(rows.shr), "s"(p.ostride[1]),
                     "s"(p.istride[0][1]), "s"(p.units));
  else if constexpr (NIN == 2)
    __asm__ volatile("" ::"s"(p.out), "s"(p.in[0]), "s"(p.in[1]), "s"(rows.d), "s"(rows.mul), "s"(rows.shr),
                     "s"(p.ostride[1]), "s"(p.istride[0][1]), "s"(p.istride[1][1]), "s"(p.units));
  else {
    dev::scalar_here(p.out);
#pragma unroll
    for (int k = 0; k < NIN; ++k) dev::scalar_here(p.in[k]);
  }
  VecT<T, V> raw[U][NIN];
  int32_t oo[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    // clamped, not predicated, as in map_dense_kernel
    const uint32_t unit = min(tile + u * kThreads + threadIdx.x, p.units - 1);
    const uint32_t r = rows.div(unit);
    const int32_t c = (int32_t)((unit - r * rows.d) * V);  // row strides may be negative
    oo[u] = (int32_t)r * p.ostride[1] + c;
#pragma unroll
    for (int k = 0; k < NIN; ++k)
      raw[u][k] = load16<NTL, VecT<T, V>>(static_cast<const T*>(p.in[k]) + ((int32_t)r * p.istride[k][1] + c));
  }
  const Op op;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t unit = tile + u * kThreads + threadIdx.x;
    if (unit >= p.units) break;
    T* dst = static_cast<T*>(p.out) + oo[u];
    if constexpr (std::is_same<Op, OpCopy>::value) {
      store16<NT>(dst, raw[u][0]);
    } else {
      VecT<T, V> r;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        T lane[NIN];
#pragma unroll
        for (int k = 0; k < NIN; ++k) lane[k] = raw[u][k].v[j];
        r.v[j] = op.template operator()<T, NIN>(lane, p.pa, p.pb);
      }
      store16<NT>(dst, r);
    }
  }
}

template <typename T, int NIN, int ND, class Op>
__global__ __launch_bounds__(kThreads) void map_scalar_kernel(MapPlan<NIN> p) {
  const uint32_t step = gridDim.x * kThreads;
  for (uint32_t u = blockIdx.x * kThreads + threadIdx.x; u < p.units; u += step) {
    int32_t oo;
    int32_t io[NIN];
    unit_offsets<NIN, ND>(p, u, oo, io);
    T lane[NIN];
#pragma unroll
    for (int k = 0; k < NIN; ++k) lane[k] = static_cast<const T*>(p.in[k])[io[k]];
    const Op op;
    static_cast<T*>(p.out)[oo] = op.template operator()<T, NIN>(lane, p.pa, p.pb);
  }
}

// Dense form: every operand is one contiguous run (one coalesced dim, unit
// stride), so unit u lives at element u * V of each operand.  One tile of
// kThreads * U vectors per block and no per-operand load-mode branches; NT
// streams both the loads and the stores.  The cache policy is a template
// parameter so that the compiler emits the non-temporal forms.
template <typename T, int V, int NIN, int U, bool NT, class Op>
__global__ __launch_bounds__(kThreads) void map_dense_kernel(MapPlan<NIN> p) {
  const uint32_t tile = blockIdx.x * (kThreads * U);
  // The operand pointers in registers before any bounds test, and loads
  // clamped to the last unit instead of predicated: the plan's scalar loads
  // go out in one round (a test on p.units first made the pointer loads wait
  // for it).  Stores stay predicated.
  dev::scalar_here(p.out);
#pragma unroll
  for (int k = 0; k < NIN; ++k) dev::scalar_here(p.in[k]);
  VecT<T, V> raw[U][NIN];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t unit = min(tile + u * kThreads + threadIdx.x, p.units - 1);
#pragma unroll
    for (int k = 0; k < NIN; ++k)
      raw[u][k] = load16<NT, VecT<T, V>>(static_cast<const T*>(p.in[k]) + (size_t)unit * V);
  }
  const Op op;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t unit = tile + u * kThreads + threadIdx.x;
    if (unit >= p.units) break;
    T* dst = static_cast<T*>(p.out) + (size_t)unit * V;
    if constexpr (std::is_same<Op, OpCopy>::value) {
      store16<NT>(dst, raw[u][0]);
    } else {
      VecT<T, V> r;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        T lane[NIN];
#pragma unroll
        for (int k = 0; k < NIN; ++k) lane[k] = raw[u][k].v[j];
        r.v[j] = op.template operator()<T, NIN>(lane, p.pa, p.pb);
      }
      store16<NT>(dst, r);
    }
  }
}

// ------------------------------------------------------------ NC1HWC0 affine

// Per-channel affine + SiLU on NC1HWC0 fp16 planes.  A plane (n, c1) is H*W*16
// contiguous halves; its 16 scale and 16 bias values are fixed for the whole
// plane, so each thread keeps the 8 it needs (its C0 half) in registers and
// the loop body has no index arithmetic beyond one add.  x*s and +b run as
// packed fp16 multiplies/adds (each correctly rounded, as the unfused fp16
// chain rounds them); SiLU runs in fp32 and rounds once.
struct AffinePlan {
  const _Float16* x;
  const _Float16* s;
  const _Float16* b;
  _Float16* out;
  int64_t x_n, x_c1, o_n, o_c1, s_n, s_c1, b_n, b_c1;  // element strides
  uint32_t c1;          // planes per image
  uint32_t planes;      // N * C1
  uint32_t plane_vecs;  // H * W * 2 (16-byte vectors per plane)
};

typedef _Float16 h8v __attribute__((ext_vector_type(8)));

template <int U, bool NT>
__global__ __launch_bounds__(kThreads) void affine_silu_blocked_kernel(AffinePlan p) {
  const uint32_t half = threadIdx.x & 1u;  // C0 lanes 0-7 or 8-15
  for (uint32_t plane = blockIdx.y; plane < p.planes; plane += gridDim.y) {
    const uint32_t n = plane / p.c1;
    const uint32_t c1 = plane - n * p.c1;
    const _Float16* xp = p.x + n * p.x_n + c1 * p.x_c1;
    _Float16* op = p.out + n * p.o_n + c1 * p.o_c1;
    const h8v sv = *reinterpret_cast<const h8v*>(p.s + n * p.s_n + c1 * p.s_c1 + half * 8);
    const h8v bv = *reinterpret_cast<const h8v*>(p.b + n * p.b_n + c1 * p.b_c1 + half * 8);
    for (uint32_t tile = blockIdx.x * kThreads * U; tile < p.plane_vecs;
         tile += gridDim.x * kThreads * U) {
      // every load issued (clamped into the plane) before the first is used
      h8v xv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t v = min(tile + u * kThreads + threadIdx.x, p.plane_vecs - 1);
        xv[u] = *reinterpret_cast<const h8v*>(xp + (size_t)v * 8);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t v = tile + u * kThreads + threadIdx.x;
        if (v >= p.plane_vecs) break;
        h8v t = xv[u] * sv;  // packed fp16, correctly rounded
        t = t + bv;
        h8v r;
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = (_Float16)silu_f<_Float16>((float)t[j]);
        store16<NT>(op + (size_t)v * 8, r);
      }
    }
  }
}

// Flat form of the same op for the common layout: within one image the C1
// planes of x and of out are contiguous (full tensors and C2f channel slices
// x[:, a:b]), and scale/bias do not vary with n.  The work is then rows (images)
// x one contiguous span of C1 * H * W * 2 vectors, split into one tile of
// kThreads * 2 vectors per block with no per-plane loop; the channel of a
// vector is its span offset / plane size and its C0 half the offset's parity.
// The image's 2 * C1 scale and bias vectors are staged once per block in LDS.
constexpr uint32_t kFlatMaxC1 = 128;

struct AffineFlatPlan {
  const h8v* x;
  h8v* out;
  const h8v* s;      // channel 0, C0 lanes 0-7; lanes 8-15 follow
  const h8v* b;
  uint32_t total;    // rows * span vectors
  FastDiv span;      // vectors per row
  FastDiv plane;     // vectors per (n, c1) plane
  uint32_t x_row, o_row;  // row strides in vectors
  uint32_t s_c1, b_c1;    // channel strides in vectors
  uint32_t c1;            // channel blocks per row
};

template <int U, bool NTL, bool NTS>
__global__ __launch_bounds__(kThreads) void affine_silu_flat_kernel(AffineFlatPlan p) {
  __shared__ h8v sb[2][2 * kFlatMaxC1];
  const uint32_t tile = blockIdx.x * (kThreads * U);
  h8v v[U];
  uint32_t oo[U], q[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t i = tile + u * kThreads + threadIdx.x;
    if (i < p.total) {
      const uint32_t row = p.span.div(i);
      const uint32_t col = i - row * p.span.d;
      oo[u] = row * p.o_row + col;
      q[u] = p.plane.div(col) * 2 + (col & 1u);
      const h8v* src = p.x + row * p.x_row + col;
      v[u] = NTL ? __builtin_nontemporal_load(src) : *src;
    }
  }
  // Scale/bias staging goes after the x loads are issued: its loads and the
  // barrier then overlap the x round trip instead of preceding it (one round
  // trip less per block; 6.35 -> 5.7 us for [32,512,20,20]).
  for (uint32_t i = threadIdx.x; i < 2 * p.c1; i += kThreads) {
    sb[0][i] = p.s[(i >> 1) * p.s_c1 + (i & 1u)];
    sb[1][i] = p.b[(i >> 1) * p.b_c1 + (i & 1u)];
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t i = tile + u * kThreads + threadIdx.x;
    if (i >= p.total) break;
    h8v t = v[u] * sb[0][q[u]];  // packed fp16, correctly rounded
    t = t + sb[1][q[u]];
    h8v r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (_Float16)silu_f<_Float16>((float)t[j]);
    store16<NTS>(p.out + oo[u], r);
  }
}

// Geometry of the flat form: x and out NC1HWC0 fp16 with dense planes, the
// C1 planes of an image contiguous, per-channel operands fixed along N.
struct FlatGeom {
  uint32_t total, span, plane_vecs, x_row, o_row, c1;
  uint32_t grid2, grid1;  // blocks for two / one vector per thread
  bool nt;
};

bool nc1hwc0_dense_plane(const thin_desc* d, int64_t h, int64_t w) {
  return d->dtype == THIN_F16 && d->rank == 5 && d->sizes[4] == 16 && (h == 1 || d->strides[2] == w * 16) &&
         (w == 1 || d->strides[3] == 16) && d->strides[4] == 1 && reinterpret_cast<uintptr_t>(d->data) % 16 == 0 &&
         d->strides[0] % 8 == 0 && d->strides[1] % 8 == 0;
}
bool nc1hwc0_per_channel(const thin_desc* d) {
  return d->dtype == THIN_F16 && d->rank == 5 && d->strides[2] == 0 && d->strides[3] == 0 && d->strides[4] == 1 &&
         reinterpret_cast<uintptr_t>(d->data) % 16 == 0 && d->strides[0] % 8 == 0 && d->strides[1] % 8 == 0;
}

bool flat_geom(const thin_desc* x, const thin_desc* out, const thin_desc* const* chan, int nchan, FlatGeom& g) {
  const int64_t n = x->sizes[0], c1 = x->sizes[1];
  const int64_t plane_elems = x->sizes[2] * x->sizes[3] * 16;
  if (c1 > (int64_t)kFlatMaxC1) return false;
  if (c1 > 1 && (x->strides[1] != plane_elems || out->strides[1] != plane_elems)) return false;
  for (int k = 0; k < nchan; ++k)
    if (n > 1 && chan[k]->strides[0] != 0) return false;
  const int64_t plane_vecs = plane_elems / 8;
  const int64_t span = c1 * plane_vecs;
  const int64_t total = n * span;
  const int64_t x_row = n > 1 ? x->strides[0] / 8 : 0, o_row = n > 1 ? out->strides[0] / 8 : 0;
  const int64_t lim = ((int64_t)1 << 32) - 1;
  if (total >= ((int64_t)1 << 31) || x_row < 0 || o_row < 0 || (n - 1) * x_row + span > lim ||
      (n - 1) * o_row + span > lim)
    return false;
  g.total = (uint32_t)total;
  g.span = (uint32_t)span;
  g.plane_vecs = (uint32_t)plane_vecs;
  g.x_row = (uint32_t)x_row;
  g.o_row = (uint32_t)o_row;
  g.c1 = (uint32_t)c1;
  g.grid2 = (uint32_t)((total + kThreads * 2 - 1) / (kThreads * 2));
  g.grid1 = (uint32_t)((total + kThreads - 1) / kThreads);
  // Streaming loads and stores from kStreamingBytes, for dense tensors and
  // for views with gaps between images (the C2f narrowed x[:, C/2:]) alike.
  // With the buffers cold (rotated over 1.25 GB) the narrowed views time
  // 10.65 / 5.63 / 4.03 us at (128,80,80) / (256,40,40) / (512,20,20), N=32,
  // against 10.82 / 6.13 / 4.38 us with cached loads (a shallower rotation,
  // which let the cache serve part of them, had favoured cached loads).
  g.nt = total * 16 >= kStreamingBytes;
  return true;
}

// Two vectors per thread, or one when that leaves fewer than 256 blocks (a
// single small image): then more blocks shorten the launch.  Streaming
// loads and stores from kStreamingBytes.
#define THIN_FLAT_LAUNCH(KERNEL, g, stream, ...)                                                           \
  do {                                                                                                    \
    if ((g).nt)                                                                                           \
      hipLaunchKernelGGL((KERNEL<2, true, true, ##__VA_ARGS__>), dim3((g).grid2), dim3(kThreads), 0, stream, p);  \
    else if ((g).grid2 >= 256)                                                                            \
      hipLaunchKernelGGL((KERNEL<2, false, false, ##__VA_ARGS__>), dim3((g).grid2), dim3(kThreads), 0, stream, p); \
    else                                                                                                  \
      hipLaunchKernelGGL((KERNEL<1, false, false, ##__VA_ARGS__>), dim3((g).grid1), dim3(kThreads), 0, stream, p); \
  } while (0)

bool try_affine_flat(const thin_desc* x, const thin_desc* sc, const thin_desc* b, const thin_desc* out,
                     hipStream_t stream) {
  const thin_desc* chan[2] = {sc, b};
  FlatGeom g;
  if (!flat_geom(x, out, chan, 2, g)) return false;
  AffineFlatPlan p;
  p.x = static_cast<const h8v*>(x->data);
  p.out = static_cast<h8v*>(out->data);
  p.s = static_cast<const h8v*>(sc->data);
  p.b = static_cast<const h8v*>(b->data);
  p.total = g.total;
  p.span = FastDiv::make(g.span);
  p.plane = FastDiv::make(g.plane_vecs);
  p.x_row = g.x_row;
  p.o_row = g.o_row;
  p.s_c1 = (uint32_t)(sc->strides[1] / 8);
  p.b_c1 = (uint32_t)(b->strides[1] / 8);
  p.c1 = g.c1;
  THIN_FLAT_LAUNCH(affine_silu_flat_kernel, g, stream);
  return true;
}

// Returns true and launches when x/s/b/out have the NC1HWC0 per-channel form.
bool try_affine_blocked(const thin_desc* x, const thin_desc* sc, const thin_desc* b,
                        const thin_desc* out, hipStream_t stream) {
  if (x->dtype != THIN_F16 || x->rank != 5 || x->sizes[4] != 16) return false;
  const int64_t h = x->sizes[2], w = x->sizes[3];
  if (!nc1hwc0_dense_plane(x, h, w) || !nc1hwc0_dense_plane(out, h, w) || !nc1hwc0_per_channel(sc) ||
      !nc1hwc0_per_channel(b))
    return false;
  if (try_affine_flat(x, sc, b, out, stream)) return true;
  const int64_t planes = x->sizes[0] * x->sizes[1];
  const int64_t plane_vecs = h * w * 2;
  if (planes >= ((int64_t)1 << 31) || plane_vecs >= ((int64_t)1 << 30)) return false;
  AffinePlan p;
  p.x = static_cast<const _Float16*>(x->data);
  p.s = static_cast<const _Float16*>(sc->data);
  p.b = static_cast<const _Float16*>(b->data);
  p.out = static_cast<_Float16*>(out->data);
  p.x_n = x->strides[0]; p.x_c1 = x->strides[1];
  p.o_n = out->strides[0]; p.o_c1 = out->strides[1];
  p.s_n = sc->strides[0]; p.s_c1 = sc->strides[1];
  p.b_n = b->strides[0]; p.b_c1 = b->strides[1];
  p.c1 = (uint32_t)x->sizes[1];
  p.planes = (uint32_t)planes;
  p.plane_vecs = (uint32_t)plane_vecs;
  const uint32_t gy = planes < 65535 ? (uint32_t)planes : 65535u;
  const bool nt = planes * plane_vecs * 16 >= kStreamingBytes;
  if (plane_vecs >= 1024) {
    uint32_t gx = (uint32_t)((plane_vecs + kThreads * 2 - 1) / (kThreads * 2));
    if (nt) hipLaunchKernelGGL((affine_silu_blocked_kernel<2, true>), dim3(gx, gy), dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((affine_silu_blocked_kernel<2, false>), dim3(gx, gy), dim3(kThreads), 0, stream, p);
  } else {
    uint32_t gx = (uint32_t)((plane_vecs + kThreads - 1) / kThreads);
    if (nt) hipLaunchKernelGGL((affine_silu_blocked_kernel<1, true>), dim3(gx, gy), dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((affine_silu_blocked_kernel<1, false>), dim3(gx, gy), dim3(kThreads), 0, stream, p);
  }
  return true;
}

// Per-channel binary op on NC1HWC0 fp16 (aten add / sub / mul / div of a
// tensor and a [.,C1,1,1,16] operand, in either order) in the flat form of
// affine_silu_flat_kernel: one vector index decomposition, the image's 2 * C1
// channel vectors staged once per block in LDS.  Every element goes through
// the same functor as the generic map kernels, so the bits are theirs.
struct ChannelFlatPlan {
  const h8v* x;
  h8v* out;
  const h8v* s;      // channel 0, C0 lanes 0-7; lanes 8-15 follow
  uint32_t total;
  FastDiv span;
  FastDiv plane;
  uint32_t x_row, o_row;
  uint32_t s_c1;
  uint32_t c1;
  float alpha;
};

template <int U, bool NTL, bool NTS, bool SFIRST, class Op>
__global__ __launch_bounds__(kThreads) void channel_binary_flat_kernel(ChannelFlatPlan p) {
  __shared__ h8v sv[2 * kFlatMaxC1];
  const uint32_t tile = blockIdx.x * (kThreads * U);
  h8v v[U];
  uint32_t oo[U], q[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t i = tile + u * kThreads + threadIdx.x;
    if (i < p.total) {
      const uint32_t row = p.span.div(i);
      const uint32_t col = i - row * p.span.d;
      oo[u] = row * p.o_row + col;
      q[u] = p.plane.div(col) * 2 + (col & 1u);
      const h8v* src = p.x + row * p.x_row + col;
      v[u] = NTL ? __builtin_nontemporal_load(src) : *src;
    }
  }
  for (uint32_t i = threadIdx.x; i < 2 * p.c1; i += kThreads) sv[i] = p.s[(i >> 1) * p.s_c1 + (i & 1u)];
  __syncthreads();
  const Op op;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t i = tile + u * kThreads + threadIdx.x;
    if (i >= p.total) break;
    const h8v c = sv[q[u]];
    h8v r;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const _Float16 lane[2] = {SFIRST ? c[j] : v[u][j], SFIRST ? v[u][j] : c[j]};
      r[j] = op.template operator()<_Float16, 2>(lane, p.alpha, 0.f);
    }
    store16<NTS>(p.out + oo[u], r);
  }
}

template <class Op>
bool try_channel_flat(const thin_desc* x, const thin_desc* y, const thin_desc* out, float alpha, hipStream_t stream) {
  if (out->dtype != THIN_F16 || out->rank != 5 || out->sizes[4] != 16) return false;
  const int64_t h = out->sizes[2], w = out->sizes[3];
  if (!nc1hwc0_dense_plane(out, h, w)) return false;
  const bool sfirst = nc1hwc0_per_channel(x) && nc1hwc0_dense_plane(y, h, w);
  if (!sfirst && !(nc1hwc0_dense_plane(x, h, w) && nc1hwc0_per_channel(y))) return false;
  const thin_desc* t = sfirst ? y : x;
  const thin_desc* c = sfirst ? x : y;
  FlatGeom g;
  if (!flat_geom(t, out, &c, 1, g)) return false;
  ChannelFlatPlan p;
  p.x = static_cast<const h8v*>(t->data);
  p.out = static_cast<h8v*>(out->data);
  p.s = static_cast<const h8v*>(c->data);
  p.total = g.total;
  p.span = FastDiv::make(g.span);
  p.plane = FastDiv::make(g.plane_vecs);
  p.x_row = g.x_row;
  p.o_row = g.o_row;
  p.s_c1 = (uint32_t)(c->strides[1] / 8);
  p.c1 = g.c1;
  p.alpha = alpha;
  if (sfirst) THIN_FLAT_LAUNCH(channel_binary_flat_kernel, g, stream, true, Op);
  else THIN_FLAT_LAUNCH(channel_binary_flat_kernel, g, stream, false, Op);
  return true;
}

// ------------------------------------------------------------ host launcher

// Elements addressable by one launch (32-bit unit decomposition and offsets).
constexpr int64_t kSpanLimit = ((int64_t)1 << 31) - 1;

constexpr int kUnroll = 2;

template <typename T, int NIN, int ND, class Op>
void launch_plan(const MapPlan<NIN>& p, bool vec, bool nt, hipStream_t stream) {
  constexpr int V = 16 / (int)sizeof(T);
  if (p.units == 0) return;  // the dense and row kernels clamp to unit units - 1
  if constexpr (ND == 1) {
    bool dense = vec && p.out_mode == kVec;
    for (int k = 0; k < NIN; ++k) dense = dense && p.in_mode[k] == kVec;
    if (dense) {
      const uint32_t grid = (p.units + kThreads * kUnroll - 1) / (kThreads * kUnroll);
      if (nt) hipLaunchKernelGGL((map_dense_kernel<T, V, NIN, kUnroll, true, Op>), dim3(grid), dim3(kThreads), 0,
                                 stream, p);
      else if (grid >= 256)
        hipLaunchKernelGGL((map_dense_kernel<T, V, NIN, kUnroll, false, Op>), dim3(grid), dim3(kThreads), 0,
                           stream, p);
      else  // small launches: one unit per thread, twice the blocks
        hipLaunchKernelGGL((map_dense_kernel<T, V, NIN, 1, false, Op>), dim3((p.units + kThreads - 1) / kThreads),
                           dim3(kThreads), 0, stream, p);
      return;
    }
  }
  if constexpr (ND == 2) {
    bool rows = vec && p.nd == 2 && p.out_mode == kVec && p.ostride[0] == 1;
    for (int k = 0; k < NIN; ++k) rows = rows && p.in_mode[k] == kVec && p.istride[k][0] == 1;
    if (rows) {
      MapPlan<NIN> q = p;
      q.div[0] = FastDiv::make(p.size[0] / (uint32_t)V);  // vectors per row
      const uint32_t grid = (p.units + kThreads * kUnroll - 1) / (kThreads * kUnroll);
      // streaming loads for one input, cached for two or more (the narrowed
      // [32,4,80,80,16] half of [32,8,80,80,16]: SiLU in place 11.6 -> 10.4 us
      // streaming; a + b of the two halves inside the captured C2f tail, where
      // the halves were just written: 52.4 us per chain cached against 54.8
      // streaming, though from cold buffers streaming is faster, 14.6 against
      // 15.4 us)
      if (nt && NIN == 1)
        hipLaunchKernelGGL((map_rows_kernel<T, V, NIN, kUnroll, true, true, Op>), dim3(grid), dim3(kThreads), 0,
                           stream, q);
      else if (nt)
        hipLaunchKernelGGL((map_rows_kernel<T, V, NIN, kUnroll, false, true, Op>), dim3(grid), dim3(kThreads), 0,
                           stream, q);
      else
        hipLaunchKernelGGL((map_rows_kernel<T, V, NIN, kUnroll, false, false, Op>), dim3(grid), dim3(kThreads), 0,
                           stream, q);
      return;
    }
  }
  if (vec) {
    if (nt) {
      uint32_t grid = grid_for(p.units, kThreads, kUnroll, 256u * 64u);
      hipLaunchKernelGGL((map_vec_kernel<T, V, NIN, ND, kUnroll, true, Op, kThreads>), dim3(grid),
                         dim3(kThreads), 0, stream, p);
    } else {
      uint32_t grid = grid_for(p.units, kThreads, kUnroll, 256u * 64u);
      hipLaunchKernelGGL((map_vec_kernel<T, V, NIN, ND, kUnroll, false, Op, kThreads>), dim3(grid),
                         dim3(kThreads), 0, stream, p);
    }
  } else {
    uint32_t grid = grid_for(p.units, kThreads, 1, 256u * 16u);
    hipLaunchKernelGGL((map_scalar_kernel<T, NIN, ND, Op>), dim3(grid), dim3(kThreads), 0, stream, p);
  }
}

template <typename T, int NIN, class Op>
thin_status launch_map(const thin_desc* out, const thin_desc* const* ins, float pa, float pb,
                       hipStream_t stream) {
  constexpr int V = 16 / (int)sizeof(T);
  const thin_desc* ops[kMaxOps];
  ops[0] = out;
  for (int k = 0; k < NIN; ++k) ops[k + 1] = ins[k];
  Coalesced c = coalesce(ops, NIN + 1);
  // Kernel plan dims are innermost-first.
  const int nd = c.nd;
  int64_t size[kMaxDims];
  int64_t st[kMaxOps][kMaxDims];
  for (int i = 0; i < nd; ++i) {
    size[i] = c.size[nd - 1 - i];
    for (int k = 0; k <= NIN; ++k) st[k][i] = c.stride[k][nd - 1 - i];
  }
  // Split the outermost dim into slabs whose element count and per-operand
  // offset span fit in 31 bits.
  int64_t inner = 1, inner_span = 0;
  for (int i = 0; i < nd - 1; ++i) inner *= size[i];
  for (int k = 0; k <= NIN; ++k) {
    int64_t span = 0;
    for (int i = 0; i < nd - 1; ++i) span += (size[i] - 1) * st[k][i];
    if (span > inner_span) inner_span = span;
  }
  int64_t outer_stride = 0;
  for (int k = 0; k <= NIN; ++k)
    if (st[k][nd - 1] > outer_stride) outer_stride = st[k][nd - 1];
  THIN_REQUIRE(inner <= kSpanLimit / 2 && inner_span <= kSpanLimit / 2, THIN_ERR_UNSUPPORTED,
               "elementwise: inner extent %lld (span %lld) exceeds one launch", (long long)inner,
               (long long)inner_span);
  const int64_t outer = size[nd - 1];
  int64_t per_slab = nd == 1 ? kSpanLimit / 2 : (kSpanLimit / 2) / inner;
  if (outer_stride > 0) {
    int64_t by_span = (kSpanLimit - inner_span) / outer_stride;
    if (by_span < per_slab) per_slab = by_span;
  }
  if (per_slab < 1) per_slab = 1;
  if (nd == 1) per_slab -= per_slab % 16;  // keep slab boundaries vector aligned

  for (int64_t o0 = 0; o0 < outer; o0 += per_slab) {
    int64_t on = outer - o0 < per_slab ? outer - o0 : per_slab;
    MapPlan<NIN> p;
    memset(&p, 0, sizeof p);
    p.nd = nd;
    for (int i = 0; i < nd; ++i) {
      int64_t s = i == nd - 1 ? on : size[i];
      p.size[i] = (uint32_t)s;
      p.div[i] = FastDiv::make((uint32_t)s);
      p.ostride[i] = (int32_t)st[0][i];
      for (int k = 0; k < NIN; ++k) p.istride[k][i] = (int32_t)st[k + 1][i];
    }
    p.out = static_cast<char*>(out->data) + o0 * st[0][nd - 1] * (int64_t)sizeof(T);
    for (int k = 0; k < NIN; ++k)
      p.in[k] = static_cast<const char*>(ins[k]->data) + o0 * st[k + 1][nd - 1] * (int64_t)sizeof(T);
    p.pa = pa;
    p.pb = pb;
    const int64_t elems = (nd == 1 ? on : inner * on);

    bool vec = V > 1 && p.size[0] % V == 0;
    if (vec) {
      auto aligned = [&](const void* ptr, const int64_t* s) {
        if (reinterpret_cast<uintptr_t>(ptr) % 16) return false;
        for (int i = 1; i < nd; ++i)
          if (s[i] % V) return false;
        return true;
      };
      p.out_mode = (st[0][0] == 1 && aligned(p.out, st[0])) ? kVec : kGather;
      for (int k = 0; k < NIN; ++k) {
        if (st[k + 1][0] == 0) p.in_mode[k] = kBcast;
        else if (st[k + 1][0] == 1 && aligned(p.in[k], st[k + 1])) p.in_mode[k] = kVec;
        else p.in_mode[k] = kGather;
      }
      p.units = (uint32_t)(elems / V);
    } else {
      p.units = (uint32_t)elems;
    }
    const bool nt = elems * (int64_t)sizeof(T) >= kStreamingBytes;
    if (nd == 1) launch_plan<T, NIN, 1, Op>(p, vec, nt, stream);
    else if (nd <= 2) launch_plan<T, NIN, 2, Op>(p, vec, nt, stream);
    else if (nd <= 4) launch_plan<T, NIN, 4, Op>(p, vec, nt, stream);
    else launch_plan<T, NIN, kMaxDims, Op>(p, vec, nt, stream);
    THIN_LAUNCH_CHECK("map");
  }
  return THIN_OK;
}

thin_status check_float_operands(const char* what, const thin_desc* const* ds, int n) {
  for (int k = 0; k < n; ++k) {
    THIN_REQUIRE(desc_valid(ds[k]), THIN_ERR_INVALID, "%s: invalid descriptor %d", what, k);
    THIN_REQUIRE(ds[k]->dtype == THIN_F16 || ds[k]->dtype == THIN_F32, THIN_ERR_INVALID,
                 "%s supports float32/float16, got %s", what, dtype_name(ds[k]->dtype));
    THIN_REQUIRE(ds[k]->dtype == ds[0]->dtype, THIN_ERR_INVALID,
                 "%s requires matching dtypes", what);
    THIN_REQUIRE(same_sizes(ds[k], ds[0]), THIN_ERR_INVALID,
                 "%s requires operands expanded to the output shape", what);
  }
  return THIN_OK;
}

// Host-side rounding of an op parameter to the tensor dtype.
float round_to(int32_t dtype, double v) {
  return dtype == THIN_F16 ? (float)(_Float16)(float)v : (float)v;
}

// An elementwise op maps each element to itself, so any order of the dims
// serves, applied to every operand alike.  The dims go in the order of the
// output's strides, largest first (a stable sort): a permuted view written
// into a view of the same permutation (channels-last memory seen as NCHW,
// x.transpose(1, 2) into out.transpose(1, 2)) then coalesces into dense
// runs instead of a gather along the view's inner dim.  Returns false when
// the order already holds.
bool order_by_output(const thin_desc* out, const thin_desc* const* ins, int nin, thin_desc& o2, thin_desc* i2) {
  int perm[THIN_MAX_DIMS];
  bool sorted = true;
  for (int d = 0; d < out->rank; ++d) perm[d] = d;
  for (int d = 1; d < out->rank; ++d) {
    const int v = perm[d];
    int j = d;
    while (j > 0 && out->strides[perm[j - 1]] < out->strides[v]) {
      perm[j] = perm[j - 1];
      --j;
      sorted = false;
    }
    perm[j] = v;
  }
  if (sorted) return false;
  auto apply = [&](const thin_desc* src, thin_desc& dst) {
    dst = *src;
    for (int d = 0; d < src->rank; ++d) {
      dst.sizes[d] = src->sizes[perm[d]];
      dst.strides[d] = src->strides[perm[d]];
    }
  };
  apply(out, o2);
  for (int k = 0; k < nin; ++k) apply(ins[k], i2[k]);
  return true;
}

template <class Op, int NIN>
thin_status dispatch_float(const thin_desc* out, const thin_desc* const* ins, float pa, float pb,
                           hipStream_t stream) {
  if (numel(out) == 0) return THIN_OK;
  thin_desc o2, i2[NIN];
  const thin_desc* ip[NIN];
  if (order_by_output(out, ins, NIN, o2, i2)) {
    for (int k = 0; k < NIN; ++k) ip[k] = &i2[k];
    out = &o2;
    ins = ip;
  }
  if (out->dtype == THIN_F16) return launch_map<_Float16, NIN, Op>(out, ins, pa, pb, stream);
  return launch_map<float, NIN, Op>(out, ins, pa, pb, stream);
}

}  // namespace

// ------------------------------------------------------------ fill
// out[...] = one element bit pattern.  Dense outputs take 16-byte stores of the
// replicated pattern; any other layout walks the coalesced dims.
__global__ __launch_bounds__(kThreads) void fill_dense_kernel(u32x4* out, uint64_t words, u32x4 pattern) {
  for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < words; i += (uint64_t)gridDim.x * kThreads)
    out[i] = pattern;
}

struct FillPlan {
  char* out;
  int32_t nd;
  int64_t size[kMaxDims];    // innermost first
  int64_t stride[kMaxDims];  // elements
  uint64_t total;
  uint64_t bits;
  FastDiv div[kMaxDims];     // of size[], for SMALL launches (total < 2^31)
};

// SMALL: fewer than 2^31 elements, so the index splits with 32-bit FastDiv
// steps instead of 64-bit divisions (a stride-2 fp16 view of [32,64,80,160]:
// 21.1 -> 17.7 us).
template <typename T, bool SMALL>
__global__ __launch_bounds__(kThreads) void fill_strided_kernel(FillPlan p) {
  const T v = __builtin_bit_cast(T, (typename std::conditional<sizeof(T) == 8, uint64_t,
                                     typename std::conditional<sizeof(T) == 4, uint32_t,
                                     typename std::conditional<sizeof(T) == 2, uint16_t, uint8_t>::type>::type>::type)p.bits);
  if constexpr (SMALL) {
    for (uint32_t e = blockIdx.x * kThreads + threadIdx.x; e < (uint32_t)p.total; e += gridDim.x * kThreads) {
      uint32_t rest = e;
      int64_t off = 0;
      for (int d = 0; d < p.nd; ++d) {
        const uint32_t q = p.div[d].div(rest);
        off += (int64_t)(rest - q * p.div[d].d) * p.stride[d];
        rest = q;
      }
      reinterpret_cast<T*>(p.out)[off] = v;
    }
    return;
  }
  for (uint64_t e = (uint64_t)blockIdx.x * kThreads + threadIdx.x; e < p.total; e += (uint64_t)gridDim.x * kThreads) {
    uint64_t rest = e;
    int64_t off = 0;
    for (int d = 0; d < p.nd; ++d) {
      const uint64_t q = rest / (uint64_t)p.size[d];
      off += (int64_t)(rest - q * (uint64_t)p.size[d]) * p.stride[d];
      rest = q;
    }
    reinterpret_cast<T*>(p.out)[off] = v;
  }
}

// Element bits of `value` (float dtypes) or `ivalue` (integer dtypes).
uint64_t fill_bits(int32_t dtype, double value, int64_t ivalue) {
  switch (dtype) {
    case THIN_F16: return __builtin_bit_cast(uint16_t, (_Float16)(float)value);
    case THIN_BF16: {
      const float f = (float)value;
      uint32_t u = __builtin_bit_cast(uint32_t, f);
      if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
      u += 0x7fffu + ((u >> 16) & 1u);                                               // round to nearest even
      return (uint16_t)(u >> 16);
    }
    case THIN_F32: return __builtin_bit_cast(uint32_t, (float)value);
    case THIN_F64: return __builtin_bit_cast(uint64_t, value);
    case THIN_I64: return (uint64_t)ivalue;
    case THIN_I32: return (uint32_t)(int32_t)ivalue;
    case THIN_I16: return (uint16_t)(int16_t)ivalue;
    case THIN_U8: return (uint8_t)ivalue;
  }
  return 0;
}

// ------------------------------------------------------------ transpose
// Batched 2-D transpose copy: dst[b][p][m] = src[b][m][p] where src rows run
// along p (unit stride) and dst rows along m (unit stride) -- the layout of
// x.permute(...).contiguous() for an NCHW <-> NHWC change.  A block moves a
// 64 x 64 tile: 16-byte loads along src rows into LDS (rows padded by one
// 4-byte word so that column reads hit distinct banks), then 16-byte stores
// along dst rows.  Tile edges and unaligned rows take per-element accesses.
constexpr uint32_t kTile = 64;

struct TransposePlan {
  const char* src;
  char* dst;
  uint32_t M, P, B;          // dst-inner extent, src-inner extent, batches
  int64_t s_m, s_b;          // src strides (elements) of m and b; p stride is 1
  int64_t d_p, d_b;          // dst strides (elements) of p and b; m stride is 1
  uint32_t tiles_m, tiles_p;
  uint32_t vec_src, vec_dst; // 16-byte rows possible (alignment checked on the host)
};

// W tiles per block along p (W = 2: 2-byte elements, every tile whole and
// both sides 16-byte aligned, which the host checks): a source row is then
// read W * 128 contiguous bytes at a time instead of 128.
template <typename T, bool NT, uint32_t W>
__global__ __launch_bounds__(kThreads) void transpose_kernel(TransposePlan p) {
  static_assert(W == 1 || (W == 2 && sizeof(T) == 2), "wide blocks: 2-byte elements only");
  constexpr uint32_t V = 16 / sizeof(T);
  constexpr uint32_t kRow = kTile + 4 / sizeof(T);  // padded LDS row, in elements
  __shared__ __attribute__((aligned(16))) T tile[W * kTile * kRow];
  // the plan in registers before the first test of one of its fields: one
  // round of scalar loads (one asm statement: each is a scheduling boundary)
  __asm__ volatile("" ::"s"(p.src), "s"(p.dst), "s"(p.M), "s"(p.P), "s"(p.s_m), "s"(p.s_b), "s"(p.d_p), "s"(p.d_b),
                   "s"(p.tiles_m), "s"(p.tiles_p), "s"(p.vec_src), "s"(p.vec_dst));
  const uint32_t tiles_p = p.tiles_p / W;  // blocks along p
  const uint32_t per_b = p.tiles_m * tiles_p;
  const uint32_t b = blockIdx.x / per_b, rest = blockIdx.x - b * per_b;
  const uint32_t tm = rest / tiles_p, tp = (rest - tm * tiles_p) * W;
  const uint32_t m0 = tm * kTile, p0 = tp * kTile;
  const T* src = reinterpret_cast<const T*>(p.src) + b * p.s_b;
  T* dst = reinterpret_cast<T*>(p.dst) + b * p.d_b;
  const bool full = m0 + kTile <= p.M && p0 + W * kTile <= p.P;
  if constexpr (sizeof(T) == 2) {
    if (W == 2 || (full && p.vec_src && p.vec_dst)) {
      // whole 2-byte tiles with 16-byte rows on both sides: every load in
      // flight before the LDS writes (4-byte words), and each thread reads
      // 4-byte column pairs from 8 tile rows to build two output vectors
      typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
      constexpr uint32_t CV = W * kTile / V;                // 16-byte vectors per staged row
      constexpr uint32_t U = W * kTile * kTile / V / kThreads;  // 2 per tile
      constexpr uint32_t kWords = kRow / 2;                 // padded row in 4-byte words (33)
      uint32_t* words = reinterpret_cast<uint32_t*>(tile);
      u32x4_t w[U];
#pragma unroll
      for (uint32_t u = 0; u < U; ++u) {
        const uint32_t i = threadIdx.x + u * kThreads;
        const uint32_t r = i / CV, cv = (i % CV) * V;
        w[u] = load16<NT, u32x4_t>(src + (int64_t)(m0 + r) * p.s_m + p0 + cv);
      }
#pragma unroll
      for (uint32_t u = 0; u < U; ++u) {
        const uint32_t i = threadIdx.x + u * kThreads;
        const uint32_t r = i / CV, cv = (i % CV) * V;
        const uint32_t t = cv / kTile, c = cv % kTile;  // tile of the block, column in it
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) words[(t * kTile + r) * kWords + c / 2 + k] = w[u][k];
      }
      __syncthreads();
      // thread -> (column pair qp of the tile, 8-row group g): lanes 8 apart
      // share a destination row, and the 64 lanes hit 64 distinct banks
      const uint32_t g = threadIdx.x % (kTile / 8), qp = threadIdx.x / (kTile / 8);
#pragma unroll
      for (uint32_t t = 0; t < W; ++t) {
        const uint32_t* tw = words + t * kTile * kWords;
        uint32_t lo[4], hi[4];
#pragma unroll
        for (uint32_t j = 0; j < 8; j += 2) {
          const uint32_t a = tw[(g * 8 + j) * kWords + qp], b = tw[(g * 8 + j + 1) * kWords + qp];
          lo[j / 2] = (a & 0xffffu) | (b << 16);           // column 2qp, rows g*8+j, +1
          hi[j / 2] = (a >> 16) | (b & 0xffff0000u);       // column 2qp+1
        }
        T* row0 = dst + (int64_t)(p0 + t * kTile + 2 * qp) * p.d_p + m0 + g * 8;
        store16<NT>(row0, (u32x4_t){lo[0], lo[1], lo[2], lo[3]});
        store16<NT>(row0 + p.d_p, (u32x4_t){hi[0], hi[1], hi[2], hi[3]});
      }
      return;
    }
  }
  if constexpr (W == 1) {
  // load: tile row r = m0 + r, columns p0 .. p0+63; every load of the thread
  // issued before the first LDS write (a partial tile loads each element
  // from a position clamped into the matrix and writes only those inside)
  constexpr uint32_t U = kTile * kTile / V / kThreads;
  VecT<T, V> w[U];
  if (full && p.vec_src) {
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t i = threadIdx.x + u * kThreads, r = i / (kTile / V), cv = (i % (kTile / V)) * V;
      w[u] = load16<NT, VecT<T, V>>(src + (int64_t)(m0 + r) * p.s_m + p0 + cv);
    }
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t i = threadIdx.x + u * kThreads, r = i / (kTile / V), cv = (i % (kTile / V)) * V;
#pragma unroll
      for (uint32_t j = 0; j < V; ++j) tile[r * kRow + cv + j] = w[u].v[j];
    }
  } else {
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t i = threadIdx.x + u * kThreads, r = i / (kTile / V), cv = (i % (kTile / V)) * V;
      const T* row = src + (int64_t)min(m0 + r, p.M - 1) * p.s_m;
#pragma unroll
      for (uint32_t j = 0; j < V; ++j) w[u].v[j] = row[min(p0 + cv + j, p.P - 1)];
    }
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t i = threadIdx.x + u * kThreads, r = i / (kTile / V), cv = (i % (kTile / V)) * V;
#pragma unroll
      for (uint32_t j = 0; j < V; ++j)
        if (m0 + r < p.M && p0 + cv + j < p.P) tile[r * kRow + cv + j] = w[u].v[j];
    }
  }
  __syncthreads();
  // store: dst row p0 + q, columns m0 .. m0+63
  for (uint32_t i = threadIdx.x; i < kTile * kTile / V; i += kThreads) {
    const uint32_t q = i / (kTile / V), cm = (i % (kTile / V)) * V;
    T* row = dst + (int64_t)(p0 + q) * p.d_p + m0 + cm;
    VecT<T, V> w;
#pragma unroll
    for (uint32_t j = 0; j < V; ++j) w.v[j] = tile[(cm + j) * kRow + q];
    if (full && p.vec_dst) {
      store16<NT>(row, w);
    } else {
#pragma unroll
      for (uint32_t j = 0; j < V; ++j)
        if (p0 + q < p.P && m0 + cm + j < p.M) row[j] = w.v[j];
    }
  }
  }
}

// Launches the tiled transpose when dst <- src is a batched 2-D transpose of
// 2- or 4-byte elements; returns false (nothing launched) otherwise.
bool try_transpose(const thin_desc* src, const thin_desc* dst, hipStream_t stream) {
  const int esz = dtype_size(dst->dtype);
  if (esz != 2 && esz != 4) return false;
  const thin_desc* ops[2] = {dst, src};
  Coalesced c = coalesce(ops, 2);
  if (c.nd < 2 || c.nd > 3) return false;
  const int in = c.nd - 1;                       // innermost dim: dst-contiguous
  if (c.stride[0][in] != 1 || c.stride[1][in] == 1) return false;
  int pd = -1;
  for (int d = 0; d < in; ++d)
    if (c.stride[1][d] == 1) pd = d;
  if (pd < 0) return false;
  const int bd = c.nd == 3 ? (pd == 0 ? 1 : 0) : -1;
  const int64_t M = c.size[in], P = c.size[pd], B = bd >= 0 ? c.size[bd] : 1;
  if (M < 16 || P < 16) return false;            // thin slabs: the vector map path is as good
  TransposePlan t;
  t.src = static_cast<const char*>(src->data);
  t.dst = static_cast<char*>(dst->data);
  t.M = (uint32_t)M;
  t.P = (uint32_t)P;
  t.B = (uint32_t)B;
  t.s_m = c.stride[1][in];
  t.d_p = c.stride[0][pd];
  t.s_b = bd >= 0 ? c.stride[1][bd] : 0;
  t.d_b = bd >= 0 ? c.stride[0][bd] : 0;
  t.tiles_m = (uint32_t)((M + kTile - 1) / kTile);
  t.tiles_p = (uint32_t)((P + kTile - 1) / kTile);
  uint64_t blocks = (uint64_t)B * t.tiles_m * t.tiles_p;
  if (M >= (1ll << 31) || P >= (1ll << 31) || blocks >= (1ull << 31)) return false;
  auto a16 = [](const void* q, int64_t stride, int e) {
    return reinterpret_cast<uintptr_t>(q) % 16 == 0 && (stride * e) % 16 == 0;
  };
  t.vec_src = a16(src->data, t.s_m, esz) && (t.s_b * esz) % 16 == 0;
  t.vec_dst = a16(dst->data, t.d_p, esz) && (t.d_b * esz) % 16 == 0;
  const bool nt = (int64_t)B * M * P * esz >= kStreamingBytes;
  // two tiles per block when every tile is whole and 16-byte aligned
  const bool wide = esz == 2 && M % kTile == 0 && P % (2 * kTile) == 0 && t.vec_src && t.vec_dst;
  if (wide) blocks /= 2;
  if (wide && nt)
    hipLaunchKernelGGL((transpose_kernel<uint16_t, true, 2>), dim3((uint32_t)blocks), dim3(kThreads), 0, stream, t);
  else if (wide)
    hipLaunchKernelGGL((transpose_kernel<uint16_t, false, 2>), dim3((uint32_t)blocks), dim3(kThreads), 0, stream, t);
  else if (esz == 2 && nt)
    hipLaunchKernelGGL((transpose_kernel<uint16_t, true, 1>), dim3((uint32_t)blocks), dim3(kThreads), 0, stream, t);
  else if (esz == 2)
    hipLaunchKernelGGL((transpose_kernel<uint16_t, false, 1>), dim3((uint32_t)blocks), dim3(kThreads), 0, stream, t);
  else if (nt)
    hipLaunchKernelGGL((transpose_kernel<uint32_t, true, 1>), dim3((uint32_t)blocks), dim3(kThreads), 0, stream, t);
  else
    hipLaunchKernelGGL((transpose_kernel<uint32_t, false, 1>), dim3((uint32_t)blocks), dim3(kThreads), 0, stream, t);
  return true;
}

// Raw bit copy used by the copy/cat/materialize paths.
thin_status copy_bits(const thin_desc* src, const thin_desc* dst, hipStream_t stream) {
  const thin_desc* ins[1] = {src};
  if (numel(dst) == 0) return THIN_OK;
  switch (dtype_size(dst->dtype)) {
    case 1: return launch_map<uint8_t, 1, OpCopy>(dst, ins, 0.f, 0.f, stream);
    case 2: return launch_map<uint16_t, 1, OpCopy>(dst, ins, 0.f, 0.f, stream);
    case 4: return launch_map<uint32_t, 1, OpCopy>(dst, ins, 0.f, 0.f, stream);
    case 8: return launch_map<uint64_t, 1, OpCopy>(dst, ins, 0.f, 0.f, stream);
  }
  set_error("copy: unsupported dtype");
  return THIN_ERR_INVALID;
}

}  // namespace thin

using namespace thin;

// Bytes [lo, hi) that a descriptor's elements span (strides are >= 0).
void byte_span(const thin_desc* d, uintptr_t& lo, uintptr_t& hi) {
  int64_t last = 0;
  for (int i = 0; i < d->rank; ++i) last += (d->sizes[i] - 1) * d->strides[i];
  lo = reinterpret_cast<uintptr_t>(d->data);
  hi = lo + (uintptr_t)(last + 1) * (uintptr_t)dtype_size(d->dtype);
}

// An operand that is a batched 2-D transpose of a dense output (a permuted
// view, x + y.transpose(1, 2)) would be gathered element by element, one
// 2-byte read per lane: 75 us for [32,64,80,80] fp16 against 10.5 us for the
// tiled transpose of the same tensor.  For outputs of 1 MB and more whose
// bytes no operand shares, that operand is first transposed into the output
// with the tiled kernel and the op then reads it there, in place (each
// element read and written at one index by one thread).  The values, and so
// the result's bits, are the same.  Returns the operand taken, or -1.
constexpr int64_t kTransposeFirstBytes = 1 << 20;
int transpose_operand_first(const thin_desc* out, const thin_desc* const* ins, int nin, hipStream_t stream) {
  if (!is_contiguous(out) || numel(out) * dtype_size(out->dtype) < kTransposeFirstBytes) return -1;
  uintptr_t olo, ohi;
  byte_span(out, olo, ohi);
  for (int k = 0; k < nin; ++k) {
    uintptr_t lo, hi;
    byte_span(ins[k], lo, hi);
    if (lo < ohi && olo < hi) return -1;
  }
  for (int k = 0; k < nin; ++k) {
    bool broadcast = false;  // stride-0 operands are read once per vector already
    for (int i = 0; i < ins[k]->rank; ++i) broadcast |= ins[k]->sizes[i] > 1 && ins[k]->strides[i] == 0;
    if (!broadcast && ins[k]->dtype == out->dtype && same_sizes(ins[k], out) && try_transpose(ins[k], out, stream))
      return k;
  }
  return -1;
}

extern "C" thin_status thin_binary(int32_t op, const thin_desc* x, const thin_desc* y,
                                   const thin_desc* out, float alpha, hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(x && y && out, THIN_ERR_INVALID, "binary: null descriptor");
  const thin_desc* all[3] = {out, x, y};
  thin_status s = check_float_operands("binary", all, 3);
  if (s) return s;
  const thin_desc* ins[2] = {x, y};
  // PyTorch CPU rounds alpha to the tensor dtype before its fp32 evaluation.
  const float a = round_to(out->dtype, alpha);
  if (numel(out) != 0) {
    bool flat = false;
    switch (op) {
      case THIN_ADD: flat = try_channel_flat<OpAdd>(x, y, out, a, stream); break;
      case THIN_SUB: flat = try_channel_flat<OpSub>(x, y, out, a, stream); break;
      case THIN_MUL: flat = try_channel_flat<OpMul>(x, y, out, 1.f, stream); break;
      case THIN_DIV: flat = try_channel_flat<OpDiv>(x, y, out, 1.f, stream); break;
    }
    if (flat) {
      THIN_LAUNCH_CHECK("binary_channel_flat");
      return THIN_OK;
    }
    const int k = transpose_operand_first(out, ins, 2, stream);
    if (k >= 0) {
      THIN_LAUNCH_CHECK("binary_transpose_operand");
      ins[k] = out;
    }
  }
  switch (op) {
    case THIN_ADD: return dispatch_float<OpAdd, 2>(out, ins, a, 0.f, stream);
    case THIN_SUB: return dispatch_float<OpSub, 2>(out, ins, a, 0.f, stream);
    case THIN_MUL: return dispatch_float<OpMul, 2>(out, ins, 1.f, 0.f, stream);
    case THIN_DIV: return dispatch_float<OpDiv, 2>(out, ins, 1.f, 0.f, stream);
  }
  set_error("binary: unknown op %d", op);
  return THIN_ERR_INVALID;
}

extern "C" thin_status thin_binary_scalar(int32_t op, const thin_desc* x, double scalar,
                                          int32_t scalar_first, const thin_desc* out, float alpha,
                                          hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(x && out, THIN_ERR_INVALID, "binary_scalar: null descriptor");
  const thin_desc* all[2] = {out, x};
  thin_status s = check_float_operands("binary_scalar", all, 2);
  if (s) return s;
  const thin_desc* ins[1] = {x};
  // PyTorch CPU semantics of a wrapped Python number on a reduced-precision
  // tensor: add/sub round the scalar (and alpha) to the tensor dtype, mul/div
  // keep it at fp32 opmath precision.
  const bool additive = op == THIN_ADD || op == THIN_SUB;
  const float sv = additive ? round_to(out->dtype, scalar) : (float)scalar;
  alpha = round_to(out->dtype, alpha);
  if (numel(out) != 0 && transpose_operand_first(out, ins, 1, stream) == 0) {
    THIN_LAUNCH_CHECK("binary_scalar_transpose_operand");
    ins[0] = out;
  }
#define THIN_SCALAR_CASE(OPC)                                                              \
  case OPC:                                                                                \
    return scalar_first ? dispatch_float<OpScalar<OPC, true>, 1>(out, ins, alpha, sv, stream) \
                        : dispatch_float<OpScalar<OPC, false>, 1>(out, ins, alpha, sv, stream);
  switch (op) {
    THIN_SCALAR_CASE(THIN_ADD)
    THIN_SCALAR_CASE(THIN_SUB)
    THIN_SCALAR_CASE(THIN_MUL)
    THIN_SCALAR_CASE(THIN_DIV)
  }
#undef THIN_SCALAR_CASE
  set_error("binary_scalar: unknown op %d", op);
  return THIN_ERR_INVALID;
}

extern "C" thin_status thin_unary(int32_t op, const thin_desc* x, const thin_desc* out,
                                  hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(x && out, THIN_ERR_INVALID, "unary: null descriptor");
  const thin_desc* all[2] = {out, x};
  thin_status s = check_float_operands("unary", all, 2);
  if (s) return s;
  const thin_desc* ins[1] = {x};
  if (numel(out) != 0 && transpose_operand_first(out, ins, 1, stream) == 0) {
    THIN_LAUNCH_CHECK("unary_transpose_operand");
    ins[0] = out;
  }
  switch (op) {
    case THIN_SIGMOID: return dispatch_float<OpSigmoid, 1>(out, ins, 0.f, 0.f, stream);
    case THIN_SILU: return dispatch_float<OpSilu, 1>(out, ins, 0.f, 0.f, stream);
  }
  set_error("unary: unknown op %d", op);
  return THIN_ERR_INVALID;
}

extern "C" thin_status thin_silu_add(const thin_desc* x, const thin_desc* y, const thin_desc* out,
                                     hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(x && y && out, THIN_ERR_INVALID, "silu_add: null descriptor");
  const thin_desc* all[3] = {out, x, y};
  thin_status s = check_float_operands("silu_add", all, 3);
  if (s) return s;
  const thin_desc* ins[2] = {x, y};
  if (numel(out) != 0) {
    const int k = transpose_operand_first(out, ins, 2, stream);
    if (k >= 0) {
      THIN_LAUNCH_CHECK("silu_add_transpose_operand");
      ins[k] = out;
    }
  }
  return dispatch_float<OpSiluAdd, 2>(out, ins, 0.f, 0.f, stream);
}

extern "C" thin_status thin_affine_silu(const thin_desc* x, const thin_desc* sc, const thin_desc* b,
                                        const thin_desc* out, hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(x && sc && b && out, THIN_ERR_INVALID, "affine_silu: null descriptor");
  const thin_desc* all[4] = {out, x, sc, b};
  thin_status s = check_float_operands("affine_silu", all, 4);
  if (s) return s;
  if (numel(out) == 0) return THIN_OK;
  if (try_affine_blocked(x, sc, b, out, stream)) {
    THIN_LAUNCH_CHECK("affine_silu_blocked");
    return THIN_OK;
  }
  const thin_desc* ins[3] = {x, sc, b};
  return dispatch_float<OpAffineSilu, 3>(out, ins, 0.f, 0.f, stream);
}

extern "C" thin_status thin_copy(const thin_desc* src, const thin_desc* dst, hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(desc_valid(src) && desc_valid(dst), THIN_ERR_INVALID, "copy: invalid descriptor");
  THIN_REQUIRE(same_sizes(src, dst), THIN_ERR_INVALID, "copy requires matching sizes");
  THIN_REQUIRE(dtype_size(src->dtype) == dtype_size(dst->dtype) && src->dtype == dst->dtype,
               THIN_ERR_INVALID, "copy requires matching dtypes");
  if (numel(dst) == 0) return THIN_OK;
  if (try_transpose(src, dst, stream)) {
    THIN_LAUNCH_CHECK("transpose");
    return THIN_OK;
  }
  return copy_bits(src, dst, stream);
}

extern "C" thin_status thin_fill(const thin_desc* out, double value, int64_t ivalue, hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(desc_valid(out), THIN_ERR_INVALID, "fill: invalid descriptor");
  const int64_t total = numel(out);
  if (total == 0) return THIN_OK;
  const int esz = dtype_size(out->dtype);
  const uint64_t bits = fill_bits(out->dtype, value, ivalue);
  const thin_desc* ops[1] = {out};
  Coalesced c = coalesce(ops, 1);
  const bool dense = c.nd == 1 && c.stride[0][0] == 1;
  if (dense && reinterpret_cast<uintptr_t>(out->data) % 16 == 0 && (total * esz) % 16 == 0) {
    uint32_t lanes[4];
    for (int w = 0; w < 4; ++w) {
      uint32_t word = 0;
      for (int b = 0; b < 4; ++b) word |= (uint32_t)((bits >> (8 * ((w * 4 + b) % esz))) & 0xffu) << (8 * b);
      lanes[w] = word;
    }
    const u32x4 pattern = {lanes[0], lanes[1], lanes[2], lanes[3]};
    const uint64_t words = (uint64_t)total * esz / 16;
    hipLaunchKernelGGL(fill_dense_kernel, dim3(grid_for(words, kThreads, 1, 65536u)), dim3(kThreads), 0, stream,
                       static_cast<u32x4*>(out->data), words, pattern);
    THIN_LAUNCH_CHECK("fill");
    return THIN_OK;
  }
  FillPlan p;
  memset(&p, 0, sizeof p);
  p.out = static_cast<char*>(out->data);
  p.nd = c.nd;
  for (int i = 0; i < c.nd; ++i) {
    p.size[i] = c.size[c.nd - 1 - i];
    p.stride[i] = c.stride[0][c.nd - 1 - i];
  }
  p.total = (uint64_t)total;
  p.bits = bits;
  const bool small = (uint64_t)total < (1ull << 31);
  if (small)
    for (int i = 0; i < c.nd; ++i) p.div[i] = FastDiv::make((uint32_t)p.size[i]);
  const uint32_t grid = grid_for((uint64_t)total, kThreads, 1, 65536u);
#define THIN_FILL(T)                                                                                          \
  do {                                                                                                        \
    if (small) hipLaunchKernelGGL((fill_strided_kernel<T, true>), dim3(grid), dim3(kThreads), 0, stream, p);  \
    else hipLaunchKernelGGL((fill_strided_kernel<T, false>), dim3(grid), dim3(kThreads), 0, stream, p);       \
  } while (0)
  switch (esz) {
    case 1: THIN_FILL(uint8_t); break;
    case 2: THIN_FILL(uint16_t); break;
    case 4: THIN_FILL(uint32_t); break;
    default: THIN_FILL(uint64_t); break;
  }
#undef THIN_FILL
  THIN_LAUNCH_CHECK("fill");
  return THIN_OK;
}
