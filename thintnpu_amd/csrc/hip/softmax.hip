// Softmax family: row softmax over a contiguous last dim, strided softmax over
// any other dim (the DFL [B,16,4,A] view included), and the fused DFL
// softmax-expectation.
//
// Arithmetic follows PyTorch CPU (and the reference kernels): fp32 max (NaN
// propagating), e = exp(x - max), s = sum(e); the last-dim form writes
// e * (1/s), the strided form e / s.  A NaN anywhere in a row, an all -inf row
// or a +inf element therefore make the whole row NaN exactly as on CPU.
// fp16 outputs use the hardware exp2 (its fp32 error is far below an fp16
// ulp); fp32 outputs use the library expf.
#include "common.h"

#include <string.h>

#include <algorithm>

namespace thin {
namespace {

using dev::fast_exp;
using dev::max_nan;
using dev::wave_max_nan;
using dev::wave_sum;

constexpr uint32_t kThreads = 256;
constexpr uint32_t kWaves = kThreads / 64;

template <bool FAST>
__device__ __forceinline__ float expo(float x) {
  if (FAST) return fast_exp(x);
  return expf(x);
}

// exp(x - m) of the column kernels.  FAST (fp16 output): exp2(x*log2e -
// m*log2e) as one fma, the row kernel's form; otherwise expf(x - m).
template <bool FAST>
__device__ __forceinline__ float expd(float x, float m) {
  constexpr float kLog2e = 1.4426950408889634f;
  if (FAST) return __builtin_amdgcn_exp2f(__builtin_fmaf(x, kLog2e, -(m * kLog2e)));
  return expf(x - m);
}

template <typename T> __device__ __forceinline__ float ldf(const T* p) { return (float)*p; }
template <typename T> __device__ __forceinline__ void stf(T* p, float v) { *p = (T)v; }

// Non-reduced ("column") index space, innermost-first, with x/out strides.
struct SoftmaxPlan {
  const void* x;
  void* out;
  int32_t nd;
  uint32_t size[kMaxDims];
  FastDiv div[kMaxDims];
  int64_t xs[kMaxDims], os[kMaxDims];
  uint32_t units;      // rows (row kernel) or column vectors (column kernel)
  uint32_t R;          // reduction length
  int64_t xr, orr;     // reduction strides (column kernel)
};

// The innermost dim is taken with no test on p.nd (a plan with nd = 0 has
// zero strides there), so its fields load in the kernel's first round of
// scalar loads; the rest follow only where nd asks for them.
__device__ __forceinline__ void col_offsets(const SoftmaxPlan& p, uint32_t e, int64_t& xo, int64_t& oo) {
  const uint32_t q0 = p.div[0].div(e);
  const int64_t c0 = (int64_t)(e - q0 * p.size[0]);
  xo = c0 * p.xs[0];
  oo = c0 * p.os[0];
  e = q0;
#pragma unroll
  for (int d = 1; d < kMaxDims; ++d) {
    if (d >= p.nd) break;
    const uint32_t q = p.div[d].div(e);
    const int64_t c = (int64_t)(e - q * p.size[d]);
    e = q;
    xo += c * p.xs[d];
    oo += c * p.os[d];
  }
}

// ---------------------------------------------------------------- rows
// G lanes per row (a power of two <= 64, so a wavefront holds 64/G rows); lane
// g of a row holds chunks g, g+G, ... (KPT of them), a chunk being VE elements
// (one 16-byte vector when VEC, else one element).  G is chosen so that KPT is
// about 2: several loads in flight per lane and few idle lanes.  The row max
// only stabilises the exponentials, so it is a plain max: a NaN element, a
// +inf element (inf - inf) or an all -inf row (-inf - -inf) makes the sum and
// so every output NaN, exactly as on CPU.  FAST (fp16 output): e = exp2(x *
// log2e - m * log2e) as one fma; an error in the common term scales every e
// alike and cancels in e / sum.
using dev::group_max;
using dev::group_sum;

template <typename TI, typename TO, bool VEC, int G, int KPT, bool FAST, bool NT>
__global__ __launch_bounds__(kThreads) void softmax_row_kernel(SoftmaxPlan p) {
  constexpr int VE = VEC ? 16 / (int)sizeof(TI) : 1;
  constexpr int RPW = 64 / G;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t g = lane % G;
  const uint32_t row = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * RPW + lane / G;
  const bool live = row < p.units;  // every lane still joins the group shuffles
  // the operand pointers in registers with the first round of scalar loads
  // (they were loaded only after the test of p.nd in col_offsets)
  __asm__ volatile("" ::"s"(p.x), "s"(p.out), "s"(p.units), "s"(p.nd), "s"(p.R));
  // offsets of a clamped row rather than under a test of live, so that the
  // plan's scalar loads are not held behind the load of p.units
  int64_t xo, oo;
  col_offsets(p, min(row, p.units - 1), xo, oo);
  const TI* xr = static_cast<const TI*>(p.x) + xo;
  TO* orow = static_cast<TO*>(p.out) + oo;
  const uint32_t chunks = VEC ? p.R / VE : p.R;
  if constexpr (VEC && FAST && sizeof(TI) == 2 && sizeof(TO) == 2) {
    // fp16 in and out: the shared fp16 row core (the fused attention kernel
    // runs the same one)
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    dev::h8 raw[KPT], out[KPT];
    bool have[KPT];
#pragma unroll
    for (int k = 0; k < KPT; ++k) {
      const uint32_t c = g + G * k;
      have[k] = live && c < chunks;
      if (have[k]) {
        const u4* src = reinterpret_cast<const u4*>(xr) + c;
        raw[k] = __builtin_bit_cast(dev::h8, NT ? __builtin_nontemporal_load(src) : *src);
      }
    }
    dev::softmax_row_h8<G, KPT>(raw, have, out);
#pragma unroll
    for (int k = 0; k < KPT; ++k) {
      if (have[k]) {
        u4* dst = reinterpret_cast<u4*>(orow) + (g + G * k);
        const u4 w = __builtin_bit_cast(u4, out[k]);
        if constexpr (NT) __builtin_nontemporal_store(w, dst);
        else *dst = w;
      }
    }
    return;
  }
  struct alignas(VE * sizeof(TI)) WI { TI e[VE]; };
  WI raw[KPT];
  // every chunk's load issued, unconditionally (chunks past the row reload
  // its last one, unused), before the first is used: one memory round trip
  // per row, not one per chunk
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    const WI* src = reinterpret_cast<const WI*>(xr) + min(g + G * k, chunks - 1);
    if constexpr (VEC && NT) raw[k] = __builtin_bit_cast(WI, __builtin_nontemporal_load(
                                 reinterpret_cast<const uint32_t __attribute__((ext_vector_type(4)))*>(src)));
    else raw[k] = *src;
  }
  float m = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    if (live && g + G * k < chunks) {
#pragma unroll
      for (int j = 0; j < VE; ++j) m = fmaxf(m, (float)raw[k].e[j]);
    }
  }
  m = group_max<G>(m);
  constexpr float kLog2e = 1.4426950408889634f;
  const float ml = m * kLog2e;
  float e[KPT][VE];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    const uint32_t c = g + G * k;
    if (live && c < chunks) {
#pragma unroll
      for (int j = 0; j < VE; ++j) {
        const float x = (float)raw[k].e[j];
        e[k][j] = FAST ? __builtin_amdgcn_exp2f(__builtin_fmaf(x, kLog2e, -ml)) : expf(x - m);
        s += e[k][j];
      }
    }
  }
  s = group_sum<G>(s);
  const float inv = 1.0f / s;
  struct alignas(VE * sizeof(TO)) WO { TO e[VE]; };
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    const uint32_t c = g + G * k;
    if (live && c < chunks) {
      WO w;
#pragma unroll
      for (int j = 0; j < VE; ++j) w.e[j] = (TO)(e[k][j] * inv);
      WO* dst = reinterpret_cast<WO*>(orow) + c;
      if constexpr (VEC && NT && sizeof(WO) == 16) __builtin_nontemporal_store(
          __builtin_bit_cast(uint32_t __attribute__((ext_vector_type(4))), w),
          reinterpret_cast<uint32_t __attribute__((ext_vector_type(4)))*>(dst));
      else *dst = w;
    }
  }
}

// One block per row, three passes over the row (rows too long for registers).
template <typename TI, typename TO, bool FAST>
__global__ __launch_bounds__(kThreads) void softmax_row_stream_kernel(SoftmaxPlan p) {
  __shared__ float red[kWaves];
  const uint32_t row = blockIdx.x;
  int64_t xo, oo;
  col_offsets(p, row, xo, oo);
  const TI* xr = static_cast<const TI*>(p.x) + xo;
  TO* orow = static_cast<TO*>(p.out) + oo;
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  // one pass over the thread's elements i = tid + k * kThreads, eight at a
  // time: all eight loads (clamped into the row) issued before the first is
  // used, the elements then taken in order
  constexpr uint32_t B = 8;
  auto pass = [&](auto&& f) {
    for (uint32_t i0 = threadIdx.x; i0 < p.R; i0 += B * kThreads) {
      float v[B];
#pragma unroll
      for (uint32_t k = 0; k < B; ++k) v[k] = ldf(xr + min(i0 + k * kThreads, p.R - 1));
#pragma unroll
      for (uint32_t k = 0; k < B; ++k)
        if (i0 + k * kThreads < p.R) f(i0 + k * kThreads, v[k]);
    }
  };
  float m = -__builtin_inff();
  pass([&](uint32_t, float v) { m = max_nan(m, v); });
  m = wave_max_nan(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = red[0];
#pragma unroll
  for (uint32_t w = 1; w < kWaves; ++w) m = max_nan(m, red[w]);
  __syncthreads();
  float s = 0.f;
  pass([&](uint32_t, float v) { s += expo<FAST>(v - m); });
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  s = 0.f;
#pragma unroll
  for (uint32_t w = 0; w < kWaves; ++w) s += red[w];
  const float inv = 1.0f / s;
  pass([&](uint32_t i, float v) { stf(orow + i, expo<FAST>(v - m) * inv); });
}

// ---------------------------------------------------------------- columns
// Thread per V adjacent columns; the reduction walks stride xr.  Reductions of
// up to RREG rows stay in registers (raw storage), longer ones take three
// passes through the cache.
template <typename TI, typename TO, int V, int RREG, bool FAST>
__global__ __launch_bounds__(kThreads) void softmax_col_kernel(SoftmaxPlan p) {
  const uint32_t u = blockIdx.x * kThreads + threadIdx.x;
  if (u >= p.units) return;
  int64_t xo, oo;
  col_offsets(p, u * (uint32_t)V, xo, oo);
  const TI* xc = static_cast<const TI*>(p.x) + xo;
  TO* oc = static_cast<TO*>(p.out) + oo;
  struct alignas(V * sizeof(TI) >= 16 ? 16 : alignof(TI)) WI { TI e[V]; };
  struct alignas(V * sizeof(TO) >= 16 ? 16 : alignof(TO)) WO { TO e[V]; };
  float m[V], s[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    m[j] = -__builtin_inff();
    s[j] = 0.f;
  }
  if (p.R <= (uint32_t)RREG) {
    // rows past R re-read row R - 1 (unconditional loads keep every row in
    // flight) and are masked out below
    WI reg[RREG];
#pragma unroll
    for (int r = 0; r < RREG; ++r)
      reg[r] = *reinterpret_cast<const WI*>(xc + (int64_t)min((uint32_t)r, p.R - 1) * p.xr);
#pragma unroll
    for (int r = 0; r < RREG; ++r) {
      if (r < (int)p.R) {
#pragma unroll
        for (int j = 0; j < V; ++j) m[j] = max_nan(m[j], (float)reg[r].e[j]);
      }
    }
    if constexpr (V * RREG <= 32) {
      // few columns per thread: each exponential once, kept in registers;
      // fp16 outputs take e * (1/s), fp32 outputs e / s
      float e[RREG][V];
#pragma unroll
      for (int r = 0; r < RREG; ++r) {
#pragma unroll
        for (int j = 0; j < V; ++j) {
          e[r][j] = r < (int)p.R ? expd<FAST>((float)reg[r].e[j], m[j]) : 0.f;
          s[j] += e[r][j];
        }
      }
      float inv[V];
#pragma unroll
      for (int j = 0; j < V; ++j) inv[j] = 1.0f / s[j];
#pragma unroll
      for (int r = 0; r < RREG; ++r) {
        if (r < (int)p.R) {
          WO w;
#pragma unroll
          for (int j = 0; j < V; ++j) w.e[j] = (TO)(FAST ? e[r][j] * inv[j] : e[r][j] / s[j]);
          *reinterpret_cast<WO*>(oc + r * p.orr) = w;
        }
      }
      return;
    }
#pragma unroll
    for (int r = 0; r < RREG; ++r) {
      if (r < (int)p.R) {
#pragma unroll
        for (int j = 0; j < V; ++j) s[j] += expd<FAST>((float)reg[r].e[j], m[j]);
      }
    }
#pragma unroll
    for (int r = 0; r < RREG; ++r) {
      if (r < (int)p.R) {
        WO w;
#pragma unroll
        for (int j = 0; j < V; ++j) w.e[j] = (TO)(expd<FAST>((float)reg[r].e[j], m[j]) / s[j]);
        *reinterpret_cast<WO*>(oc + r * p.orr) = w;
      }
    }
    return;
  }
  // longer columns: three passes, each over the rows eight at a time with
  // all eight loads (clamped into the column) issued before the first is
  // used, the rows then taken in order
  constexpr uint32_t B = 8;
  auto pass = [&](auto&& f) {
    for (uint32_t r0 = 0; r0 < p.R; r0 += B) {
      WI w[B];
#pragma unroll
      for (uint32_t k = 0; k < B; ++k) w[k] = *reinterpret_cast<const WI*>(xc + (int64_t)min(r0 + k, p.R - 1) * p.xr);
#pragma unroll
      for (uint32_t k = 0; k < B; ++k)
        if (r0 + k < p.R) f(r0 + k, w[k]);
    }
  };
  pass([&](uint32_t, const WI& w) {
#pragma unroll
    for (int j = 0; j < V; ++j) m[j] = max_nan(m[j], (float)w.e[j]);
  });
  pass([&](uint32_t, const WI& w) {
#pragma unroll
    for (int j = 0; j < V; ++j) s[j] += expd<FAST>((float)w.e[j], m[j]);
  });
  pass([&](uint32_t r, const WI& w) {
    WO o;
#pragma unroll
    for (int j = 0; j < V; ++j) o.e[j] = (TO)(expd<FAST>((float)w.e[j], m[j]) / s[j]);
    *reinterpret_cast<WO*>(oc + (int64_t)r * p.orr) = o;
  });
}

// Long columns (R > 16) when there are too few column units to fill the chip
// with one thread per unit: a block takes kSplitUnits adjacent units (V
// columns each) and splits their rows over kSplitSlices slices, thread
// (slice s, unit g) taking rows s, s + kSplitSlices, ...  A row's eight units
// are then 8 x 16 bytes side by side.  Per-slice maxima and sums meet in LDS
// (the sums added in slice order); exp(x - max) / sum as the column kernel.
constexpr uint32_t kSplitUnits = 8, kSplitSlices = kThreads / kSplitUnits;
// Below this many units the split form is taken: one thread per unit would
// give fewer than 256 blocks of kThreads.
constexpr uint32_t kSplitMin = 256 * kThreads;
template <typename TI, typename TO, int V, bool FAST>
__global__ __launch_bounds__(kThreads) void softmax_col_split_kernel(SoftmaxPlan p) {
  constexpr uint32_t C = kSplitUnits * V;  // columns of the block
  __shared__ float part[kSplitSlices][C + 1];
  __shared__ float col_max[C], col_sum[C];
  const uint32_t g = threadIdx.x % kSplitUnits, sl = threadIdx.x / kSplitUnits;
  const uint32_t unit = blockIdx.x * kSplitUnits + g;
  const bool live = unit < p.units;
  int64_t xo, oo;
  col_offsets(p, min(unit, p.units - 1) * (uint32_t)V, xo, oo);
  const TI* xc = static_cast<const TI*>(p.x) + xo;
  TO* oc = static_cast<TO*>(p.out) + oo;
  struct alignas(V * sizeof(TI) >= 16 ? 16 : alignof(TI)) WI { TI e[V]; };
  struct alignas(V * sizeof(TO) >= 16 ? 16 : alignof(TO)) WO { TO e[V]; };
  // one pass over the slice's rows, eight at a time: all eight loads
  // (clamped into the column) issued before the first is used
  constexpr uint32_t B = 8;
  auto pass = [&](auto&& f) {
    for (uint32_t r0 = sl; r0 < p.R; r0 += B * kSplitSlices) {
      WI w[B];
#pragma unroll
      for (uint32_t k = 0; k < B; ++k)
        w[k] = *reinterpret_cast<const WI*>(xc + (int64_t)min(r0 + k * kSplitSlices, p.R - 1) * p.xr);
#pragma unroll
      for (uint32_t k = 0; k < B; ++k)
        if (r0 + k * kSplitSlices < p.R) f(r0 + k * kSplitSlices, w[k]);
    }
  };
  float m[V], s[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    m[j] = -__builtin_inff();
    s[j] = 0.f;
  }
  pass([&](uint32_t, const WI& w) {
#pragma unroll
    for (int j = 0; j < V; ++j) m[j] = max_nan(m[j], (float)w.e[j]);
  });
#pragma unroll
  for (int j = 0; j < V; ++j) part[sl][g * V + j] = m[j];
  __syncthreads();
  if (threadIdx.x < C) {
    float t = part[0][threadIdx.x];
    for (uint32_t q = 1; q < kSplitSlices; ++q) t = max_nan(t, part[q][threadIdx.x]);
    col_max[threadIdx.x] = t;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < V; ++j) m[j] = col_max[g * V + j];
  pass([&](uint32_t, const WI& w) {
#pragma unroll
    for (int j = 0; j < V; ++j) s[j] += expd<FAST>((float)w.e[j], m[j]);
  });
#pragma unroll
  for (int j = 0; j < V; ++j) part[sl][g * V + j] = s[j];
  __syncthreads();
  if (threadIdx.x < C) {
    float t = 0.f;
    for (uint32_t q = 0; q < kSplitSlices; ++q) t += part[q][threadIdx.x];
    col_sum[threadIdx.x] = t;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < V; ++j) s[j] = col_sum[g * V + j];
  if (!live) return;
  pass([&](uint32_t r, const WI& w) {
    WO o;
#pragma unroll
    for (int j = 0; j < V; ++j) o.e[j] = (TO)(expd<FAST>((float)w.e[j], m[j]) / s[j]);
    *reinterpret_cast<WO*>(oc + (int64_t)r * p.orr) = o;
  });
}

// Short fp16 column reductions (R <= 16 rows) over 16-byte column groups: the
// DFL bin softmax over the [B,16,4,A] view (R = 16 rows at stride A).  A unit
// is eight adjacent columns; SPLIT lanes share a unit, each holding 16/SPLIT
// of its rows as one 16-byte load per row, so a load instruction moves
// 64/SPLIT units (1 KB / SPLIT) of SPLIT rows.  The column max travels between
// the lanes of a unit by xor shuffles.  The sum is taken in row order: part q
// adds its rows to the running sum it receives from part q-1, and the total
// is broadcast back.  That is the column kernel's arithmetic term for term
// (e = exp(x - max), sums in row order, e * (1/s) for fp16 output, expf and
// e / s for fp32 output), so both kernels give the same bits.  The column max
// only stabilises the exponentials: a packed fp16 maximum that skips NaN
// still leaves a NaN column all NaN (its e and so its sum are NaN), as on CPU.
//
// LOOP: each wave walks its units with a grid stride and loads its next units
// before it computes and stores the current ones, so HBM reads, the
// exponentials and the stores of different rounds overlap instead of every
// wave of a single-round launch loading, computing and storing in lockstep.
// Without LOOP the grid covers every unit once (small launches).
template <typename TO, bool FAST, bool NT, int SPLIT, bool LOOP, bool R16>
__global__ __launch_bounds__(kThreads) void softmax_cols8_kernel(SoftmaxPlan p) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  typedef float f4 __attribute__((ext_vector_type(4)));
  constexpr int RP = 16 / SPLIT;            // rows per lane
  constexpr uint32_t kSlots = 64 / SPLIT;   // units per wave and round
  const uint32_t lane = threadIdx.x & 63u, part = lane / kSlots, slot = lane % kSlots;
  const uint32_t row0 = part * RP;
  const uint32_t R = R16 ? 16u : p.R;  // R16: every row of every lane is live (no masks)
  const uint32_t stride = gridDim.x * kWaves * kSlots;
  // Blocks are dealt to the 8 XCDs round robin; block b runs as logical block
  // (b % 8) * (grid / 8) + b / 8, so each XCD walks one contiguous run of
  // units and the 128-byte lines that neighbouring units share in a row stay
  // in one L2.  The grid is a multiple of 8.
  const uint32_t logical = (blockIdx.x & 7u) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  uint32_t base = (logical * kWaves + (threadIdx.x >> 6)) * kSlots;  // wave-uniform
  // the plan fields of the first two column dims in registers before the
  // bounds tests: one round of scalar loads (one asm statement: each is a
  // scheduling boundary)
  __asm__ volatile("" ::"s"(p.x), "s"(p.out), "s"(p.xr), "s"(p.orr), "s"(p.units), "s"(p.nd), "s"(p.div[0].mul),
                   "s"(p.div[0].shr), "s"(p.size[0]), "s"(p.xs[0]), "s"(p.os[0]), "s"(p.div[1].mul),
                   "s"(p.div[1].shr), "s"(p.size[1]), "s"(p.xs[1]), "s"(p.os[1]));
  if (base >= p.units) return;

  auto load = [&](uint32_t u, h8 (&v)[RP]) {
    if (u < p.units) {
      int64_t xo, oo;
      col_offsets(p, u * 8u, xo, oo);
      const _Float16* xc = static_cast<const _Float16*>(p.x) + xo;
#pragma unroll
      for (int i = 0; i < RP; ++i) {
        // rows past R re-read row R - 1 (every load stays unconditional) and are masked below
        const u4* src = reinterpret_cast<const u4*>(xc + (int64_t)(R16 ? row0 + i : min(row0 + i, R - 1)) * p.xr);
        v[i] = __builtin_bit_cast(h8, NT ? __builtin_nontemporal_load(src) : *src);
      }
    } else {
#pragma unroll
      for (int i = 0; i < RP; ++i) v[i] = (h8)(_Float16)0;
    }
  };

  h8 cur[RP], nxt[RP];
  load(base + slot, cur);
  for (;;) {
    const uint32_t next = base + stride;
    if (LOOP && next < p.units) load(next + slot, nxt);
    const uint32_t u = base + slot;
    // column max over this lane's rows, then across the unit's lanes
    h8 mh = (h8)(_Float16)(-__builtin_inff());
#pragma unroll
    for (int i = 0; i < RP; ++i)
      if (R16 || row0 + i < R) mh = __builtin_elementwise_max(mh, cur[i]);
#pragma unroll
    for (uint32_t o = kSlots; o < 64; o <<= 1) {
      u4 w = __builtin_bit_cast(u4, mh), t;
#pragma unroll
      for (int q = 0; q < 4; ++q) t[q] = (uint32_t)__shfl_xor((int)w[q], (int)o, 64);
      mh = __builtin_elementwise_max(mh, __builtin_bit_cast(h8, t));
    }
    float m[8], e[RP][8], s[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      m[j] = (float)mh[j];
      s[j] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < RP; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) e[i][j] = R16 || row0 + i < R ? expd<FAST>((float)cur[i][j], m[j]) : 0.f;
    // running sum in row order: part q continues the sum of part q - 1
#pragma unroll
    for (uint32_t q = 0; q < (uint32_t)SPLIT; ++q) {
      if (part == q) {
#pragma unroll
        for (int i = 0; i < RP; ++i)
#pragma unroll
          for (int j = 0; j < 8; ++j) s[j] += e[i][j];
      }
      const uint32_t from = slot + (q + 1 < (uint32_t)SPLIT ? q : (uint32_t)SPLIT - 1) * kSlots;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float t = __shfl(s[j], (int)from, 64);
        if (part == q + 1 || q + 1 == (uint32_t)SPLIT) s[j] = t;
      }
    }
    float inv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) inv[j] = 1.0f / s[j];
    if (u < p.units) {
      int64_t xo, oo;
      col_offsets(p, u * 8u, xo, oo);
      TO* oc = static_cast<TO*>(p.out) + oo;
#pragma unroll
      for (int i = 0; i < RP; ++i) {
        if (R16 || row0 + i < R) {
          u4* dst = reinterpret_cast<u4*>(oc + (int64_t)(row0 + i) * p.orr);
          u4 w[sizeof(TO) / 2];
          if constexpr (sizeof(TO) == 2) {
            h8 o;
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = (_Float16)(FAST ? e[i][j] * inv[j] : e[i][j] / s[j]);
            w[0] = __builtin_bit_cast(u4, o);
          } else {
            f4 lo, hi;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              lo[j] = FAST ? e[i][j] * inv[j] : e[i][j] / s[j];
              hi[j] = FAST ? e[i][4 + j] * inv[4 + j] : e[i][4 + j] / s[4 + j];
            }
            w[0] = __builtin_bit_cast(u4, lo);
            w[1] = __builtin_bit_cast(u4, hi);
          }
#pragma unroll
          for (int q = 0; q < (int)(sizeof(TO) / 2); ++q) {
            if constexpr (NT) __builtin_nontemporal_store(w[q], dst + q);
            else dst[q] = w[q];
          }
        }
      }
    }
    if (!LOOP || next >= p.units) break;
#pragma unroll
    for (int i = 0; i < RP; ++i) cur[i] = nxt[i];
    base = next;
  }
}

// ---------------------------------------------------------------- DFL
// out[n,s,a] = sum_i i * softmax_i(x[n, 16s+i, a]) for V adjacent anchors.
struct DflPlan {
  const _Float16* x;
  void* out;
  int64_t xn, xc, xa;   // element strides of x [N, 64, A]
  int64_t on, os, oa;   // element strides of out [N, 4, A]
  uint32_t sides;       // N * 4
  uint32_t avecs;       // A / V
  uint32_t units;       // sides * avecs
  FastDiv div_avecs;
  uint32_t x_bytes;     // byte extent of x from its base (32-bit offset form)
};

// Thread per V (1 or 2) adjacent anchors of one box side; the math is
// dev::dfl_side (shared with the detect-decode kernel, so both give the same
// bits).
// LOAD 0: 64-bit pointers.  LOAD 1/2: every byte offset into x fits 32 bits
// (non-negative strides), so the bins are read through a buffer resource over
// x_bytes, and every element offset into out fits 32 bits; 2 adds streaming
// loads and stores (launches of at least kStreamingBytes).  The 32-bit output
// offset and the streaming store took [32,64,8400] from 8.11 to 7.85 us.
template <typename TO, int V, bool FAST, int LOAD>
__global__ __launch_bounds__(kThreads) void dfl_expect_kernel(DflPlan p) {
  static_assert(V == 1 || V == 2, "one or two anchors per thread");
  // threads past the end recompute the last unit and store nothing: no
  // early exit, so the plan's scalar loads all go out in one round
  const uint32_t u0 = blockIdx.x * kThreads + threadIdx.x, u = min(u0, p.units - 1);
  const uint32_t side = p.div_avecs.div(u);
  const uint32_t a0 = (u - side * p.avecs) * V;
  const uint32_t n = side >> 2, sd = side & 3u;
  _Float16 bins[16][V];
  if constexpr (LOAD > 0) {
    const uint32_t off = 2u * (n * (uint32_t)p.xn + sd * 16u * (uint32_t)p.xc + a0 * (uint32_t)p.xa);
    dev::dfl_load_buffer<V, LOAD == 2>(dev::buffer_rsrc(p.x, p.x_bytes), off, 2u * (uint32_t)p.xc, bins);
  } else {
    const uint64_t off = 2 * (uint64_t)(n * p.xn + (int64_t)(sd * 16) * p.xc + (int64_t)a0 * p.xa);
    dev::dfl_load<V>(reinterpret_cast<const char*>(p.x), off, 2 * (uint64_t)p.xc, bins);
  }
  float r[V];
  dev::dfl_side<V, FAST>(bins, r);
  if (u0 >= p.units) return;
  TO* op = static_cast<TO*>(p.out);
  if constexpr (LOAD > 0) op += n * (uint32_t)p.on + sd * (uint32_t)p.os + a0 * (uint32_t)p.oa;
  else op += n * p.on + (int64_t)sd * p.os + (int64_t)a0 * p.oa;
  if constexpr (V == 2) {
    typedef TO ov __attribute__((ext_vector_type(2)));
    const ov v = {(TO)r[0], (TO)r[1]};
    if constexpr (LOAD == 2) __builtin_nontemporal_store(v, reinterpret_cast<ov*>(op));
    else *reinterpret_cast<ov*>(op) = v;
  } else {
    if constexpr (LOAD == 2) __builtin_nontemporal_store((TO)r[0], op);
    else op[0] = (TO)r[0];
  }
}

// Anchor-major logits (bin stride 1, anchor rows of 64 bins, the layout of
// a channels-last head seen as [N,64,A]): a thread per (anchor, side), side
// fastest, reads its 16 bins as two 16-byte loads, so four threads read an
// anchor's 128 bytes together; units = N * A * 4, div_avecs divides by A.
// The math is dev::dfl_side<1> (the one-anchor form's bits).
template <typename TO, bool FAST>
__global__ __launch_bounds__(kThreads) void dfl_expect_rows_kernel(DflPlan p) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  const uint32_t u0 = blockIdx.x * kThreads + threadIdx.x, u = min(u0, p.units - 1);
  const uint32_t sd = u & 3u, rest = u >> 2;
  const uint32_t n = p.div_avecs.div(rest), a = rest - n * p.avecs;
  const _Float16* src = p.x + (int64_t)n * p.xn + (int64_t)a * p.xa + sd * 16u;
  const h8 lo = *reinterpret_cast<const h8*>(src), hi = *reinterpret_cast<const h8*>(src + 8);
  _Float16 bins[16][1];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    bins[i][0] = lo[i];
    bins[8 + i][0] = hi[i];
  }
  float r[1];
  dev::dfl_side<1, FAST>(bins, r);
  if (u0 >= p.units) return;
  static_cast<TO*>(p.out)[(int64_t)n * p.on + (int64_t)sd * p.os + (int64_t)a * p.oa] = (TO)r[0];
}

// ---------------------------------------------------------------- detect decode
// Anchor-free detect head in one launch (whole_blocked.py:118-146):
//   distance = DFL(boxes)                      [B,4,A] fp16 (dev::dfl_side)
//   lower = anchor - distance[:, :2], upper = anchor + distance[:, 2:]
//   xyxy: (lower, upper) * stride;  xywh: ((lower+upper)/2, upper-lower) * stride
//   out = cat(boxes, sigmoid(scores))          [B,4+nc,A] fp16
// Each arithmetic step is one correctly rounded fp16 operation, as the
// reference's fp16 tensor ops are.  Anchors are the per-level grid cell
// centres (x + 0.5, y + 0.5) in fp16, anchor index = level start + y*w + x.
// Blocks [0, box_blocks) decode boxes: a thread takes one axis (x or y) of V
// adjacent anchors and so the box sides axis and axis+2.  The remaining blocks
// apply the sigmoid to the class logits, 8 per thread when rows are aligned.
constexpr int kMaxLevels = 8;

struct DecodePlan {
  const _Float16* boxes;  // [B,64,A] DFL logits, or [B,4,A] distances (direct)
  const _Float16* scores; // [B,nc,A]
  _Float16* out;          // [B,4+nc,A]
  int64_t bb, bc, ba, sb, sc, sa, ob, oc, oa;  // element strides
  uint32_t levels;
  uint32_t start[kMaxLevels + 1];
  FastDiv width[kMaxLevels];
  uint16_t stride_bits[kMaxLevels];  // fp16 stride per level
  uint32_t apairs;        // A / VB
  uint32_t box_units;     // B * 2 * apairs
  uint32_t box_blocks;
  uint32_t nc;
  uint32_t svecs;         // A / VS
  uint32_t score_units;   // B * nc * svecs
  FastDiv div_apairs, div_svecs, div_nc;
  int32_t xywh;
  uint32_t boxes_bytes;   // byte extent of boxes from its base (buffer-load forms)
  int32_t direct;         // boxes are the distances themselves (reg_max = 1 heads)
};

__device__ __forceinline__ _Float16 h_from_bits(uint16_t b) { return __builtin_bit_cast(_Float16, b); }

// Score vectors per thread: two for the 16-byte form (as the other streaming
// kernels, which measured best with two), one element otherwise.
template <int VS>
constexpr uint32_t kDecodeScoreUnits = VS == 8 ? 2u : 1u;

// LOAD 0: 64-bit pointers.  LOAD 1/2: box offsets fit 32 bits and the bins
// are read through a buffer resource; 2 also streams the score loads and the
// output stores (launches of at least kStreamingBytes).
template <int VB, int VS, int LOAD>
__global__ __launch_bounds__(kThreads) void detect_decode_kernel(DecodePlan p) {
  // Both roles' plan fields in registers before the test of the role: they
  // then load in the same round of scalar loads as p.box_blocks, not in two
  // or three more behind it.  (One statement: each inline asm is a
  // scheduling boundary of its own.)
  __asm__ volatile("" ::"s"(p.scores), "s"(p.out), "s"(p.sb), "s"(p.sc), "s"(p.sa), "s"(p.ob), "s"(p.oc),
                   "s"(p.oa), "s"(p.score_units), "s"(p.svecs), "s"(p.nc), "s"(p.div_svecs.mul),
                   "s"(p.div_svecs.shr), "s"(p.div_nc.mul), "s"(p.div_nc.shr), "s"(p.box_blocks), "s"(p.boxes),
                   "s"(p.bb), "s"(p.bc), "s"(p.ba), "s"(p.boxes_bytes), "s"(p.box_units), "s"(p.apairs),
                   "s"(p.div_apairs.mul), "s"(p.div_apairs.shr), "s"(p.xywh), "s"(p.levels), "s"(p.direct));
  if (blockIdx.x < p.box_blocks) {
    const uint32_t u = blockIdx.x * kThreads + threadIdx.x;
    if (u >= p.box_units) return;
    const uint32_t ba_ = p.div_apairs.div(u);          // b * 2 + axis
    const uint32_t a0 = (u - ba_ * p.apairs) * VB;
    const uint32_t b = ba_ >> 1, axis = ba_ & 1u;
    // Both sides' bins are loaded before either is reduced, and the anchors'
    // level, centre and stride (plan fields only) are worked out under those
    // loads: one memory round trip per thread instead of two, and the level
    // search off the path after it.
    _Float16 bins[16][VB], bins_hi[16][VB];
    float lo[VB], hi[VB];
    if (p.direct) {
      // distances as they are: the lt / rb channels of this axis
      const _Float16* xc = p.boxes + b * p.bb + (int64_t)a0 * p.ba;
      if constexpr (VB == 2) {  // anchor pairs are 4-byte aligned here (host checks)
        typedef _Float16 hv __attribute__((ext_vector_type(2)));
        const hv l = *reinterpret_cast<const hv*>(xc + (int64_t)axis * p.bc);
        const hv h = *reinterpret_cast<const hv*>(xc + (int64_t)(axis + 2) * p.bc);
        lo[0] = (float)l[0];
        lo[1] = (float)l[1];
        hi[0] = (float)h[0];
        hi[1] = (float)h[1];
      } else {
        lo[0] = (float)xc[(int64_t)axis * p.bc];
        hi[0] = (float)xc[(int64_t)(axis + 2) * p.bc];
      }
    } else if constexpr (LOAD > 0) {
      const __amdgpu_buffer_rsrc_t rs = dev::buffer_rsrc(p.boxes, p.boxes_bytes);
      const uint32_t bc = 2u * (uint32_t)p.bc;
      const uint32_t off = 2u * (b * (uint32_t)p.bb + a0 * (uint32_t)p.ba) + axis * 16u * bc;
      dev::dfl_load_buffer<VB, LOAD == 2>(rs, off, bc, bins);
      dev::dfl_load_buffer<VB, LOAD == 2>(rs, off + 32u * bc, bc, bins_hi);
    } else {
      const char* xc = reinterpret_cast<const char*>(p.boxes + b * p.bb + (int64_t)a0 * p.ba);
      dev::dfl_load<VB>(xc, 2 * (uint64_t)((int64_t)(axis * 16) * p.bc), 2 * (uint64_t)p.bc, bins);
      dev::dfl_load<VB>(xc, 2 * (uint64_t)((int64_t)((axis + 2) * 16) * p.bc), 2 * (uint64_t)p.bc, bins_hi);
    }
    _Float16 centre[VB], stride[VB];
#pragma unroll
    for (int j = 0; j < VB; ++j) {
      const uint32_t a = a0 + j;
      uint32_t l = 0;
      while (l + 1 < p.levels && a >= p.start[l + 1]) ++l;
      const uint32_t local = a - p.start[l];
      const uint32_t y = p.width[l].div(local), x = local - y * p.width[l].d;
      centre[j] = (_Float16)(float)(axis ? y : x) + (_Float16)0.5f;
      stride[j] = h_from_bits(p.stride_bits[l]);
    }
    if (!p.direct) {
      dev::dfl_side<VB, true>(bins, lo);
      dev::dfl_side<VB, true>(bins_hi, hi);
    }
    _Float16 first[VB], second[VB];
#pragma unroll
    for (int j = 0; j < VB; ++j) {
      const _Float16 lower = centre[j] - (_Float16)lo[j];
      const _Float16 upper = centre[j] + (_Float16)hi[j];
      if (p.xywh) {
        first[j] = ((lower + upper) / (_Float16)2.0f) * stride[j];
        second[j] = (upper - lower) * stride[j];
      } else {
        first[j] = lower * stride[j];
        second[j] = upper * stride[j];
      }
    }
    _Float16* o = p.out + b * p.ob + (int64_t)a0 * p.oa;
    if constexpr (VB == 2) {
      typedef _Float16 hv __attribute__((ext_vector_type(2)));
      hv* o1 = reinterpret_cast<hv*>(o + (int64_t)axis * p.oc);
      hv* o2 = reinterpret_cast<hv*>(o + (int64_t)(axis + 2) * p.oc);
      if constexpr (LOAD == 2) {
        __builtin_nontemporal_store((hv){first[0], first[1]}, o1);
        __builtin_nontemporal_store((hv){second[0], second[1]}, o2);
      } else {
        *o1 = (hv){first[0], first[1]};
        *o2 = (hv){second[0], second[1]};
      }
    } else {
      o[(int64_t)axis * p.oc] = first[0];
      o[(int64_t)(axis + 2) * p.oc] = second[0];
    }
    return;
  }
  // scores: two 16-byte vectors per thread (both loads issued first), or one
  // element per thread in the unaligned form
  constexpr uint32_t SU = kDecodeScoreUnits<VS>;
  const uint32_t v0 = (blockIdx.x - p.box_blocks) * (kThreads * SU) + threadIdx.x;
  const _Float16* sp[SU];
  _Float16* op[SU];
#pragma unroll
  for (uint32_t s = 0; s < SU; ++s) {
    const uint32_t v = min(v0 + s * kThreads, p.score_units - 1);
    const uint32_t row = p.div_svecs.div(v);               // b * nc + c
    const uint32_t a0 = (v - row * p.svecs) * VS;
    const uint32_t b = p.div_nc.div(row), c = row - b * p.nc;
    sp[s] = p.scores + b * p.sb + (int64_t)c * p.sc + (int64_t)a0 * p.sa;
    op[s] = p.out + b * p.ob + (int64_t)(4 + c) * p.oc + (int64_t)a0 * p.oa;
  }
  if constexpr (VS == 8) {
    dev::h8 x[SU];
#pragma unroll
    for (uint32_t s = 0; s < SU; ++s) {
      const dev::h8* src = reinterpret_cast<const dev::h8*>(sp[s]);
      x[s] = LOAD == 2 ? __builtin_nontemporal_load(src) : *src;
    }
#pragma unroll
    for (uint32_t s = 0; s < SU; ++s) {
      if (v0 + s * kThreads >= p.score_units) break;
      dev::h8 y;
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = (_Float16)dev::sigmoid_fast((float)x[s][j]);
      if constexpr (LOAD == 2) __builtin_nontemporal_store(y, reinterpret_cast<dev::h8*>(op[s]));
      else *reinterpret_cast<dev::h8*>(op[s]) = y;
    }
  } else {
    if (v0 < p.score_units) op[0][0] = (_Float16)dev::sigmoid_fast((float)sp[0][0]);
  }
}

// ---------------------------------------------------------------- host

bool aligned(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

// Coalesces every dim except `dim` jointly for x and out (innermost-first into
// the plan).  Returns false if more than kMaxDims remain (cannot happen).
void column_space(const thin_desc* x, const thin_desc* out, int dim, SoftmaxPlan& p) {
  thin_desc xs = *x, os = *out;
  // drop the reduced dim
  int r = 0;
  for (int d = 0; d < x->rank; ++d) {
    if (d == dim) continue;
    xs.sizes[r] = x->sizes[d];
    xs.strides[r] = x->strides[d];
    os.sizes[r] = out->sizes[d];
    os.strides[r] = out->strides[d];
    ++r;
  }
  xs.rank = os.rank = r;
  const thin_desc* ops[2] = {&xs, &os};
  Coalesced c = coalesce(ops, 2);
  p.nd = c.nd;
  for (int i = 0; i < c.nd; ++i) {
    const int s = c.nd - 1 - i;
    p.size[i] = (uint32_t)c.size[s];
    p.div[i] = FastDiv::make((uint32_t)c.size[s]);
    p.xs[i] = c.stride[0][s];
    p.os[i] = c.stride[1][s];
  }
}

// Streaming (non-temporal) loads and stores for launches moving at least
// kStreamingBytes.

}  // namespace

// Lanes per row G and chunks per lane KPT of the row kernel for `rows` rows of
// `chunks` (<= 512) chunks each.  The fused attention kernel takes its softmax
// tree from here too, so both give the same bits.
RowTree row_tree(int64_t chunks, uint64_t rows) {
  auto blocks = [&](int g) { return (rows + (uint64_t)kWaves * (64 / g) - 1) / ((uint64_t)kWaves * (64 / g)); };
  if (chunks <= 2) return {1, 2};
  if (chunks <= 4) return {2, 2};
  if (chunks <= 8) return {4, 2};
  if (chunks <= 16) return {8, 2};
  if (chunks <= 32) return {16, 2};
  if (chunks <= 64 && blocks(32) < 256) return {64, 1};  // few rows: one row per wave, more waves
  if (chunks <= 64) return {32, 2};
  if (chunks <= 128) return {64, 2};
  if (chunks <= 256) return {64, 4};
  return {64, 8};
}

namespace {

template <typename TI, typename TO, bool VEC, bool FAST, bool NT>
void launch_rows(const SoftmaxPlan& p, int64_t chunks, uint64_t rows, hipStream_t stream) {
  auto grid = [&](int g) { return (uint32_t)((rows + (uint64_t)kWaves * (64 / g) - 1) / ((uint64_t)kWaves * (64 / g))); };
#define THIN_ROWG(G, K) hipLaunchKernelGGL((softmax_row_kernel<TI, TO, VEC, G, K, FAST, NT>), dim3(grid(G)), \
                                           dim3(kThreads), 0, stream, p)
  const RowTree t = row_tree(chunks, rows);
  switch (t.lanes * 16 + t.chunks_per_lane) {
    case 1 * 16 + 2: THIN_ROWG(1, 2); break;
    case 2 * 16 + 2: THIN_ROWG(2, 2); break;
    case 4 * 16 + 2: THIN_ROWG(4, 2); break;
    case 8 * 16 + 2: THIN_ROWG(8, 2); break;
    case 16 * 16 + 2: THIN_ROWG(16, 2); break;
    case 64 * 16 + 1: THIN_ROWG(64, 1); break;
    case 32 * 16 + 2: THIN_ROWG(32, 2); break;
    case 64 * 16 + 2: THIN_ROWG(64, 2); break;
    case 64 * 16 + 4: THIN_ROWG(64, 4); break;
    default: THIN_ROWG(64, 8); break;
  }
#undef THIN_ROWG
}

// Units of eight columns per lane group.  Launches of at least 65536 units
// (the DFL bin softmax at N=32: 134400) run two lanes per unit in a 512-block
// grid-stride loop (8 waves per CU, about two rounds each); smaller ones run
// four lanes per unit, one round, for more waves in flight.  Measured on the
// [32,16,4,8400] view: 14.9 us (16.8 with the two-column kernel), which is the
// time of a plain 16-byte copy with the same sixteen-rows-per-unit access
// pattern (14.8 us); a linear copy of the same bytes takes 12.6 us.
constexpr uint32_t kCols8Blocks = 512;

template <typename TO, bool FAST>
void launch_cols8(const SoftmaxPlan& p, bool nt, hipStream_t stream) {
  const bool wide = p.units >= 32u * kCols8Blocks * kWaves;
  const uint32_t per_block = (wide ? 32u : 16u) * kWaves;
  const uint32_t grid = wide ? kCols8Blocks : ((p.units + per_block - 1) / per_block + 7u) / 8u * 8u;
#define THIN_COLS8(NT, SPLIT, LOOP, R16) \
  hipLaunchKernelGGL((softmax_cols8_kernel<TO, FAST, NT, SPLIT, LOOP, R16>), dim3(grid), dim3(kThreads), 0, stream, p)
#define THIN_COLS8_R(NT, SPLIT, LOOP) \
  if (p.R == 16) THIN_COLS8(NT, SPLIT, LOOP, true); else THIN_COLS8(NT, SPLIT, LOOP, false)
  if (wide) {
    if (nt) { THIN_COLS8_R(true, 2, true); }
    else { THIN_COLS8_R(false, 2, true); }
  } else {
    if (nt) { THIN_COLS8_R(true, 4, false); }
    else { THIN_COLS8_R(false, 4, false); }
  }
#undef THIN_COLS8_R
#undef THIN_COLS8
}

template <typename TI, typename TO, bool FAST>
thin_status launch_softmax(const thin_desc* x, int dim, const thin_desc* out, hipStream_t stream) {
  SoftmaxPlan p;
  memset(&p, 0, sizeof p);
  p.x = x->data;
  p.out = out->data;
  const int64_t R = x->rank ? x->sizes[dim] : 1;
  p.R = (uint32_t)R;
  if (x->rank == 0) {
    p.nd = 1;
    p.size[0] = 1;
    p.div[0] = FastDiv::make(1);
    p.xr = p.orr = 1;
  } else {
    column_space(x, out, dim, p);
    p.xr = x->strides[dim];
    p.orr = out->strides[dim];
  }
  uint64_t cols = 1;
  for (int i = 0; i < p.nd; ++i) cols *= p.size[i];
  THIN_REQUIRE(cols < (1ull << 31) && R < (1ll << 31), THIN_ERR_UNSUPPORTED, "softmax: tensor too large");
  const bool rowform = R == 1 || (p.xr == 1 && p.orr == 1);
  if (rowform) {
    p.xr = p.orr = 1;
    p.units = (uint32_t)cols;
    constexpr int VE = 16 / (int)sizeof(TI);
    bool vec = R % VE == 0 && aligned(x->data, 16) && aligned(out->data, 16);
    for (int i = 0; vec && i < p.nd; ++i)
      vec = (p.xs[i] * (int64_t)sizeof(TI)) % 16 == 0 && (p.os[i] * (int64_t)sizeof(TO)) % 16 == 0;
    const int64_t chunks = vec ? R / VE : R;
    const bool nt = vec && (int64_t)cols * R * (int64_t)(sizeof(TI) + sizeof(TO)) >= kStreamingBytes;
    if (chunks > 512) {
      hipLaunchKernelGGL((softmax_row_stream_kernel<TI, TO, FAST>), dim3((uint32_t)cols), dim3(kThreads), 0, stream,
                         p);
    } else if (vec) {
      if (nt) launch_rows<TI, TO, true, FAST, true>(p, chunks, cols, stream);
      else launch_rows<TI, TO, true, FAST, false>(p, chunks, cols, stream);
    } else {
      launch_rows<TI, TO, false, FAST, false>(p, chunks, cols, stream);
    }
    THIN_LAUNCH_CHECK("softmax_row");
    return THIN_OK;
  }
  constexpr int V = 16 / (int)sizeof(TI);
  bool vec = p.nd >= 1 && p.xs[0] == 1 && p.os[0] == 1 && p.size[0] % V == 0 && aligned(x->data, 16) &&
             aligned(out->data, V * sizeof(TO) >= 16 ? 16 : sizeof(TO)) &&
             (p.xr * (int64_t)sizeof(TI)) % 16 == 0 && (p.orr * (int64_t)sizeof(TO)) % (V * sizeof(TO) >= 16 ? 16 : 1) == 0;
  for (int i = 1; vec && i < p.nd; ++i)
    vec = (p.xs[i] * (int64_t)sizeof(TI)) % 16 == 0 && (p.os[i] * (int64_t)sizeof(TO)) % 16 == 0;
  // short fp16 columns (the DFL bin softmax over [B,16,4,A], R = 16): two
  // columns per thread keep every exponential in registers and many waves in
  // flight ([32,16,4,8400]: 16.8 us; 19.3 us with four columns per thread and
  // their exponentials kept, 37 us with eight; streaming loads and stores
  // measured the same 16.8 us)
  // Eight fp16 columns per thread through 16-byte accesses when every row
  // and column group is 16-byte aligned (the DFL view with A % 8 == 0).
  bool oct = sizeof(TI) == 2 && R <= 16 && p.nd >= 1 && p.xs[0] == 1 && p.os[0] == 1 && p.size[0] % 8 == 0 &&
             aligned(x->data, 16) && aligned(out->data, 16) && p.xr % 8 == 0 && p.orr % 8 == 0;
  for (int i = 1; oct && i < p.nd; ++i) oct = p.xs[i] % 8 == 0 && p.os[i] % 8 == 0;
  bool pair = sizeof(TI) == 2 && R <= 16 && p.nd >= 1 && p.xs[0] == 1 && p.os[0] == 1 && p.size[0] % 2 == 0 &&
              aligned(x->data, 4) && aligned(out->data, 2 * sizeof(TO)) && p.xr % 2 == 0 && p.orr % 2 == 0;
  for (int i = 1; pair && i < p.nd; ++i) pair = p.xs[i] % 2 == 0 && p.os[i] % 2 == 0;
  if (oct) {
    p.units = (uint32_t)(cols / 8);
    const bool nt = (int64_t)cols * R * (int64_t)(sizeof(TI) + sizeof(TO)) >= kStreamingBytes;
    launch_cols8<TO, FAST>(p, nt, stream);
  } else if (pair) {
    p.units = (uint32_t)(cols / 2);
    const uint32_t grid = (p.units + kThreads - 1) / kThreads;
    hipLaunchKernelGGL((softmax_col_kernel<TI, TO, 2, 16, FAST>), dim3(grid), dim3(kThreads), 0, stream, p);
  } else if (vec) {
    p.units = (uint32_t)(cols / V);
    if (R > 16 && p.units < kSplitMin) {
      const uint32_t grid = (p.units + kSplitUnits - 1) / kSplitUnits;
      hipLaunchKernelGGL((softmax_col_split_kernel<TI, TO, V, FAST>), dim3(grid), dim3(kThreads), 0, stream, p);
    } else {
      const uint32_t grid = (p.units + kThreads - 1) / kThreads;
      hipLaunchKernelGGL((softmax_col_kernel<TI, TO, V, 16, FAST>), dim3(grid), dim3(kThreads), 0, stream, p);
    }
  } else {
    p.units = (uint32_t)cols;
    if (R > 32 && p.units < kSplitMin) {
      const uint32_t grid = (p.units + kSplitUnits - 1) / kSplitUnits;
      hipLaunchKernelGGL((softmax_col_split_kernel<TI, TO, 1, FAST>), dim3(grid), dim3(kThreads), 0, stream, p);
    } else {
      const uint32_t grid = (p.units + kThreads - 1) / kThreads;
      hipLaunchKernelGGL((softmax_col_kernel<TI, TO, 1, 32, FAST>), dim3(grid), dim3(kThreads), 0, stream, p);
    }
  }
  THIN_LAUNCH_CHECK("softmax_col");
  return THIN_OK;
}

}  // namespace
}  // namespace thin

using namespace thin;

extern "C" thin_status thin_softmax(const thin_desc* x, int32_t dim, const thin_desc* out, hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(desc_valid(x) && desc_valid(out), THIN_ERR_INVALID, "softmax: invalid descriptor");
  THIN_REQUIRE(same_sizes(x, out), THIN_ERR_INVALID, "softmax: output must have the input's sizes");
  THIN_REQUIRE(x->dtype == THIN_F16 || x->dtype == THIN_F32, THIN_ERR_INVALID, "softmax supports float32/float16");
  THIN_REQUIRE(out->dtype == x->dtype || (x->dtype == THIN_F16 && out->dtype == THIN_F32), THIN_ERR_INVALID,
               "softmax output dtype must equal the input's, or be float32 for float16 input (half_to_float)");
  THIN_REQUIRE(x->rank == 0 ? (dim == 0 || dim == -1) : (dim >= 0 && dim < x->rank), THIN_ERR_INVALID,
               "softmax: dim %d out of range", dim);
  if (numel(x) == 0) return THIN_OK;
  const int d = x->rank == 0 ? 0 : dim;
  if (x->dtype == THIN_F32) return launch_softmax<float, float, false>(x, d, out, stream);
  if (out->dtype == THIN_F32) return launch_softmax<_Float16, float, false>(x, d, out, stream);
  return launch_softmax<_Float16, _Float16, true>(x, d, out, stream);
}

extern "C" thin_status thin_dfl_expect(const thin_desc* x, const thin_desc* out, hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(desc_valid(x) && desc_valid(out), THIN_ERR_INVALID, "dfl_expect: invalid descriptor");
  THIN_REQUIRE(x->dtype == THIN_F16 && (out->dtype == THIN_F16 || out->dtype == THIN_F32), THIN_ERR_INVALID,
               "dfl_expect takes float16 logits and writes float16 or float32");
  THIN_REQUIRE(x->rank == 3 && x->sizes[1] == 64 && out->rank == 3 && out->sizes[0] == x->sizes[0] &&
               out->sizes[1] == 4 && out->sizes[2] == x->sizes[2], THIN_ERR_INVALID,
               "dfl_expect expects x [N,64,A] and out [N,4,A]");
  if (numel(out) == 0) return THIN_OK;
  DflPlan p;
  p.x = static_cast<const _Float16*>(x->data);
  p.out = out->data;
  p.xn = x->strides[0]; p.xc = x->strides[1]; p.xa = x->strides[2];
  p.on = out->strides[0]; p.os = out->strides[1]; p.oa = out->strides[2];
  const int64_t A = x->sizes[2];
  p.sides = (uint32_t)(x->sizes[0] * 4);
  const int esz = out->dtype == THIN_F32 ? 4 : 2;
  if (p.xc == 1 && p.xa % 8 == 0 && p.xn % 8 == 0 && aligned(x->data, 16) && p.xa >= 64) {
    // anchor-major bins: 16 -> 2 load instructions per (anchor, side) and
    // whole 128-byte anchor rows per four lanes ([32,64,8400] as the
    // transpose of [32,8400,64]: 111.6 us through the strided form)
    const uint64_t units = (uint64_t)p.sides * (uint64_t)A;
    THIN_REQUIRE(units < (1ull << 31), THIN_ERR_UNSUPPORTED, "dfl_expect: tensor too large");
    p.units = (uint32_t)units;
    p.avecs = (uint32_t)A;
    p.div_avecs = FastDiv::make(p.avecs);
    const uint32_t grid = (p.units + kThreads - 1) / kThreads;
    if (out->dtype == THIN_F16)
      hipLaunchKernelGGL((dfl_expect_rows_kernel<_Float16, true>), dim3(grid), dim3(kThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((dfl_expect_rows_kernel<float, false>), dim3(grid), dim3(kThreads), 0, stream, p);
    THIN_LAUNCH_CHECK("dfl_expect_rows");
    return THIN_OK;
  }
  // Two anchors per thread (4-byte loads): more waves than wider vectors, so
  // the 32 exponentials per thread overlap the loads of other waves.
  constexpr int V = 2;
  const bool vec = A % V == 0 && p.xa == 1 && p.oa == 1 && aligned(x->data, 2 * V) &&
                   aligned(out->data, esz * V) && p.xn % V == 0 && p.xc % V == 0 && p.on % V == 0 &&
                   p.os % V == 0;
  const int v = vec ? V : 1;
  p.avecs = (uint32_t)(A / v);
  const uint64_t units = (uint64_t)p.sides * p.avecs;
  THIN_REQUIRE(units < (1ull << 31), THIN_ERR_UNSUPPORTED, "dfl_expect: tensor too large");
  p.units = (uint32_t)units;
  p.div_avecs = FastDiv::make(p.avecs);
  const uint32_t grid = (p.units + kThreads - 1) / kThreads;
  // 32-bit byte offsets when the whole of x lies within 4 GiB of its base
  bool o32 = true;
  uint64_t extent = 2, out_extent = 1;
  for (int i = 0; i < 3; ++i) {
    if (x->strides[i] < 0 || out->strides[i] < 0) o32 = false;
    else {
      extent += 2 * (uint64_t)(x->sizes[i] - 1) * (uint64_t)x->strides[i];
      out_extent += (uint64_t)(out->sizes[i] - 1) * (uint64_t)out->strides[i];
    }
  }
  // and every element offset into out (the largest one plus a pair) fits 32 bits
  o32 = o32 && extent < (1ull << 32) && out_extent + 2 < (1ull << 32);
  p.x_bytes = o32 ? (uint32_t)extent : 0u;
  const bool nt = (int64_t)p.sides * 16 * A * 2 >= kStreamingBytes;
#define THIN_DFL(TO, VV, FAST)                                                                                    \
  do {                                                                                                            \
    if (o32 && nt) hipLaunchKernelGGL((dfl_expect_kernel<TO, VV, FAST, 2>), dim3(grid), dim3(kThreads), 0, stream, p); \
    else if (o32) hipLaunchKernelGGL((dfl_expect_kernel<TO, VV, FAST, 1>), dim3(grid), dim3(kThreads), 0, stream, p);  \
    else hipLaunchKernelGGL((dfl_expect_kernel<TO, VV, FAST, 0>), dim3(grid), dim3(kThreads), 0, stream, p);           \
  } while (0)
  if (out->dtype == THIN_F16) {
    if (vec) THIN_DFL(_Float16, V, true);
    else THIN_DFL(_Float16, 1, true);
  } else {
    if (vec) THIN_DFL(float, V, false);
    else THIN_DFL(float, 1, false);
  }
#undef THIN_DFL
  THIN_LAUNCH_CHECK("dfl_expect");
  return THIN_OK;
}

extern "C" thin_status thin_detect_decode(const thin_desc* boxes, const thin_desc* scores, const int32_t* level_hw,
                                          const double* level_stride, int32_t levels, int32_t xywh,
                                          const thin_desc* out, hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(desc_valid(boxes) && desc_valid(scores) && desc_valid(out), THIN_ERR_INVALID,
               "detect_decode: invalid descriptor");
  THIN_REQUIRE(boxes->dtype == THIN_F16 && scores->dtype == THIN_F16 && out->dtype == THIN_F16 &&
               boxes->rank == 3 && scores->rank == 3 && out->rank == 3, THIN_ERR_INVALID,
               "detect_decode takes float16 boxes [B,64,A] or [B,4,A], scores [B,nc,A] and out [B,4+nc,A]");
  const int64_t B = boxes->sizes[0], A = boxes->sizes[2], nc = scores->sizes[1];
  THIN_REQUIRE((boxes->sizes[1] == 64 || boxes->sizes[1] == 4) && scores->sizes[0] == B && scores->sizes[2] == A &&
               out->sizes[0] == B && out->sizes[1] == 4 + nc && out->sizes[2] == A, THIN_ERR_INVALID,
               "detect_decode expects boxes [B,64,A] or [B,4,A], scores [B,nc,A], out [B,4+nc,A]");
  THIN_REQUIRE(levels >= 1 && levels <= kMaxLevels && level_hw && level_stride, THIN_ERR_INVALID,
               "detect_decode takes 1..%d levels", kMaxLevels);
  DecodePlan p;
  memset(&p, 0, sizeof p);
  int64_t total = 0;
  for (int l = 0; l < levels; ++l) {
    THIN_REQUIRE(level_hw[2 * l] > 0 && level_hw[2 * l + 1] > 0, THIN_ERR_INVALID,
                 "detect_decode: level sizes must be positive");
    p.start[l] = (uint32_t)total;
    p.width[l] = FastDiv::make((uint32_t)level_hw[2 * l + 1]);
    const _Float16 st = (_Float16)(float)level_stride[l];
    p.stride_bits[l] = __builtin_bit_cast(uint16_t, st);
    total += (int64_t)level_hw[2 * l] * level_hw[2 * l + 1];
  }
  THIN_REQUIRE(total == A, THIN_ERR_INVALID, "detect_decode: level sizes cover %lld anchors, tensors have %lld",
               (long long)total, (long long)A);
  if (numel(out) == 0) return THIN_OK;
  p.start[levels] = (uint32_t)total;
  p.levels = (uint32_t)levels;
  p.boxes = static_cast<const _Float16*>(boxes->data);
  p.scores = static_cast<const _Float16*>(scores->data);
  p.out = static_cast<_Float16*>(out->data);
  p.bb = boxes->strides[0]; p.bc = boxes->strides[1]; p.ba = boxes->strides[2];
  p.sb = scores->strides[0]; p.sc = scores->strides[1]; p.sa = scores->strides[2];
  p.ob = out->strides[0]; p.oc = out->strides[1]; p.oa = out->strides[2];
  p.nc = (uint32_t)nc;
  p.xywh = xywh ? 1 : 0;
  p.direct = boxes->sizes[1] == 4 ? 1 : 0;
  const bool vb = A % 2 == 0 && p.ba == 1 && p.oa == 1 && aligned(boxes->data, 4) && aligned(out->data, 4) &&
                  p.bb % 2 == 0 && p.bc % 2 == 0 && p.ob % 2 == 0 && p.oc % 2 == 0;
  const bool vs = A % 8 == 0 && p.sa == 1 && p.oa == 1 && aligned(scores->data, 16) && aligned(out->data, 16) &&
                  p.sb % 8 == 0 && p.sc % 8 == 0 && p.ob % 8 == 0 && p.oc % 8 == 0;
  const int VB = vb ? 2 : 1, VS = vs ? 8 : 1;
  p.apairs = (uint32_t)(A / VB);
  const uint64_t box_units = (uint64_t)B * 2 * p.apairs;
  p.svecs = (uint32_t)(A / VS);
  const uint64_t score_units = (uint64_t)B * nc * p.svecs;
  THIN_REQUIRE(box_units < (1ull << 31) && score_units < (1ull << 31), THIN_ERR_UNSUPPORTED,
               "detect_decode: tensors too large");
  p.box_units = (uint32_t)box_units;
  p.score_units = (uint32_t)score_units;
  p.box_blocks = (uint32_t)((box_units + kThreads - 1) / kThreads);
  p.div_apairs = FastDiv::make(p.apairs);
  p.div_svecs = FastDiv::make(p.svecs);
  p.div_nc = FastDiv::make((uint32_t)nc);
  const uint32_t su = vs ? kDecodeScoreUnits<8> : kDecodeScoreUnits<1>;
  const uint32_t grid = p.box_blocks + (uint32_t)((score_units + kThreads * su - 1) / (kThreads * su));
  // 32-bit box offsets (buffer loads) when boxes lie within 4 GiB of their base
  bool o32 = true;
  uint64_t extent = 2;
  for (int i = 0; i < 3; ++i) {
    if (boxes->strides[i] < 0) o32 = false;
    else extent += 2 * (uint64_t)(boxes->sizes[i] - 1) * (uint64_t)boxes->strides[i];
  }
  o32 = o32 && extent < (1ull << 32);
  p.boxes_bytes = o32 ? (uint32_t)extent : 0u;
  const int load = !o32 ? 0 : numel(out) * 2 >= kStreamingBytes ? 2 : 1;
#define THIN_DECODE(B_, S_)                                                                                      \
  do {                                                                                                           \
    if (load == 2) hipLaunchKernelGGL((detect_decode_kernel<B_, S_, 2>), dim3(grid), dim3(kThreads), 0, stream, p); \
    else if (load == 1) hipLaunchKernelGGL((detect_decode_kernel<B_, S_, 1>), dim3(grid), dim3(kThreads), 0, stream, p); \
    else hipLaunchKernelGGL((detect_decode_kernel<B_, S_, 0>), dim3(grid), dim3(kThreads), 0, stream, p);           \
  } while (0)
  if (vb && vs) THIN_DECODE(2, 8);
  else if (vb) THIN_DECODE(2, 1);
  else if (vs) THIN_DECODE(1, 8);
  else THIN_DECODE(1, 1);
#undef THIN_DECODE
  THIN_LAUNCH_CHECK("detect_decode");
  return THIN_OK;
}
