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

__device__ __forceinline__ void col_offsets(const SoftmaxPlan& p, uint32_t e, int64_t& xo, int64_t& oo) {
  xo = 0;
  oo = 0;
#pragma unroll
  for (int d = 0; d < kMaxDims; ++d) {
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
template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, G));
  return v;
}
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, G);
  return v;
}

template <typename TI, typename TO, bool VEC, int G, int KPT, bool FAST, bool NT>
__global__ __launch_bounds__(kThreads) void softmax_row_kernel(SoftmaxPlan p) {
  constexpr int VE = VEC ? 16 / (int)sizeof(TI) : 1;
  constexpr int RPW = 64 / G;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t g = lane % G;
  const uint32_t row = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * RPW + lane / G;
  const bool live = row < p.units;  // every lane still joins the group shuffles
  int64_t xo = 0, oo = 0;
  if (live) col_offsets(p, row, xo, oo);
  const TI* xr = static_cast<const TI*>(p.x) + xo;
  TO* orow = static_cast<TO*>(p.out) + oo;
  const uint32_t chunks = VEC ? p.R / VE : p.R;
  struct alignas(VE * sizeof(TI)) WI { TI e[VE]; };
  WI raw[KPT];
  float m = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    const uint32_t c = g + G * k;
    if (live && c < chunks) {
      const WI* src = reinterpret_cast<const WI*>(xr) + c;
      if constexpr (VEC && NT) raw[k] = __builtin_bit_cast(WI, __builtin_nontemporal_load(
                                   reinterpret_cast<const uint32_t __attribute__((ext_vector_type(4)))*>(src)));
      else raw[k] = *src;
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
  float m = -__builtin_inff();
  for (uint32_t i = threadIdx.x; i < p.R; i += kThreads) m = max_nan(m, ldf(xr + i));
  m = wave_max_nan(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = red[0];
#pragma unroll
  for (uint32_t w = 1; w < kWaves; ++w) m = max_nan(m, red[w]);
  __syncthreads();
  float s = 0.f;
  for (uint32_t i = threadIdx.x; i < p.R; i += kThreads) s += expo<FAST>(ldf(xr + i) - m);
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  s = 0.f;
#pragma unroll
  for (uint32_t w = 0; w < kWaves; ++w) s += red[w];
  const float inv = 1.0f / s;
  for (uint32_t i = threadIdx.x; i < p.R; i += kThreads) stf(orow + i, expo<FAST>(ldf(xr + i) - m) * inv);
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
    WI reg[RREG];
#pragma unroll
    for (int r = 0; r < RREG; ++r) {
      if (r >= (int)p.R) continue;
      reg[r] = *reinterpret_cast<const WI*>(xc + r * p.xr);
#pragma unroll
      for (int j = 0; j < V; ++j) m[j] = max_nan(m[j], (float)reg[r].e[j]);
    }
#pragma unroll
    for (int r = 0; r < RREG; ++r) {
      if (r >= (int)p.R) continue;
#pragma unroll
      for (int j = 0; j < V; ++j) s[j] += expo<FAST>((float)reg[r].e[j] - m[j]);
    }
#pragma unroll
    for (int r = 0; r < RREG; ++r) {
      if (r >= (int)p.R) continue;
      WO w;
#pragma unroll
      for (int j = 0; j < V; ++j) w.e[j] = (TO)(expo<FAST>((float)reg[r].e[j] - m[j]) / s[j]);
      *reinterpret_cast<WO*>(oc + r * p.orr) = w;
    }
    return;
  }
  for (uint32_t r = 0; r < p.R; ++r) {
    WI w = *reinterpret_cast<const WI*>(xc + r * p.xr);
#pragma unroll
    for (int j = 0; j < V; ++j) m[j] = max_nan(m[j], (float)w.e[j]);
  }
  for (uint32_t r = 0; r < p.R; ++r) {
    WI w = *reinterpret_cast<const WI*>(xc + r * p.xr);
#pragma unroll
    for (int j = 0; j < V; ++j) s[j] += expo<FAST>((float)w.e[j] - m[j]);
  }
  for (uint32_t r = 0; r < p.R; ++r) {
    WI w = *reinterpret_cast<const WI*>(xc + r * p.xr);
    WO o;
#pragma unroll
    for (int j = 0; j < V; ++j) o.e[j] = (TO)(expo<FAST>((float)w.e[j] - m[j]) / s[j]);
    *reinterpret_cast<WO*>(oc + r * p.orr) = o;
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
};

// The bin maximum only stabilises the exponentials, so it is taken without
// NaN propagation (in packed fp16 for two anchors, where max is exact): a NaN
// bin, a +inf bin (inf - inf) or an all -inf side (-inf - -inf) already makes
// the sum, and so the result, NaN -- as CPU's softmax then expectation does.
// FAST (fp16 output): e = exp2(x*log2e - m*log2e) as one fma (an error in the
// common term m*log2e scales every e_i alike and cancels in w/s) and w * 1/s;
// the fp32 output uses expf and an IEEE division.
template <typename TO, int V, bool FAST>
__global__ __launch_bounds__(kThreads) void dfl_expect_kernel(DflPlan p) {
  static_assert(V == 1 || V == 2, "one or two anchors per thread");
  const uint32_t u = blockIdx.x * kThreads + threadIdx.x;
  if (u >= p.units) return;
  const uint32_t side = p.div_avecs.div(u);
  const uint32_t a0 = (u - side * p.avecs) * V;
  const uint32_t n = side >> 2, sd = side & 3u;
  const _Float16* xp = p.x + n * p.xn + (int64_t)(sd * 16) * p.xc + (int64_t)a0 * p.xa;
  typedef _Float16 hv __attribute__((ext_vector_type(2)));
  _Float16 bins[16][V];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (V == 2) {
      const hv b = *reinterpret_cast<const hv*>(xp + i * p.xc);
      bins[i][0] = b[0];
      bins[i][V - 1] = b[1];
    } else {
      bins[i][0] = xp[i * p.xc];
    }
  }
  float m[V];
  if (V == 2) {
    hv mv = {bins[0][0], bins[0][V - 1]};
#pragma unroll
    for (int i = 1; i < 16; ++i) mv = __builtin_elementwise_max(mv, (hv){bins[i][0], bins[i][V - 1]});
    m[0] = (float)mv[0];
    m[V - 1] = (float)mv[1];
  } else {
    m[0] = (float)bins[0][0];
#pragma unroll
    for (int i = 1; i < 16; ++i) m[0] = fmaxf(m[0], (float)bins[i][0]);
  }
  constexpr float kLog2e = 1.4426950408889634f;
  float r[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const float ml = m[j] * kLog2e;
    float s = 0.f, w = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float x = (float)bins[i][j];
      const float e = FAST ? __builtin_amdgcn_exp2f(__builtin_fmaf(x, kLog2e, -ml)) : expf(x - m[j]);
      s += e;
      w += e * (float)i;
    }
    r[j] = FAST ? w * __builtin_amdgcn_rcpf(s) : w / s;
  }
  TO* op = static_cast<TO*>(p.out) + n * p.on + (int64_t)sd * p.os + (int64_t)a0 * p.oa;
  if (V == 2) {
    typedef TO ov __attribute__((ext_vector_type(2)));
    *reinterpret_cast<ov*>(op) = (ov){(TO)r[0], (TO)r[V - 1]};
  } else {
    op[0] = (TO)r[0];
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

// Streaming (non-temporal) loads and stores for launches moving at least this
// many bytes; smaller ones stay cached for their producer and consumer.
constexpr int64_t kStreamingBytes = (int64_t)16 << 20;

// Lanes per row G and chunks per lane KPT for a row of `chunks` (<= 512).
template <typename TI, typename TO, bool VEC, bool FAST, bool NT>
void launch_rows(const SoftmaxPlan& p, int64_t chunks, uint64_t rows, hipStream_t stream) {
  auto grid = [&](int g) { return (uint32_t)((rows + (uint64_t)kWaves * (64 / g) - 1) / ((uint64_t)kWaves * (64 / g))); };
#define THIN_ROWG(G, K) hipLaunchKernelGGL((softmax_row_kernel<TI, TO, VEC, G, K, FAST, NT>), dim3(grid(G)), \
                                           dim3(kThreads), 0, stream, p)
  if (chunks <= 2) THIN_ROWG(1, 2);
  else if (chunks <= 4) THIN_ROWG(2, 2);
  else if (chunks <= 8) THIN_ROWG(4, 2);
  else if (chunks <= 16) THIN_ROWG(8, 2);
  else if (chunks <= 32) THIN_ROWG(16, 2);
  else if (chunks <= 64) THIN_ROWG(32, 2);
  else if (chunks <= 128) THIN_ROWG(64, 2);
  else if (chunks <= 256) THIN_ROWG(64, 4);
  else THIN_ROWG(64, 8);
#undef THIN_ROWG
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
  if (vec) {
    p.units = (uint32_t)(cols / V);
    const uint32_t grid = (p.units + kThreads - 1) / kThreads;
    hipLaunchKernelGGL((softmax_col_kernel<TI, TO, V, 16, FAST>), dim3(grid), dim3(kThreads), 0, stream, p);
  } else {
    p.units = (uint32_t)cols;
    const uint32_t grid = (p.units + kThreads - 1) / kThreads;
    hipLaunchKernelGGL((softmax_col_kernel<TI, TO, 1, 32, FAST>), dim3(grid), dim3(kThreads), 0, stream, p);
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
  if (out->dtype == THIN_F16) {
    if (vec) hipLaunchKernelGGL((dfl_expect_kernel<_Float16, V, true>), dim3(grid), dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((dfl_expect_kernel<_Float16, 1, true>), dim3(grid), dim3(kThreads), 0, stream, p);
  } else {
    if (vec) hipLaunchKernelGGL((dfl_expect_kernel<float, V, false>), dim3(grid), dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((dfl_expect_kernel<float, 1, false>), dim3(grid), dim3(kThreads), 0, stream, p);
  }
  THIN_LAUNCH_CHECK("dfl_expect");
  return THIN_OK;
}
