// Data movement, all bit-exact: cat, NC1HWC0 nearest-2x upsample (alone and
// fused into a channel concat), NCHW nearest-2x upsample, and the
// NCHW <-> NC1HWC0 (C0 = 16) repack.
//
// These kernels are HBM-bound byte movers: 16-byte vector loads/stores wherever
// the layout allows, streaming stores for large outputs, index math done once
// per block where it is uniform (plane / input selection), and LDS only for the
// channel transpose of the repack.
#include "common.h"

#include <algorithm>
#include <type_traits>

#include <string.h>

namespace thin {
thin_status copy_bits(const thin_desc* src, const thin_desc* dst, hipStream_t stream);

namespace {

constexpr uint32_t kThreads = 256;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <bool NT>
__device__ __forceinline__ void st16(void* dst, u32x4 v) {
  if (NT) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst));
  else *reinterpret_cast<u32x4*>(dst) = v;
}
__device__ __forceinline__ u32x4 ld16(const void* src) { return *reinterpret_cast<const u32x4*>(src); }
// Streaming (non-temporal) load for data read exactly once by a launch that
// also streams its stores.
template <bool NT>
__device__ __forceinline__ u32x4 ld16s(const void* src) {
  if (NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
  return *reinterpret_cast<const u32x4*>(src);
}

// Launches whose output reaches kStreamingBytes use streaming stores, and
// streaming loads for inputs read once (cat, plane copies, pack).
constexpr uint32_t kStreamThreads = 256;

// ============================================================ cat

constexpr int kCatPerLaunch = 16;
constexpr int64_t kCatShortRun = 512;  // bytes: shorter row runs copy through the strided path
constexpr int kCatOuterDims = THIN_MAX_DIMS - 1;

// One input of a cat launch: its fields lie together, so that a block reads
// the ones of its input in one round of scalar loads.
struct CatInput {
  const char* src;
  int64_t outer_stride[kCatOuterDims];  // bytes
  int64_t col;                          // bytes into the output row
  uint32_t units;                       // units per row of this input (< 2^31)
  uint32_t first;                       // its first block task
  FastDiv chunks;                       // chunks (blocks) per row
};

struct CatPlan {
  char* out;                         // out row r starts at out + r * out_row (bytes)
  int64_t out_row;                   // bytes per output row
  int32_t n_outer;                   // outer dims (before the cat dim)
  int64_t outer_size[kCatOuterDims];
  int32_t count;                     // inputs in this launch
  uint32_t chunks_prefix[kCatPerLaunch + 1];  // block-task prefix over inputs
  CatInput in[kCatPerLaunch];
};

// Units of type W (16-byte vectors or single elements).  A block copies one
// chunk (kThreads * U units) of one (input, row) run; all index math except
// the unit offset is uniform per block.  OUTER1: at most one dim before the
// cat dim (every NC1HWC0 channel cat), so the row's source offset is one
// product.
template <typename W, int U, bool NT, uint32_t BS, bool OUTER1>
__global__ __launch_bounds__(BS) void cat_kernel(CatPlan p) {
  const uint32_t task = blockIdx.x;
  // This block's input: a select chain over the task prefixes, which are all
  // loaded at once, then one round of scalar loads of that input's record
  // (the index is block-uniform).  Selecting the input's fields step by step
  // made each step wait for the previous one's loads: the C2f cat of four
  // [32,64,80,80] tensors took 37.2 us that way and 33.3 us with one round.
  uint32_t sel = 0;
#pragma unroll
  for (int j = 1; j < kCatPerLaunch; ++j)
    if (j < p.count && task >= p.chunks_prefix[j]) sel = j;
  const CatInput& in = p.in[sel];
  const uint32_t local = task - in.first;  // < 2^31
  const uint32_t row = in.chunks.div(local);
  const uint32_t chunk = local - row * in.chunks.d;
  int64_t src_off;
  if constexpr (OUTER1) {
    src_off = (int64_t)row * in.outer_stride[0];  // 0 when the cat dim is the first
  } else {
    // decompose row over the shared outer sizes; the outermost dim takes the
    // rest of row, with no division
    src_off = 0;
    uint32_t r = row;
#pragma unroll
    for (int d = kCatOuterDims - 1; d >= 1; --d) {
      if (d >= p.n_outer) continue;
      const uint32_t sz = (uint32_t)p.outer_size[d];
      const uint32_t c = r % sz;
      r /= sz;
      src_off += (int64_t)c * in.outer_stride[d];
    }
    src_off += (int64_t)r * in.outer_stride[0];
  }
  const char* src_base = in.src;
  const int64_t col = in.col;
  const uint32_t nu = in.units;
  const W* src = reinterpret_cast<const W*>(src_base + src_off);
  // a row run holds fewer than 2^31 units (checked on the host)
  const uint32_t base = chunk * BS * U;
  // loads clamped into the run (a selected input holds at least one unit)
  // rather than predicated, so that no branch holds the source's scalar loads
  W v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t k = min(base + u * BS + threadIdx.x, nu - 1);
    if constexpr (sizeof(W) == 16) v[u] = __builtin_bit_cast(W, ld16s<NT>(src + k));
    else v[u] = src[k];
  }
  // the destination's kernel-argument loads go out under the data loads, not
  // before them (the scheduler would otherwise wait for them first)
  __builtin_amdgcn_sched_barrier(0);
  W* dst = reinterpret_cast<W*>(p.out + (int64_t)row * p.out_row + col);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t k = base + u * BS + threadIdx.x;
    if (k < nu) {
      if constexpr (sizeof(W) == 16) st16<NT>(dst + k, __builtin_bit_cast(u32x4, v[u]));
      else dst[k] = v[u];
    }
  }
}

// An input whose dims [dim, rank) are dense (row-major, size-1 dims ignored)
// copies as one run per output row.
bool run_dense(const thin_desc* t, int dim) {
  int64_t expect = 1;
  for (int d = t->rank - 1; d >= dim; --d) {
    if (t->sizes[d] == 1) continue;
    if (t->strides[d] != expect) return false;
    expect *= t->sizes[d];
  }
  return true;
}

template <typename W>
thin_status launch_cat_group(const thin_desc* const* ins, int count, int dim, const thin_desc* out,
                             const int64_t* col_elems, int esize, bool nt, hipStream_t stream) {
  const bool stream_cfg = nt && sizeof(W) == 16;
  // one 16-byte vector per thread when streaming (C2f cat 4x[32,64,80,80]:
  // 5.56 TB/s, against 5.40 with two and 5.24 with four) and below the
  // streaming size (4x[1,64,80,80]: 3.93 us, against 4.10 with two and 5.54
  // with four); four for large cats of single elements
  const int U = (stream_cfg || !nt) ? 1 : 4;
  const int64_t BS = stream_cfg ? kStreamThreads : kThreads;
  const int64_t wsize = sizeof(W);
  CatPlan p;
  memset(&p, 0, sizeof p);
  int64_t inner = 1;
  for (int d = dim + 1; d < out->rank; ++d) inner *= out->sizes[d];
  int64_t outer = 1;
  for (int d = 0; d < dim; ++d) outer *= out->sizes[d];
  p.out = static_cast<char*>(out->data);
  p.out_row = out->sizes[dim] * inner * esize;
  p.n_outer = dim;
  for (int d = 0; d < dim; ++d) p.outer_size[d] = out->sizes[d];
  p.count = count;
  uint64_t total = 0;
  for (int k = 0; k < count; ++k) {
    const thin_desc* t = ins[k];
    CatInput& in = p.in[k];
    in.src = static_cast<const char*>(t->data);
    for (int d = 0; d < dim; ++d) in.outer_stride[d] = t->strides[d] * esize;
    in.col = col_elems[k] * esize;
    const int64_t run_bytes = t->sizes[dim] * inner * esize;
    const int64_t units = run_bytes / wsize;
    THIN_REQUIRE(units < ((int64_t)1 << 31), THIN_ERR_UNSUPPORTED,
                 "cat: input %d moves %lld units per row, beyond one launch", k, (long long)units);
    in.units = (uint32_t)units;
    const int64_t cpr = (units + BS * U - 1) / (BS * U);
    in.chunks = FastDiv::make((uint32_t)cpr);
    in.first = (uint32_t)total;
    p.chunks_prefix[k] = (uint32_t)total;
    total += (uint64_t)cpr * (uint64_t)outer;
  }
  p.chunks_prefix[count] = (uint32_t)total;
  THIN_REQUIRE(total < (1ull << 31), THIN_ERR_UNSUPPORTED, "cat: too many row chunks (%llu)",
               (unsigned long long)total);
  if (total == 0) return THIN_OK;
#define THIN_CAT(O1)                                                                                      \
  do {                                                                                                    \
    if (stream_cfg)                                                                                       \
      hipLaunchKernelGGL((cat_kernel<W, 1, true, kStreamThreads, O1>), dim3((uint32_t)total), dim3(kStreamThreads), \
                         0, stream, p);                                                                   \
    else if (!nt)                                                                                         \
      hipLaunchKernelGGL((cat_kernel<W, 1, false, kThreads, O1>), dim3((uint32_t)total), dim3(kThreads), 0, stream, p); \
    else                                                                                                  \
      hipLaunchKernelGGL((cat_kernel<W, 4, false, kThreads, O1>), dim3((uint32_t)total), dim3(kThreads), 0, stream, p); \
  } while (0)
  if (dim <= 1) THIN_CAT(true);
  else THIN_CAT(false);
#undef THIN_CAT
  THIN_LAUNCH_CHECK("cat");
  return THIN_OK;
}

// ============================================================ NC1HWC0 planes

// Output plane (n, c1) of an NC1HWC0 tensor is either a copy of an input plane
// or the nearest-2x upsample of one.  Plane = H*W*C0 dense elements; a pixel is
// `vpp` 16-byte vectors (C0 * element size / 16).
constexpr int kPlaneInputs = 16;
// One input of a plane launch: its fields lie together, so that a block
// reads the ones of its input in one round of scalar loads.
struct PlaneInput {
  const char* src;
  int64_t src_n, src_c1;       // bytes
  uint32_t c1_first;           // its first output channel block
  uint32_t up;                 // 1 = upsample 2x
};

struct PlanePlan {
  char* out;
  int64_t out_n, out_c1;       // bytes
  uint32_t out_c1_total;       // C1 of the output
  uint32_t oh, ow;             // output H, W
  uint32_t vpp;                // 16-byte vectors per pixel
  uint32_t plane_vecs;         // oh * ow * vpp
  int32_t count;
  uint32_t c1_prefix[kPlaneInputs + 1];
  PlaneInput in[kPlaneInputs];
  uint32_t tiles;              // blocks per output plane
  FastDiv div_tiles;
  FastDiv div_row;             // ow * vpp (vectors per output row)
  FastDiv div_vpp;
  FastDiv div_c1;              // out_c1_total
};
constexpr uint32_t kPlaneXcdRun = 32;

// One block per (output plane, tile of BS * U vectors).  Everything that
// depends on the plane -- which input feeds it, its offsets, whether it is
// upsampled -- is block-uniform, so it lives in scalar registers and comes
// through scalar loads of the plan; a lane only locates its vector inside the
// plane.  (A flat grid over all output vectors chose the input per lane,
// which put vector loads of the plan in front of every data load: 49.3 against
// 39.4 us for the C3 upsample->cat at N=32 from cold buffers.)
// NIN: the launch's input count when 1 or 2, else kPlaneInputs (at most that many).
template <int U, bool NT, uint32_t BS, bool XCD, int NIN>
__global__ __launch_bounds__(BS) void plane_kernel(PlanePlan p) {
  // XCD (streaming launches that upsample): consecutive tiles read the same
  // source rows, so each XCD takes runs of kPlaneXcdRun consecutive tiles.
  // (Upsample [32,256,40,40] 25.0 -> 23.9 us, upsample->cat 39.9 -> 39.1 us;
  // runs of 16 or 64 tiles measured between, one contiguous range per XCD
  // 26.0 and 42.3 us, small launches slightly slower with any grouping.)  A
  // compile-time choice: a test of a plan field here held every later scalar
  // load behind its wait (with NIN: upsample 23.1 -> 21.8 us at N=32,
  // 3.70 -> 3.21 us at N=1).
  const uint32_t blk = XCD ? dev::xcd_grouped<kPlaneXcdRun>(blockIdx.x, gridDim.x) : blockIdx.x;
  const uint32_t plane = p.div_tiles.div(blk);
  const uint32_t tile = blk - plane * p.tiles;
  const uint32_t n = p.div_c1.div(plane);
  const uint32_t c1 = plane - n * p.out_c1_total;
  // the input: a select chain over the channel prefixes (loaded at once),
  // then one round of scalar loads of its record
  uint32_t i = 0;
#pragma unroll
  for (int j = 1; j < NIN; ++j)
    if ((NIN <= 2 || j < p.count) && c1 >= p.c1_prefix[j]) i = j;
  const PlaneInput& in = p.in[i];
  const char* src = in.src + (int64_t)n * in.src_n + (int64_t)(c1 - in.c1_first) * in.src_c1;
  char* dst = p.out + (int64_t)n * p.out_n + (int64_t)c1 * p.out_c1;
  const uint32_t first = tile * (BS * U) + threadIdx.x;
  u32x4 v[U];
  if (in.up) {
    const uint32_t in_row = (p.ow >> 1) * p.vpp;  // vectors per input row
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t o = first + u * BS;
      if (o >= p.plane_vecs) break;
      const uint32_t oy = p.div_row.div(o);
      const uint32_t r = o - oy * p.div_row.d;
      const uint32_t ox = p.div_vpp.div(r);
      const uint32_t k = r - ox * p.vpp;
      // each source vector feeds four outputs: keep it cacheable
      v[u] = ld16(src + (size_t)((oy >> 1) * in_row + (ox >> 1) * p.vpp + k) * 16);
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t o = first + u * BS;
      if (o >= p.plane_vecs) break;
      v[u] = ld16s<NT>(src + (size_t)o * 16);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t o = first + u * BS;
    if (o >= p.plane_vecs) break;
    st16<NT>(dst + (size_t)o * 16, v[u]);
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Validates an NC1HWC0-style operand: rank 5, H/W/C0 dense, N/C1 strides and
// base 16-byte aligned.
bool plane_dense(const thin_desc* d, int esize) {
  if (d->rank != 5) return false;
  const int64_t h = d->sizes[2], w = d->sizes[3], c0 = d->sizes[4];
  if ((c0 * esize) % 16) return false;
  if (!(c0 == 1 || d->strides[4] == 1)) return false;
  if (!(w == 1 || d->strides[3] == c0)) return false;
  if (!(h == 1 || d->strides[2] == w * c0)) return false;
  return aligned16(d->data) && (d->strides[0] * esize) % 16 == 0 && (d->strides[1] * esize) % 16 == 0;
}

thin_status launch_planes(const thin_desc* ins, const int32_t* up, int count, const thin_desc* out,
                          hipStream_t stream) {
  const int esize = dtype_size(out->dtype);
  PlanePlan p;
  memset(&p, 0, sizeof p);
  p.out = static_cast<char*>(out->data);
  p.out_n = out->strides[0] * esize;
  p.out_c1 = out->strides[1] * esize;
  p.out_c1_total = (uint32_t)out->sizes[1];
  p.oh = (uint32_t)out->sizes[2];
  p.ow = (uint32_t)out->sizes[3];
  p.vpp = (uint32_t)(out->sizes[4] * esize / 16);
  THIN_REQUIRE((uint64_t)out->sizes[2] * out->sizes[3] * p.vpp < (1ull << 31), THIN_ERR_UNSUPPORTED,
               "upsample/cat: output plane too large for one launch");
  p.plane_vecs = p.oh * p.ow * p.vpp;
  p.count = count;
  uint32_t c1 = 0;
  for (int k = 0; k < count; ++k) {
    p.c1_prefix[k] = c1;
    PlaneInput& in = p.in[k];
    in.src = static_cast<const char*>(ins[k].data);
    in.src_n = ins[k].strides[0] * esize;
    in.src_c1 = ins[k].strides[1] * esize;
    in.c1_first = c1;
    in.up = up ? (uint32_t)(up[k] != 0) : 0u;
    c1 += (uint32_t)ins[k].sizes[1];
  }
  p.c1_prefix[count] = c1;
  const uint64_t planes = (uint64_t)out->sizes[0] * out->sizes[1];
  p.div_row = FastDiv::make(p.ow * p.vpp);
  p.div_vpp = FastDiv::make(p.vpp);
  p.div_c1 = FastDiv::make(p.out_c1_total);
  if (planes == 0 || p.plane_vecs == 0) return THIN_OK;
  // streaming launches: two vectors per thread; below the streaming size one
  // (upsample [1,256,40,40]: more blocks in flight)
  const bool nt = (int64_t)planes * p.plane_vecs * 16 >= kStreamingBytes;
  const uint32_t per_block = nt ? 2 * kStreamThreads : kThreads;
  p.tiles = (p.plane_vecs + per_block - 1) / per_block;
  p.div_tiles = FastDiv::make(p.tiles);
  const uint64_t blocks = planes * p.tiles;
  THIN_REQUIRE(blocks < (1ull << 31), THIN_ERR_UNSUPPORTED, "upsample/cat: output too large for one launch");
  bool upsamples = false;
  for (int k = 0; k < count; ++k) upsamples = upsamples || p.in[k].up;
  // the launch's input count fixed at compile time when it is 1 or 2 (upsample,
  // upsample->cat): fewer rounds of scalar loads to choose the input
#define THIN_PLANES(NIN)                                                                                       \
  do {                                                                                                         \
    if (nt && upsamples) /* XCD-grouped block order */                                                         \
      hipLaunchKernelGGL((plane_kernel<2, true, kStreamThreads, true, NIN>), dim3((uint32_t)blocks),           \
                         dim3(kStreamThreads), 0, stream, p);                                                  \
    else if (nt)                                                                                               \
      hipLaunchKernelGGL((plane_kernel<2, true, kStreamThreads, false, NIN>), dim3((uint32_t)blocks),          \
                         dim3(kStreamThreads), 0, stream, p);                                                  \
    else                                                                                                       \
      hipLaunchKernelGGL((plane_kernel<1, false, kThreads, false, NIN>), dim3((uint32_t)blocks), dim3(kThreads), \
                         0, stream, p);                                                                        \
  } while (0)
  if (count == 1) THIN_PLANES(1);
  else if (count == 2) THIN_PLANES(2);
  else THIN_PLANES(kPlaneInputs);
#undef THIN_PLANES
  THIN_LAUNCH_CHECK("plane");
  return THIN_OK;
}

// ------------------------------------------------------------ generic index map
// Fallback for layouts the vector kernels do not take: one element per thread,
// output element (n, c, oy, ox, k) of a 5-D view reads input (n, c, oy>>sy, ox>>sx, k).
struct Up5Plan {
  const char* src;
  char* dst;
  int64_t size[5];                 // output sizes
  int64_t ss[5], ds[5];            // element strides
  int32_t shift_h, shift_w;        // 1 for the upsampled axes
  int64_t total;
  int32_t esize;
};

template <typename E>
__global__ __launch_bounds__(kThreads) void up5_kernel(Up5Plan p) {
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < p.total;
       e += (int64_t)gridDim.x * kThreads) {
    int64_t r = e, so = 0, dof = 0;
    for (int d = 4; d >= 0; --d) {
      const int64_t c = r % p.size[d];
      r /= p.size[d];
      dof += c * p.ds[d];
      int64_t ci = c;
      if (d == 2) ci = c >> p.shift_h;
      if (d == 3) ci = c >> p.shift_w;
      so += ci * p.ss[d];
    }
    reinterpret_cast<E*>(p.dst)[dof] = reinterpret_cast<const E*>(p.src)[so];
  }
}

thin_status launch_up5(const thin_desc* x5, const thin_desc* y5, bool up, hipStream_t stream) {
  Up5Plan p;
  p.src = static_cast<const char*>(x5->data);
  p.dst = static_cast<char*>(y5->data);
  p.total = 1;
  for (int d = 0; d < 5; ++d) {
    p.size[d] = y5->sizes[d];
    p.ss[d] = x5->strides[d];
    p.ds[d] = y5->strides[d];
    p.total *= p.size[d];
  }
  p.shift_h = up ? 1 : 0;
  p.shift_w = up ? 1 : 0;
  p.esize = dtype_size(y5->dtype);
  if (p.total == 0) return THIN_OK;
  const uint32_t grid = grid_for((uint64_t)p.total, kThreads, 1, 256u * 16u);
  switch (p.esize) {
    case 1: hipLaunchKernelGGL(up5_kernel<uint8_t>, dim3(grid), dim3(kThreads), 0, stream, p); break;
    case 2: hipLaunchKernelGGL(up5_kernel<uint16_t>, dim3(grid), dim3(kThreads), 0, stream, p); break;
    case 4: hipLaunchKernelGGL(up5_kernel<uint32_t>, dim3(grid), dim3(kThreads), 0, stream, p); break;
    default: hipLaunchKernelGGL(up5_kernel<uint64_t>, dim3(grid), dim3(kThreads), 0, stream, p); break;
  }
  THIN_LAUNCH_CHECK("up5");
  return THIN_OK;
}

// ============================================================ NCHW upsample
// Output row vector j (8 halves) = input elements 4j..4j+3 each twice.
struct NchwUpPlan {
  const char* src;
  char* dst;
  int64_t s_n, s_c, s_h;   // input strides (bytes); w stride == element
  int64_t d_n, d_c, d_h;   // output strides (bytes); w dense
  uint32_t c, oh, row_vecs;  // channels, output rows, 16-byte vectors per output row
  uint32_t rows;             // N * C * oh
  FastDiv div_row_vecs, div_oh, div_c;
};

template <typename E, bool NT>
__global__ __launch_bounds__(kThreads) void nchw_up_kernel(NchwUpPlan p) {
  constexpr int PER = 16 / sizeof(E);        // output elements per vector
  const uint32_t total = p.rows * p.row_vecs;  // < 2^31, checked on the host
  for (uint32_t v = blockIdx.x * kThreads + threadIdx.x; v < total; v += gridDim.x * kThreads) {
    const uint32_t row = p.div_row_vecs.div(v);
    const uint32_t j = v - row * p.row_vecs;
    const uint32_t nc = p.div_oh.div(row);
    const uint32_t oy = row - nc * p.oh;
    const uint32_t n = p.div_c.div(nc);
    const uint32_t c = nc - n * p.c;
    const E* s = reinterpret_cast<const E*>(p.src + n * p.s_n + c * p.s_c + (int64_t)(oy >> 1) * p.s_h) + j * (PER / 2);
    E out[PER];
#pragma unroll
    for (int k = 0; k < PER / 2; ++k) {
      E e = s[k];
      out[2 * k] = e;
      out[2 * k + 1] = e;
    }
    char* d = p.dst + n * p.d_n + c * p.d_c + (int64_t)oy * p.d_h + (size_t)j * 16;
    st16<NT>(d, __builtin_bit_cast(u32x4, out));
  }
}

// NCHW 2x upsample for rows the 16-byte form cannot take (odd or unaligned
// output widths, gapped or strided input rows): a thread per input element
// stores it to its two output rows as one two-element word each (columns 2x
// and 2x + 1), so a wave writes 2 x 64 words side by side.
struct NchwPairPlan {
  const char* src;
  char* dst;
  int64_t s_n, s_c, s_h, s_w;  // input strides (bytes)
  int64_t d_n, d_c, d_h;       // output strides (bytes); w dense
  uint32_t w, h, c, total;     // input width, height, channels; N * C * H * W
  FastDiv div_w, div_h, div_c;
};

template <typename E, typename E2>
__global__ __launch_bounds__(kThreads) void nchw_up_pair_kernel(NchwPairPlan p) {
  for (uint32_t e = blockIdx.x * kThreads + threadIdx.x; e < p.total; e += gridDim.x * kThreads) {
    const uint32_t r = p.div_w.div(e), x = e - r * p.w;
    const uint32_t nc = p.div_h.div(r), y = r - nc * p.h;
    const uint32_t n = p.div_c.div(nc), c = nc - n * p.c;
    const E v = *reinterpret_cast<const E*>(p.src + n * p.s_n + c * p.s_c + (int64_t)y * p.s_h + (int64_t)x * p.s_w);
    E2 pair;
    pair[0] = v;
    pair[1] = v;
    char* d = p.dst + n * p.d_n + c * p.d_c + (int64_t)(2 * y) * p.d_h + (int64_t)x * (int64_t)sizeof(E2);
    *reinterpret_cast<E2*>(d) = pair;
    *reinterpret_cast<E2*>(d + p.d_h) = pair;
  }
}

// ============================================================ max pool
// Stride-1 max pool with an odd k x k window and "same" padding (taps outside
// the plane are skipped, i.e. -inf).  A thread owns one pixel vector (V
// values at one (plane, x): 8 channels of an NC1HWC0 pixel, or one NCHW
// element) and walks a chunk of output rows, keeping the horizontal maxima of
// the last k input rows in registers; output row y is the vertical max of
// those k maxima.  Both passes keep the first strictly greater value, so the
// selected value is the first maximum in row-major window order -- the one
// PyTorch CPU's max_pool2d keeps (a +0/-0 tie resolves the same way).  A NaN
// in the window gives NaN.
struct PoolPlan {
  const char* x;
  char* y;
  int64_t xs[4], ys[4];   // element strides of (n, c, h, w); NC1HWC0 adds the C0 part as V elements
  uint32_t c, h, w;       // channels (or channel blocks), height, width
  uint32_t parts;         // pixel vectors per pixel: 2 for NC1HWC0, 1 for NCHW
  uint32_t rows;          // output rows per thread
  uint32_t units;         // planes * chunks * w * parts
  FastDiv div_parts, div_w, div_chunks, div_c;
  FastDiv div_row;        // w * parts (LDS form)
  FastDiv div_prow;       // (w + k - 1) * parts: LDS input rows padded with k/2 -inf pixels each side
};

template <typename T, int V>
struct alignas(sizeof(T) * V) PoolVec {
  T e[V];
};

template <typename T, int V>
__device__ __forceinline__ void keep_max(PoolVec<T, V>& m, const PoolVec<T, V>& v) {
#pragma unroll
  for (int j = 0; j < V; ++j)
    if (v.e[j] > m.e[j] || v.e[j] != v.e[j]) m.e[j] = v.e[j];
}

template <typename T, int V, int K>
__global__ __launch_bounds__(kThreads) void maxpool_kernel(PoolPlan p) {
  constexpr int R = K / 2;
  const uint32_t u = blockIdx.x * kThreads + threadIdx.x;
  if (u >= p.units) return;
  uint32_t q = p.div_parts.div(u);
  const uint32_t part = u - q * p.parts;
  uint32_t r = p.div_w.div(q);
  const uint32_t x = q - r * p.w;
  const uint32_t plane = p.div_chunks.div(r);
  const uint32_t chunk = r - plane * p.div_chunks.d;
  const uint32_t n = p.div_c.div(plane), c = plane - n * p.c;
  const T* xp = reinterpret_cast<const T*>(p.x) + n * p.xs[0] + c * p.xs[1] + (int64_t)part * V;
  T* yp = reinterpret_cast<T*>(p.y) + n * p.ys[0] + c * p.ys[1] + (int64_t)part * V + (int64_t)x * p.ys[3];
  const int y0 = (int)(chunk * p.rows);
  const int y1 = min((int)p.h, y0 + (int)p.rows);
  PoolVec<T, V> ninf;
#pragma unroll
  for (int j = 0; j < V; ++j) ninf.e[j] = (T)(-__builtin_inff());
  // horizontal max of input row yy at column x (-inf outside the plane):
  // the K taps are loaded unconditionally from positions clamped into the
  // plane, all in flight before the first is used, and a tap outside the
  // plane is skipped (as an -inf tap would be)
  auto hmax = [&](int yy) {
    const bool row_ok = yy >= 0 && yy < (int)p.h;
    const T* row = xp + (int64_t)min(max(yy, 0), (int)p.h - 1) * p.xs[2];
    PoolVec<T, V> t[K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const int xx = min(max((int)x + i - R, 0), (int)p.w - 1);
      t[i] = *reinterpret_cast<const PoolVec<T, V>*>(row + (int64_t)xx * p.xs[3]);
    }
    PoolVec<T, V> m = ninf;
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const int xx = (int)x + i - R;
      if (row_ok && xx >= 0 && xx < (int)p.w) keep_max(m, t[i]);
    }
    return m;
  };
  PoolVec<T, V> hm[K];
#pragma unroll
  for (int i = 0; i < K - 1; ++i) hm[i + 1] = hmax(y0 - R + i);
  for (int y = y0; y < y1; ++y) {
#pragma unroll
    for (int i = 0; i < K - 1; ++i) hm[i] = hm[i + 1];
    hm[K - 1] = hmax(y + R);
    PoolVec<T, V> m = ninf;
#pragma unroll
    for (int i = 0; i < K; ++i) keep_max(m, hm[i]);
    *reinterpret_cast<PoolVec<T, V>*>(yp + (int64_t)y * p.ys[2]) = m;
  }
}

// LDS-tiled form: a block takes one plane band of `rows` output rows.  The
// band's input rows plus the 2R halo rows are read once (coalesced) into LDS,
// with R -inf pixels padding each row on both sides (so no tap needs a bounds
// check), horizontal maxima go to a second LDS buffer, vertical maxima to HBM
// -- one global round trip per block instead of one per output row.
//
// fp16 pixel vectors take a packed path: the IEEE-754 2019 maximum
// (v_pk_maximum3_f16, two taps per instruction) propagates NaN and orders
// -0 < +0, so it selects the same bits as the first-maximum rule except where
// a window's maximum is a +0/-0 tie.  A block whose tile holds zeros of both
// signs therefore keeps the first-maximum selects; other blocks take the
// packed path.
template <typename T, int V, int K>
__global__ __launch_bounds__(kThreads) void maxpool_tile_kernel(PoolPlan p, uint32_t bands) {
  constexpr int R = K / 2;
  constexpr bool kPacked = std::is_same<T, _Float16>::value && V == 8;
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
  extern __shared__ __attribute__((aligned(16))) char pool_lds[];
  __shared__ uint32_t wave_zero_signs[kThreads / 64];
  typedef PoolVec<T, V> PV;
  const uint32_t plane = blockIdx.x / bands, band = blockIdx.x - plane * bands;
  const uint32_t n = p.div_c.div(plane), c = plane - n * p.c;
  const int y0 = (int)(band * p.rows);
  const int tile_rows = (int)p.rows + 2 * R;
  const uint32_t row_vecs = p.w * p.parts;
  const uint32_t prow = p.div_prow.d;
  const uint32_t tile = (uint32_t)tile_rows * prow;
  const uint32_t htile = (uint32_t)tile_rows * row_vecs;
  PV* in = reinterpret_cast<PV*>(pool_lds);
  PV* hm = in + tile;
  PV ninf;
#pragma unroll
  for (int j = 0; j < V; ++j) ninf.e[j] = (T)(-__builtin_inff());
  const T* xp = reinterpret_cast<const T*>(p.x) + n * p.xs[0] + c * p.xs[1];
  const uint32_t pshift = p.parts == 2 ? 1u : 0u;
  // per-thread minima of the loaded bits and of the bits with the sign
  // flipped: a zero lane means the tile holds a +0 (resp. a -0)
  u16x8 min_pos = (u16x8)(uint16_t)0xffff, min_neg = (u16x8)(uint16_t)0xffff;
  // four loads in flight per thread before their LDS writes.  The packed
  // form, which uses each loaded vector for its zero-sign minima, issues its
  // loads unconditionally from positions clamped into the plane and replaces
  // a pixel outside the plane (or past the tile) by -inf afterwards: a load
  // under a branch and used inside it is waited for before the next load is
  // issued.  The other forms load under the branch and use nothing there.
  constexpr int U = 4;
  for (uint32_t i0 = threadIdx.x; i0 < tile; i0 += U * kThreads) {
    PV v[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t i = i0 + u * kThreads;
      const uint32_t rr = p.div_prow.div(i), k = i - rr * prow;
      const int x = (int)(k >> pshift) - R;
      const uint32_t part = k & pshift;
      const int yy = y0 - R + (int)rr;
      ok[u] = i < tile && yy >= 0 && yy < (int)p.h && x >= 0 && x < (int)p.w;
      if constexpr (kPacked) {
        const int yc = min(max(yy, 0), (int)p.h - 1), xc = min(max(x, 0), (int)p.w - 1);
        v[u] = *reinterpret_cast<const PV*>(xp + (int64_t)yc * p.xs[2] + (int64_t)xc * p.xs[3] + (int64_t)part * V);
      } else {
        v[u] = ninf;
        if (ok[u]) v[u] = *reinterpret_cast<const PV*>(xp + (int64_t)yy * p.xs[2] + (int64_t)x * p.xs[3] + (int64_t)part * V);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (kPacked) {
        if (!ok[u]) {
          v[u] = ninf;
        } else {
          const u16x8 b = __builtin_bit_cast(u16x8, v[u]);
          min_pos = __builtin_elementwise_min(min_pos, b);
          min_neg = __builtin_elementwise_min(min_neg, b ^ (uint16_t)0x8000);
        }
      }
      if (i0 + u * kThreads < tile) in[i0 + u * kThreads] = v[u];
    }
  }
  bool exact = !kPacked;
  if constexpr (kPacked) {
    const uint32_t has = (__ballot(__builtin_reduce_min(min_pos) == 0) != 0 ? 1u : 0u) |
                         (__ballot(__builtin_reduce_min(min_neg) == 0) != 0 ? 2u : 0u);
    if ((threadIdx.x & 63u) == 0) wave_zero_signs[threadIdx.x >> 6] = has;
  }
  __syncthreads();
  if constexpr (kPacked) {
    uint32_t has = 0;
#pragma unroll
    for (int wv = 0; wv < kThreads / 64; ++wv) has |= wave_zero_signs[wv];
    exact = has == 3u;
  }
  for (uint32_t i = threadIdx.x; i < htile; i += kThreads) {
    const uint32_t rr = p.div_row.div(i), k = i - rr * row_vecs;
    const uint32_t base = rr * prow + k;
    if constexpr (kPacked) {
      if (!exact) {
        const h8* ih = reinterpret_cast<const h8*>(in);
        h8 m = ih[base];
#pragma unroll
        for (int j = 1; j <= 2 * R; ++j) m = __builtin_elementwise_maximum(m, ih[base + j * (int)p.parts]);
        reinterpret_cast<h8*>(hm)[i] = m;
        continue;
      }
    }
    PV m = ninf;
#pragma unroll
    for (int j = 0; j <= 2 * R; ++j) keep_max(m, in[base + j * (int)p.parts]);
    hm[i] = m;
  }
  __syncthreads();
  T* yp = reinterpret_cast<T*>(p.y) + n * p.ys[0] + c * p.ys[1];
  const uint32_t outs = p.rows * row_vecs;
  for (uint32_t i = threadIdx.x; i < outs; i += kThreads) {
    const uint32_t ry = p.div_row.div(i), k = i - ry * row_vecs;
    const int y = y0 + (int)ry;
    if (y >= (int)p.h) break;
    const uint32_t x = k >> pshift, part = k & pshift;
    PV m;
    if constexpr (kPacked) {
      if (!exact) {
        const h8* hh = reinterpret_cast<const h8*>(hm);
        h8 mh = hh[ry * row_vecs + k];
#pragma unroll
        for (int dy = 1; dy <= 2 * R; ++dy) mh = __builtin_elementwise_maximum(mh, hh[(ry + dy) * row_vecs + k]);
        m = __builtin_bit_cast(PV, mh);
      }
    }
    if (exact) {
      m = ninf;
#pragma unroll
      for (int dy = 0; dy <= 2 * R; ++dy) keep_max(m, hm[(ry + dy) * row_vecs + k]);
    }
    *reinterpret_cast<PV*>(yp + (int64_t)y * p.ys[2] + (int64_t)x * p.ys[3] + (int64_t)part * V) = m;
  }
}

constexpr size_t kPoolLdsBytes = 64 * 1024;

template <typename T, int V>
thin_status launch_pool(PoolPlan& p, uint32_t planes, int kernel, hipStream_t stream) {
  const int R = kernel / 2;
  const size_t row_bytes = (size_t)p.w * p.parts * sizeof(PoolVec<T, V>);
  const size_t prow_bytes = (size_t)(p.w + 2 * R) * p.parts * sizeof(PoolVec<T, V>);
  const uint64_t plane_rows = (uint64_t)planes * p.h;
  // LDS form: band height for >= ~2048 blocks (several per CU to overlap the
  // load round trip of one band with the max passes of another), within the
  // LDS budget (padded in + hm); halo rows are re-read from L2
  const size_t max_tile_rows = kPoolLdsBytes / (prow_bytes + row_bytes);
  if (max_tile_rows > (size_t)(2 * R)) {
    uint32_t rows = (uint32_t)((plane_rows + 2047) / 2048);
    rows = std::max<uint32_t>(1u, std::min<uint32_t>(rows, p.h));
    rows = std::min<uint32_t>(rows, (uint32_t)(max_tile_rows - 2 * R));
    const uint32_t bands = (p.h + rows - 1) / rows;
    const uint64_t blocks = (uint64_t)planes * bands;
    THIN_REQUIRE(blocks < (1ull << 31), THIN_ERR_UNSUPPORTED, "maxpool: tensor too large");
    p.rows = rows;
    p.div_c = FastDiv::make(p.c);
    p.div_row = FastDiv::make(p.w * p.parts);
    p.div_prow = FastDiv::make((p.w + 2 * R) * p.parts);
    const size_t lds = (size_t)(rows + 2 * R) * (prow_bytes + row_bytes);
    switch (kernel) {
#define THIN_POOLT(KK)                                                                                       \
  case KK:                                                                                                    \
    hipLaunchKernelGGL((maxpool_tile_kernel<T, V, KK>), dim3((uint32_t)blocks), dim3(kThreads), lds, stream, p, \
                       bands);                                                                                \
    break;
      THIN_POOLT(1) THIN_POOLT(3) THIN_POOLT(5) THIN_POOLT(7) THIN_POOLT(9) THIN_POOLT(11) THIN_POOLT(13)
      THIN_POOLT(15)
#undef THIN_POOLT
      default: break;
    }
    THIN_LAUNCH_CHECK("maxpool");
    return THIN_OK;
  }
  // register form for rows too wide for LDS: rows per thread chosen to fill the chip
  uint32_t rows = p.h;
  const uint64_t cols = (uint64_t)planes * p.w * p.parts;
  while (rows > 4 && cols * ((p.h + rows - 1) / rows) < 256u * 256u) rows = (rows + 1) / 2;
  const uint32_t chunks = (p.h + rows - 1) / rows;
  const uint64_t units = cols * chunks;
  THIN_REQUIRE(units < (1ull << 31), THIN_ERR_UNSUPPORTED, "maxpool: tensor too large");
  p.rows = rows;
  p.units = (uint32_t)units;
  p.div_parts = FastDiv::make(p.parts);
  p.div_w = FastDiv::make(p.w);
  p.div_chunks = FastDiv::make(chunks);
  p.div_c = FastDiv::make(p.c);
  const uint32_t grid = (uint32_t)((units + kThreads - 1) / kThreads);
  switch (kernel) {
#define THIN_POOLK(KK) \
  case KK: hipLaunchKernelGGL((maxpool_kernel<T, V, KK>), dim3(grid), dim3(kThreads), 0, stream, p); break;
    THIN_POOLK(1) THIN_POOLK(3) THIN_POOLK(5) THIN_POOLK(7) THIN_POOLK(9) THIN_POOLK(11) THIN_POOLK(13)
    THIN_POOLK(15)
#undef THIN_POOLK
    default: break;
  }
  THIN_LAUNCH_CHECK("maxpool");
  return THIN_OK;
}

bool pool_kernel_ok(int32_t k) { return k >= 1 && k <= 15 && (k & 1); }

// ============================================================ SPPF pool chain
// out = cat([x, p(x), p(p(x)), ...], dim 1) over NC1HWC0 fp16, p the stride-1
// k x k max pool above, `repeats` times: the SPPF block's pooling and concat
// in one pass over x.  A block takes one (n, c1) plane: the plane sits in LDS
// inside a border of R -inf pixels; each repeat is a horizontal pass into a
// second buffer and a vertical pass back into the plane's interior, written
// to its output slot as it goes.  Every repeat composes the same pool (not a
// wider window), so +0/-0 ties resolve exactly as chained pools do.  Each
// pass takes the packed IEEE maximum of its window and redoes with
// first-maximum selects only the vectors whose maximum has a +0/-0 lane: a
// nonzero maximum has the same bits whichever tied element supplies it (NaN:
// any NaN), so only zero maxima depend on the selection order.  With
// pool_only (one repeat, no copy of x) the same kernel is the plain max pool
// for planes that fit LDS.
struct SppfPlan {
  const _Float16* x;
  _Float16* y;
  int64_t xs[2], ys[2];   // element strides of (n, c1)
  uint32_t xh, yh;        // element strides of h (a plane's offsets fit 32 bits); pixels are dense (W stride 16)
  uint32_t c1, h, w, repeats;
  uint32_t pool_only;     // 1: out holds the last pool only (a plain max pool), no copy of x
  FastDiv div_c1, div_row, div_prow;  // row: w * 2 vectors; padded row: (w + k - 1) * 2
};

constexpr size_t kSppfLdsBytes = 144 * 1024;
// 1024 threads per plane: the serial passes take fewer steps ([N,256,20,20] k5
// x3: 7.8 us at N=32 and 5.2 us at N=1, against 9.4 and 7.6 with 256)
constexpr uint32_t kSppfThreads = 1024;

// Whether a window maximum has a +0/-0 lane.
__device__ __forceinline__ bool has_zero(const _Float16 __attribute__((ext_vector_type(8))) m) {
  typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
  return __builtin_reduce_min(__builtin_bit_cast(u16x8, m) & (uint16_t)0x7fff) == 0;
}

// VPP: 16-byte vectors per pixel held by a block.  2: the block pools all 16
// C0 lanes of its plane; 1: one C0 half (lanes 0-7 or 8-15, block parity), so
// that a small batch launches twice the blocks (channels pool independently).
// HH, WW: the plane's height and width when fixed at compile time (the 20x20
// planes of a 640-pixel input's SPPF block: the index arithmetic folds to
// constants), 0 to read them from the plan.
template <int K, bool NT, uint32_t BS, uint32_t VPP, uint32_t HH = 0, uint32_t WW = 0>
__global__ __launch_bounds__(BS) void sppf_kernel(SppfPlan p) {
  constexpr int R = K / 2;
  const uint32_t ph = HH ? HH : p.h, pw = HH ? WW : p.w;
  const uint32_t row_vecs = HH ? WW * VPP : p.div_row.d, prow = HH ? (WW + 2 * R) * VPP : p.div_prow.d;
  auto row_of = [&](uint32_t i) { return HH ? i / (WW * VPP) : p.div_row.div(i); };
  auto prow_of = [&](uint32_t i) { return HH ? i / ((WW + 2 * R) * VPP) : p.div_prow.div(i); };
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  typedef PoolVec<_Float16, 8> PV;
  extern __shared__ __attribute__((aligned(16))) char sppf_lds[];
  const uint32_t plane = VPP == 2 ? blockIdx.x : blockIdx.x >> 1;
  const uint32_t half = VPP == 2 ? 0u : (blockIdx.x & 1u) * 8u;  // C0 lane offset
  const uint32_t n = p.div_c1.div(plane), c = plane - n * p.c1;
  const uint32_t prows = ph + 2 * R;
  const uint32_t tile = prows * prow, htile = prows * row_vecs, outs = ph * row_vecs;
  PV* in = reinterpret_cast<PV*>(sppf_lds);
  PV* hm = in + tile;
  const h8* ih = reinterpret_cast<const h8*>(in);
  const h8* hh = reinterpret_cast<const h8*>(hm);
  const h8 ninf = (h8)(_Float16)(-__builtin_inff());
  const _Float16* xp = p.x + n * p.xs[0] + c * p.xs[1] + half;
  auto slot = [&](uint32_t r) { return p.y + n * p.ys[0] + ((r - p.pool_only) * p.c1 + c) * p.ys[1] + half; };
  // a pixel vector's element offset inside a plane (32-bit)
  auto pix = [&](uint32_t row_stride, uint32_t y, uint32_t k) {
    return y * row_stride + (k / VPP) * 16u + (VPP == 2 ? (k & 1u) * 8u : 0u);
  };
  // stage the padded plane; copy x to output slot 0
  _Float16* y0 = p.pool_only ? nullptr : slot(0);
  for (uint32_t i = threadIdx.x; i < tile; i += BS) {
    const uint32_t rr = prow_of(i), k = i - rr * prow;
    const uint32_t xx = k / VPP - R, yy = rr - R;  // wraps for the -inf border
    h8 v = ninf;
    if (yy < ph && xx < pw) {
      const uint32_t kk = k - R * VPP;
      v = *reinterpret_cast<const h8*>(xp + pix(p.xh, yy, kk));
      if (!p.pool_only) {
        h8* dst = reinterpret_cast<h8*>(y0 + pix(p.yh, yy, kk));
        if constexpr (NT) __builtin_nontemporal_store(v, dst);
        else *dst = v;
      }
    }
    reinterpret_cast<h8*>(in)[i] = v;
  }
  __syncthreads();
  for (uint32_t rep = 1; rep <= p.repeats; ++rep) {
    for (uint32_t i = threadIdx.x; i < htile; i += BS) {
      const uint32_t rr = row_of(i), k = i - rr * row_vecs;
      const uint32_t base = rr * prow + k;
      h8 m = ih[base];
#pragma unroll
      for (int j = 1; j <= 2 * R; ++j) m = __builtin_elementwise_maximum(m, ih[base + VPP * j]);
      if (has_zero(m)) {  // first maximum in window order
        PV e;
#pragma unroll
        for (int j = 0; j < 8; ++j) e.e[j] = (_Float16)(-__builtin_inff());
#pragma unroll
        for (int j = 0; j <= 2 * R; ++j) keep_max(e, in[base + VPP * j]);
        m = __builtin_bit_cast(h8, e);
      }
      reinterpret_cast<h8*>(hm)[i] = m;
    }
    __syncthreads();
    _Float16* yr = slot(rep);
    for (uint32_t i = threadIdx.x; i < outs; i += BS) {
      const uint32_t r = row_of(i), k = i - r * row_vecs;
      h8 m = hh[r * row_vecs + k];
#pragma unroll
      for (int dy = 1; dy <= 2 * R; ++dy) m = __builtin_elementwise_maximum(m, hh[(r + dy) * row_vecs + k]);
      if (has_zero(m)) {
        PV e;
#pragma unroll
        for (int j = 0; j < 8; ++j) e.e[j] = (_Float16)(-__builtin_inff());
#pragma unroll
        for (int dy = 0; dy <= 2 * R; ++dy) keep_max(e, hm[(r + dy) * row_vecs + k]);
        m = __builtin_bit_cast(h8, e);
      }
      if (rep < p.repeats) reinterpret_cast<h8*>(in)[(r + R) * prow + k + VPP * R] = m;  // the next repeat's input
      h8* dst = reinterpret_cast<h8*>(yr + pix(p.yh, r, k));
      if constexpr (NT) __builtin_nontemporal_store(m, dst);
      else *dst = m;
    }
    __syncthreads();
  }
}

// Per-block LDS bytes of sppf_kernel: the padded plane and the horizontal
// maxima, vpp 16-byte vectors per pixel.
uint64_t sppf_lds_bytes(int64_t H, int64_t W, int R, int64_t vpp) {
  return (uint64_t)(H + 2 * R) * (uint64_t)((W + 2 * R) + W) * (uint64_t)vpp * 16u;
}

// Whether sppf_kernel takes x / out: the padded plane fits one block's LDS,
// the planes number under 2^31, and every offset inside a plane (rows at
// strides[2], pixels 16 elements apart) fits 31 bits.
bool sppf_whole_plane(const thin_desc* x, const thin_desc* out, int R) {
  const int64_t H = x->sizes[2], W = x->sizes[3];
  if (sppf_lds_bytes(H, W, R, 2) > kSppfLdsBytes || x->sizes[0] * x->sizes[1] >= ((int64_t)1 << 31)) return false;
  for (const thin_desc* d : {x, out})
    if (d->strides[2] < 0 || (H - 1) * d->strides[2] + W * 16 >= ((int64_t)1 << 31)) return false;
  return true;
}

// Launches sppf_kernel for x [N,C1,H,W,16] (validated by the caller, whose
// plane fits kSppfLdsBytes with two vectors per pixel): out = cat of x and
// `repeats` chained pools, or with pool_only the single pool.
thin_status launch_sppf(const thin_desc* x, int32_t kernel, int32_t repeats, bool pool_only,
                        const thin_desc* out, hipStream_t stream) {
  const int64_t N = x->sizes[0], C1 = x->sizes[1], H = x->sizes[2], W = x->sizes[3];
  const int R = kernel / 2;
  SppfPlan p;
  memset(&p, 0, sizeof p);
  p.x = static_cast<const _Float16*>(x->data);
  p.y = static_cast<_Float16*>(out->data);
  for (int d = 0; d < 2; ++d) {
    p.xs[d] = x->strides[d];
    p.ys[d] = out->strides[d];
  }
  p.xh = (uint32_t)x->strides[2];
  p.yh = (uint32_t)out->strides[2];
  p.c1 = (uint32_t)C1;
  p.h = (uint32_t)H;
  p.w = (uint32_t)W;
  p.repeats = (uint32_t)repeats;
  p.pool_only = pool_only ? 1u : 0u;
  p.div_c1 = FastDiv::make((uint32_t)C1);
  // fewer than 256 planes: one block per C0 half of a plane
  // ([1,256,20,20] k5 x3 + cat: see the SPPF row of the kernel notes)
  const bool split = N * C1 < 256;
  const int64_t vpp = split ? 1 : 2;
  const size_t lds = (size_t)sppf_lds_bytes(H, W, R, vpp);  // the split form holds half the vectors
  p.div_row = FastDiv::make((uint32_t)(W * vpp));
  p.div_prow = FastDiv::make((uint32_t)((W + 2 * R) * vpp));
  const bool nt = numel(out) * 2 >= kStreamingBytes;
  const uint32_t blocks = (uint32_t)(N * C1 * (split ? 2 : 1));
  if (!split && H == 20 && W == 20 && kernel == 5) {  // SPPF of a 640-pixel input's stride-32 level
    if (nt) hipLaunchKernelGGL((sppf_kernel<5, true, kSppfThreads, 2, 20, 20>), dim3(blocks), dim3(kSppfThreads),
                               lds, stream, p);
    else hipLaunchKernelGGL((sppf_kernel<5, false, kSppfThreads, 2, 20, 20>), dim3(blocks), dim3(kSppfThreads),
                            lds, stream, p);
    THIN_LAUNCH_CHECK("sppf");
    return THIN_OK;
  }
  switch (kernel) {
#define THIN_SPPF(KK)                                                                                        \
  case KK:                                                                                                   \
    if (split) hipLaunchKernelGGL((sppf_kernel<KK, false, kSppfThreads, 1>), dim3(blocks), dim3(kSppfThreads), \
                                  lds, stream, p);                                                   \
    else if (nt) hipLaunchKernelGGL((sppf_kernel<KK, true, kSppfThreads, 2>), dim3(blocks), dim3(kSppfThreads), \
                                    lds, stream, p);                                                 \
    else hipLaunchKernelGGL((sppf_kernel<KK, false, kSppfThreads, 2>), dim3(blocks), dim3(kSppfThreads),     \
                            lds, stream, p);                                                         \
    break;
    THIN_SPPF(1) THIN_SPPF(3) THIN_SPPF(5) THIN_SPPF(7) THIN_SPPF(9) THIN_SPPF(11) THIN_SPPF(13) THIN_SPPF(15)
#undef THIN_SPPF
    default: break;
  }
  THIN_LAUNCH_CHECK("sppf");
  return THIN_OK;
}

// ============================================================ pack / unpack
// Per (n, c1, tile of kTile pixels): LDS tile [16][kTile] of halves.  Large
// packs take tiles of kWideTile pixels: each block then reads 1 KB runs of
// its sixteen channel rows instead of 512 B ([32,64,160,160]: 35.1 -> 34.4
// us), while smaller ones keep kTile so that every CU still gets blocks
// ([1,64,160,160]: 3.63 us against 3.86).
constexpr int kTile = 256;
constexpr int kWideTile = 512;

struct PackPlan {
  const uint16_t* x;   // NCHW fp16 bits (pack) or NC1HWC0 (unpack)
  uint16_t* y;
  int64_t x_n, x_c, x_hw;   // pack: NCHW strides (elements); hw = pixel stride (1 when dense)
  int64_t y_n, y_c1;        // NC1HWC0 output strides (elements), plane dense
  uint32_t channels;        // C
  uint32_t c1;              // C1 = ceil(C/16)
  uint32_t hw;              // pixels per plane
  uint32_t tiles;           // ceil(hw / tile pixels)
  uint32_t vec_ok;          // pixel rows 16-byte aligned and dense
  FastDiv div_tiles, div_c1;  // block index -> (n, c1 block, tile) with no integer division sequence
};

// pack: NCHW -> NC1HWC0 (zero-fill channels >= C), TILE pixels a block
template <bool NT, int TILE>
__global__ __launch_bounds__(kThreads) void pack_kernel(PackPlan p) {
  __shared__ uint16_t tile[16][TILE + 2];
  // the plan in registers before the first test of one of its fields: one
  // round of scalar loads (one asm statement: each is a scheduling boundary)
  __asm__ volatile("" ::"s"(p.x), "s"(p.y), "s"(p.x_n), "s"(p.x_c), "s"(p.x_hw), "s"(p.y_n), "s"(p.y_c1),
                   "s"(p.channels), "s"(p.c1), "s"(p.hw), "s"(p.tiles), "s"(p.vec_ok), "s"(p.div_tiles.mul),
                   "s"(p.div_tiles.shr), "s"(p.div_c1.mul), "s"(p.div_c1.shr));
  const uint32_t plane = p.div_tiles.div(blockIdx.x), t = blockIdx.x - plane * p.tiles;  // plane = n * c1 + cb
  const uint32_t n = p.div_c1.div(plane), cb = plane - n * p.c1;
  const uint32_t pix0 = t * TILE;
  const uint32_t count = min((uint32_t)TILE, p.hw - pix0);
  // load: 16 channel rows x count pixels
  if (p.vec_ok && count == TILE) {
    // every vector of the thread in flight before the first is staged: one
    // memory round trip per block rather than one per vector
    constexpr uint32_t kPer = 16 * (TILE / 8) / kThreads;
    static_assert(kPer * kThreads == 16 * (TILE / 8), "whole vectors per thread");
    u32x4 v[kPer];
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t k = threadIdx.x + i * kThreads;
      const uint32_t c = k / (TILE / 8), j = k % (TILE / 8);
      const uint32_t ch = min(cb * 16 + c, p.channels - 1);  // channels past C: loaded, then zeroed
      v[i] = ld16s<NT>(p.x + n * p.x_n + (int64_t)ch * p.x_c + pix0 + j * 8);
    }
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t k = threadIdx.x + i * kThreads;
      const uint32_t c = k / (TILE / 8), j = k % (TILE / 8);
      const u32x4 w = cb * 16 + c < p.channels ? v[i] : (u32x4){0u, 0u, 0u, 0u};
      const uint16_t* h = reinterpret_cast<const uint16_t*>(&w);
#pragma unroll
      for (int q = 0; q < 8; ++q) tile[c][j * 8 + q] = h[q];
    }
  } else {
    for (uint32_t k = threadIdx.x; k < 16 * TILE; k += kThreads) {
      const uint32_t c = k / TILE, j = k % TILE;
      const uint32_t ch = cb * 16 + c;
      uint16_t v = 0;
      if (ch < p.channels && j < count) v = p.x[n * p.x_n + (int64_t)ch * p.x_c + (int64_t)(pix0 + j) * p.x_hw];
      tile[c][j] = v;
    }
  }
  __syncthreads();
  // store: count pixels x 16 channels, dense in the output plane
  uint16_t* yp = p.y + n * p.y_n + (int64_t)cb * p.y_c1 + (int64_t)pix0 * 16;
  for (uint32_t k = threadIdx.x; k < count * 2; k += kThreads) {
    const uint32_t pix = k >> 1, half = k & 1;
    uint16_t h[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) h[q] = tile[half * 8 + q][pix];
    st16<NT>(yp + (size_t)k * 8, __builtin_bit_cast(u32x4, h));
  }
}

// unpack: NC1HWC0 -> NCHW for channels < C
__global__ __launch_bounds__(kThreads) void unpack_kernel(PackPlan p) {
  __shared__ uint16_t tile[16][kTile + 2];
  const uint32_t plane = p.div_tiles.div(blockIdx.x), t = blockIdx.x - plane * p.tiles;
  const uint32_t n = p.div_c1.div(plane), cb = plane - n * p.c1;
  const uint32_t pix0 = t * kTile;
  const uint32_t count = min((uint32_t)kTile, p.hw - pix0);
  const uint16_t* xp = p.y + n * p.y_n + (int64_t)cb * p.y_c1 + (int64_t)pix0 * 16;  // y holds the blocked source
  for (uint32_t k = threadIdx.x; k < count * 2; k += kThreads) {
    const uint32_t pix = k >> 1, half = k & 1;
    u32x4 v = ld16(xp + (size_t)k * 8);
    const uint16_t* h = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
    for (int q = 0; q < 8; ++q) tile[half * 8 + q][pix] = h[q];
  }
  __syncthreads();
  uint16_t* out = const_cast<uint16_t*>(p.x);  // x holds the NCHW destination
  if (p.vec_ok && count == kTile) {
    for (uint32_t k = threadIdx.x; k < 16 * (kTile / 8); k += kThreads) {
      const uint32_t c = k / (kTile / 8), j = k % (kTile / 8);
      const uint32_t ch = cb * 16 + c;
      if (ch >= p.channels) continue;
      uint16_t h[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) h[q] = tile[c][j * 8 + q];
      *reinterpret_cast<u32x4*>(out + n * p.x_n + (int64_t)ch * p.x_c + pix0 + j * 8) =
          __builtin_bit_cast(u32x4, h);
    }
  } else {
    for (uint32_t k = threadIdx.x; k < 16 * kTile; k += kThreads) {
      const uint32_t c = k / kTile, j = k % kTile;
      const uint32_t ch = cb * 16 + c;
      if (ch < p.channels && j < count)
        out[n * p.x_n + (int64_t)ch * p.x_c + (int64_t)(pix0 + j) * p.x_hw] = tile[c][j];
    }
  }
}

// NCHW descriptor -> (n, c, hw) strides when H and W merge into one pixel axis.
bool pixels_axis(const thin_desc* x, int64_t& hw_stride) {
  const int64_t h = x->sizes[2], w = x->sizes[3];
  if (h == 1) { hw_stride = w == 1 ? 1 : x->strides[3]; return true; }
  if (w == 1) { hw_stride = x->strides[2]; return true; }
  if (x->strides[2] != w * x->strides[3]) return false;
  hw_stride = x->strides[3];
  return true;
}

thin_status repack(const thin_desc* nchw, const thin_desc* blocked, bool to_blocked, hipStream_t stream) {
  THIN_REQUIRE(desc_valid(nchw) && desc_valid(blocked), THIN_ERR_INVALID, "repack: invalid descriptor");
  THIN_REQUIRE(nchw->rank == 4 && blocked->rank == 5 && blocked->sizes[4] == 16, THIN_ERR_INVALID,
               "repack expects NCHW [N,C,H,W] and NC1HWC0 [N,C1,H,W,16]");
  THIN_REQUIRE(dtype_size(nchw->dtype) == 2 && nchw->dtype == blocked->dtype, THIN_ERR_INVALID,
               "repack supports 16-bit elements (float16) with matching dtypes");
  const int64_t n = nchw->sizes[0], c = nchw->sizes[1], h = nchw->sizes[2], w = nchw->sizes[3];
  const int64_t c1 = (c + 15) / 16;
  THIN_REQUIRE(blocked->sizes[0] == n && blocked->sizes[2] == h && blocked->sizes[3] == w,
               THIN_ERR_INVALID, "repack: N/H/W mismatch");
  if (to_blocked)
    THIN_REQUIRE(blocked->sizes[1] == c1, THIN_ERR_INVALID, "pack: C1 must be ceil(C/16)");
  else
    THIN_REQUIRE(blocked->sizes[1] * 16 >= c && blocked->sizes[1] == c1, THIN_ERR_INVALID,
                 "unpack: C must satisfy ceil(C/16) == C1");
  if (n * c1 * h * w == 0) return THIN_OK;
  const bool bdense = (w == 1 || blocked->strides[3] == 16) && (h == 1 || blocked->strides[2] == w * 16) &&
                      blocked->strides[4] == 1 && aligned16(blocked->data) && blocked->strides[0] % 8 == 0 &&
                      blocked->strides[1] % 8 == 0;
  int64_t hw_stride = 0;
  const bool pix = pixels_axis(nchw, hw_stride);
  // channels-last NCHW (channel stride 1): the tiled kernel below reads
  // pixels along its lanes, which there lie C elements apart
  const bool chan_last = nchw->strides[1] == 1 && c > 1 && c % 16 == 0;
  if (!bdense || !pix || chan_last) {
    // general strides: the strided copy through the 5-D view of NCHW
    // (x[n, c1*16+k, h, w] <-> y[n, c1, h, w, k]), whose kernels coalesce and
    // vectorise what the layouts share (a channels-last x moves 32-byte C0
    // runs: [32,64,80,80] 205 us through an element-wise index map); channels
    // >= C of a pack must read as zero, which a view cannot express, so
    // require C % 16.
    THIN_REQUIRE(c % 16 == 0 || !to_blocked, THIN_ERR_UNSUPPORTED,
                 "pack: non-dense layouts need C %% 16 == 0");
    thin_desc v5 = *nchw;
    v5.rank = 5;
    const int64_t cs = nchw->strides[1];
    v5.sizes[0] = n; v5.strides[0] = nchw->strides[0];
    v5.sizes[1] = to_blocked ? c1 : blocked->sizes[1]; v5.strides[1] = cs * 16;
    v5.sizes[2] = h; v5.strides[2] = nchw->strides[2];
    v5.sizes[3] = w; v5.strides[3] = nchw->strides[3];
    v5.sizes[4] = 16; v5.strides[4] = cs;
    if (to_blocked) return copy_bits(&v5, blocked, stream);
    // unpack of the first C channels only
    thin_desc b5 = *blocked;
    if (c % 16 == 0) return copy_bits(blocked, &v5, stream);
    // partial last block: full blocks, then the tail channels
    THIN_REQUIRE(false, THIN_ERR_UNSUPPORTED, "unpack: non-dense layout with C %% 16 != 0");
    (void)b5;
  }
  PackPlan p;
  p.x = static_cast<const uint16_t*>(nchw->data);
  p.y = static_cast<uint16_t*>(blocked->data);
  p.x_n = nchw->strides[0];
  p.x_c = nchw->strides[1];
  p.x_hw = hw_stride;
  p.y_n = blocked->strides[0];
  p.y_c1 = blocked->strides[1];
  p.channels = (uint32_t)c;
  p.c1 = (uint32_t)c1;
  p.hw = (uint32_t)(h * w);
  p.vec_ok = (hw_stride == 1 && aligned16(nchw->data) && nchw->strides[0] % 8 == 0 && nchw->strides[1] % 8 == 0)
                 ? 1u : 0u;
  const uint64_t wide_blocks = (uint64_t)n * c1 * ((p.hw + kWideTile - 1) / kWideTile);
  const bool wide = to_blocked && wide_blocks >= 2048;
  const int tile_px = wide ? kWideTile : kTile;
  p.tiles = (p.hw + tile_px - 1) / tile_px;
  const uint64_t blocks = (uint64_t)n * c1 * p.tiles;
  THIN_REQUIRE(blocks < (1ull << 31), THIN_ERR_UNSUPPORTED, "repack: too many tiles");
  p.div_tiles = FastDiv::make(p.tiles);
  p.div_c1 = FastDiv::make(p.c1);
  const bool nt = n * c1 * h * w * 32 >= kStreamingBytes;
  if (wide && nt)
    hipLaunchKernelGGL((pack_kernel<true, kWideTile>), dim3((uint32_t)blocks), dim3(kThreads), 0, stream, p);
  else if (wide)
    hipLaunchKernelGGL((pack_kernel<false, kWideTile>), dim3((uint32_t)blocks), dim3(kThreads), 0, stream, p);
  else if (to_blocked && nt)
    hipLaunchKernelGGL((pack_kernel<true, kTile>), dim3((uint32_t)blocks), dim3(kThreads), 0, stream, p);
  else if (to_blocked)
    hipLaunchKernelGGL((pack_kernel<false, kTile>), dim3((uint32_t)blocks), dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(unpack_kernel, dim3((uint32_t)blocks), dim3(kThreads), 0, stream, p);
  THIN_LAUNCH_CHECK("repack");
  return THIN_OK;
}

}  // namespace
}  // namespace thin

using namespace thin;

extern "C" thin_status thin_cat(const thin_desc* inputs, int32_t n, int32_t dim, const thin_desc* out,
                                hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(inputs && out && n >= 1 && n <= THIN_MAX_CAT_INPUTS, THIN_ERR_INVALID,
               "cat: 1..%d inputs required", THIN_MAX_CAT_INPUTS);
  THIN_REQUIRE(desc_valid(out), THIN_ERR_INVALID, "cat: invalid output descriptor");
  THIN_REQUIRE(dim >= 0 && dim < out->rank, THIN_ERR_INVALID, "cat: dim %d out of range", dim);
  const int esize = dtype_size(out->dtype);
  int64_t total = 0;
  for (int k = 0; k < n; ++k) {
    const thin_desc* t = &inputs[k];
    THIN_REQUIRE(desc_valid(t), THIN_ERR_INVALID, "cat: invalid input %d", k);
    THIN_REQUIRE(t->dtype == out->dtype, THIN_ERR_INVALID, "cat requires matching dtypes");
    THIN_REQUIRE(t->rank == out->rank, THIN_ERR_INVALID, "cat rank mismatch");
    for (int d = 0; d < t->rank; ++d)
      THIN_REQUIRE(d == dim || t->sizes[d] == out->sizes[d], THIN_ERR_INVALID,
                   "cat shape mismatch outside concatenation dimension");
    total += t->sizes[dim];
  }
  THIN_REQUIRE(total == out->sizes[dim], THIN_ERR_INVALID, "cat: output size along dim %d is %lld, inputs sum to %lld",
               dim, (long long)out->sizes[dim], (long long)total);
  if (numel(out) == 0) return THIN_OK;

  // Fused launch for inputs whose rows are dense, when the output is dense.
  const bool out_dense = is_contiguous(out);
  int64_t inner = 1;
  for (int d = dim + 1; d < out->rank; ++d) inner *= out->sizes[d];
  const bool nt = numel(out) * esize >= kStreamingBytes;
  const bool out_vec = aligned16(out->data) && (out->sizes[dim] * inner * esize) % 16 == 0;
  const thin_desc* vec_in[kCatPerLaunch];
  int64_t vec_col[kCatPerLaunch];
  int nv = 0;
  const thin_desc* el_in[kCatPerLaunch];
  int64_t el_col[kCatPerLaunch];
  int ne = 0;
  int64_t col = 0;
  thin_status s = THIN_OK;
  auto flush = [&](bool vec) -> thin_status {
    thin_status st = THIN_OK;
    if (vec && nv) {
      st = launch_cat_group<u32x4>(vec_in, nv, dim, out, vec_col, esize, nt, stream);
      nv = 0;
    }
    if (!vec && ne) {
      switch (esize) {
        case 1: st = launch_cat_group<uint8_t>(el_in, ne, dim, out, el_col, esize, false, stream); break;
        case 2: st = launch_cat_group<uint16_t>(el_in, ne, dim, out, el_col, esize, false, stream); break;
        case 4: st = launch_cat_group<uint32_t>(el_in, ne, dim, out, el_col, esize, false, stream); break;
        default: st = launch_cat_group<uint64_t>(el_in, ne, dim, out, el_col, esize, false, stream); break;
      }
      ne = 0;
    }
    return st;
  };
  for (int k = 0; k < n; ++k) {
    const thin_desc* t = &inputs[k];
    const int64_t seg = t->sizes[dim];
    if (seg == 0 || numel(t) == 0) continue;
    // a block per row run: runs under kCatShortRun would leave most of its
    // lanes idle, so those inputs take the strided copy below, whose kernels
    // pack many rows into a block (2 x [32,64,80,40] along the last dim, 80-byte
    // runs: 333 us through blocks per run)
    if (out_dense && run_dense(t, dim) && seg * inner * esize >= kCatShortRun) {
      bool vec = out_vec && aligned16(t->data) && (seg * inner * esize) % 16 == 0 && (col * inner * esize) % 16 == 0;
      for (int d = 0; vec && d < dim; ++d) vec = (t->strides[d] * esize) % 16 == 0 || t->sizes[d] == 1;
      if (vec) {
        vec_in[nv] = t;
        vec_col[nv++] = col * inner;
        if (nv == kCatPerLaunch && (s = flush(true))) return s;
      } else {
        el_in[ne] = t;
        el_col[ne++] = col * inner;
        if (ne == kCatPerLaunch && (s = flush(false))) return s;
      }
    } else {
      // strided leftover: copy into the output slice out.narrow(dim, col, seg)
      thin_desc slice = *out;
      slice.sizes[dim] = seg;
      slice.data = static_cast<char*>(out->data) + col * out->strides[dim] * esize;
      if ((s = copy_bits(t, &slice, stream))) return s;
    }
    col += seg;
  }
  if ((s = flush(true))) return s;
  return flush(false);
}

extern "C" thin_status thin_upsample_cat_nc1hwc0(const thin_desc* inputs, const int32_t* upsample, int32_t n,
                                                 const thin_desc* out, hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(inputs && out && n >= 1 && n <= kPlaneInputs, THIN_ERR_INVALID,
               "upsample_cat: 1..%d inputs required", kPlaneInputs);
  THIN_REQUIRE(desc_valid(out) && out->rank == 5, THIN_ERR_INVALID, "upsample_cat: NC1HWC0 output required");
  const int esize = dtype_size(out->dtype);
  int64_t c1 = 0;
  bool fast = plane_dense(out, esize);
  for (int k = 0; k < n; ++k) {
    const thin_desc* t = &inputs[k];
    const bool up = upsample && upsample[k];
    THIN_REQUIRE(desc_valid(t) && t->rank == 5 && t->dtype == out->dtype, THIN_ERR_INVALID,
                 "upsample_cat: input %d must be NC1HWC0 with the output dtype", k);
    THIN_REQUIRE(t->sizes[0] == out->sizes[0] && t->sizes[4] == out->sizes[4] &&
                 t->sizes[2] * (up ? 2 : 1) == out->sizes[2] && t->sizes[3] * (up ? 2 : 1) == out->sizes[3],
                 THIN_ERR_INVALID, "upsample_cat: input %d has incompatible N/H/W/C0", k);
    fast = fast && plane_dense(t, esize);
    c1 += t->sizes[1];
  }
  THIN_REQUIRE(c1 == out->sizes[1], THIN_ERR_INVALID, "upsample_cat: C1 of inputs sum to %lld, output has %lld",
               (long long)c1, (long long)out->sizes[1]);
  if (numel(out) == 0) return THIN_OK;
  if (fast) return launch_planes(inputs, upsample, n, out, stream);
  // general strides: per-input element map into the output slice
  int64_t off = 0;
  for (int k = 0; k < n; ++k) {
    thin_desc slice = *out;
    slice.sizes[1] = inputs[k].sizes[1];
    slice.data = static_cast<char*>(out->data) + off * out->strides[1] * esize;
    thin_status s = launch_up5(&inputs[k], &slice, upsample && upsample[k], stream);
    if (s) return s;
    off += inputs[k].sizes[1];
  }
  return THIN_OK;
}

extern "C" thin_status thin_upsample2x_nc1hwc0(const thin_desc* x, const thin_desc* y, hipStream_t stream) {
  const int32_t up = 1;
  return thin_upsample_cat_nc1hwc0(x, &up, 1, y, stream);
}

extern "C" thin_status thin_upsample2x_nchw(const thin_desc* x, const thin_desc* y, hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(desc_valid(x) && desc_valid(y) && x->rank == 4 && y->rank == 4, THIN_ERR_INVALID,
               "upsample2x_nchw expects NCHW tensors");
  THIN_REQUIRE(x->dtype == y->dtype, THIN_ERR_INVALID, "upsample2x_nchw requires matching dtypes");
  THIN_REQUIRE(y->sizes[0] == x->sizes[0] && y->sizes[1] == x->sizes[1] && y->sizes[2] == 2 * x->sizes[2] &&
               y->sizes[3] == 2 * x->sizes[3], THIN_ERR_INVALID, "upsample2x_nchw: output must be [N,C,2H,2W]");
  if (numel(y) == 0) return THIN_OK;
  const int esize = dtype_size(y->dtype);
  const int64_t ow = y->sizes[3];
  const bool vec = (esize == 2 || esize == 4) && (ow * esize) % 16 == 0 && x->strides[3] == 1 &&
                   y->strides[3] == 1 && aligned16(y->data) && (y->strides[0] * esize) % 16 == 0 &&
                   (y->strides[1] * esize) % 16 == 0 && (y->strides[2] * esize) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(x->data) % 8 == 0 && (x->strides[0] * esize) % 8 == 0 &&
                   (x->strides[1] * esize) % 8 == 0 && (x->strides[2] * esize) % 8 == 0;
  const uint64_t rows = (uint64_t)y->sizes[0] * y->sizes[1] * y->sizes[2];
  const uint64_t in_elems = (uint64_t)numel(x);
  const bool pair = (esize == 2 || esize == 4) && y->strides[3] == 1 && y->strides[0] % 2 == 0 &&
                    y->strides[1] % 2 == 0 && y->strides[2] % 2 == 0 &&
                    reinterpret_cast<uintptr_t>(y->data) % (2 * esize) == 0 && in_elems < (1ull << 31);
  if (!vec && pair) {
    NchwPairPlan p;
    p.src = static_cast<const char*>(x->data);
    p.dst = static_cast<char*>(y->data);
    p.s_n = x->strides[0] * esize; p.s_c = x->strides[1] * esize;
    p.s_h = x->strides[2] * esize; p.s_w = x->strides[3] * esize;
    p.d_n = y->strides[0] * esize; p.d_c = y->strides[1] * esize; p.d_h = y->strides[2] * esize;
    p.w = (uint32_t)x->sizes[3];
    p.h = (uint32_t)x->sizes[2];
    p.c = (uint32_t)x->sizes[1];
    p.total = (uint32_t)in_elems;
    p.div_w = FastDiv::make(p.w);
    p.div_h = FastDiv::make(p.h);
    p.div_c = FastDiv::make(p.c);
    const uint32_t grid = grid_for(in_elems, kThreads, 1, 256u * 16u);
    typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    if (esize == 2) hipLaunchKernelGGL((nchw_up_pair_kernel<uint16_t, u16x2>), dim3(grid), dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((nchw_up_pair_kernel<uint32_t, u32x2>), dim3(grid), dim3(kThreads), 0, stream, p);
    THIN_LAUNCH_CHECK("upsample2x_nchw_pairs");
    return THIN_OK;
  }
  if (!vec || rows * (uint64_t)(ow * esize / 16) >= (1ull << 31)) {
    thin_desc x5 = *x, y5 = *y;
    x5.rank = y5.rank = 5;
    x5.sizes[4] = y5.sizes[4] = 1;
    x5.strides[4] = y5.strides[4] = 1;
    // NCHW as [N, C, H, W, 1]: the 5-D index map upsamples axes 2 and 3.
    return launch_up5(&x5, &y5, true, stream);
  }
  NchwUpPlan p;
  p.src = static_cast<const char*>(x->data);
  p.dst = static_cast<char*>(y->data);
  p.s_n = x->strides[0] * esize; p.s_c = x->strides[1] * esize; p.s_h = x->strides[2] * esize;
  p.d_n = y->strides[0] * esize; p.d_c = y->strides[1] * esize; p.d_h = y->strides[2] * esize;
  p.c = (uint32_t)y->sizes[1];
  p.oh = (uint32_t)y->sizes[2];
  p.row_vecs = (uint32_t)(ow * esize / 16);
  p.rows = (uint32_t)rows;
  p.div_row_vecs = FastDiv::make(p.row_vecs);
  p.div_oh = FastDiv::make(p.oh);
  p.div_c = FastDiv::make(p.c);
  const bool nt = numel(y) * esize >= kStreamingBytes;
  const uint32_t grid = grid_for(rows * p.row_vecs, kThreads, 1, 256u * 16u);
  if (esize == 2) {
    if (nt) hipLaunchKernelGGL((nchw_up_kernel<uint16_t, true>), dim3(grid), dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((nchw_up_kernel<uint16_t, false>), dim3(grid), dim3(kThreads), 0, stream, p);
  } else {
    if (nt) hipLaunchKernelGGL((nchw_up_kernel<uint32_t, true>), dim3(grid), dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((nchw_up_kernel<uint32_t, false>), dim3(grid), dim3(kThreads), 0, stream, p);
  }
  THIN_LAUNCH_CHECK("nchw_up");
  return THIN_OK;
}

extern "C" thin_status thin_pack_nc1hwc0(const thin_desc* x, const thin_desc* y, hipStream_t stream) {
  clear_error();
  return repack(x, y, true, stream);
}

extern "C" thin_status thin_unpack_nc1hwc0(const thin_desc* x, const thin_desc* y, hipStream_t stream) {
  clear_error();
  return repack(y, x, false, stream);
}

extern "C" thin_status thin_maxpool_nc1hwc0(const thin_desc* x, int32_t kernel, const thin_desc* out,
                                            hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(desc_valid(x) && desc_valid(out), THIN_ERR_INVALID, "maxpool: invalid descriptor");
  THIN_REQUIRE(x->dtype == THIN_F16 && out->dtype == THIN_F16 && x->rank == 5 && x->sizes[4] == 16 &&
               same_sizes(x, out), THIN_ERR_INVALID, "maxpool expects float16 NC1HWC0 x and out of one shape");
  THIN_REQUIRE(pool_kernel_ok(kernel), THIN_ERR_INVALID, "maxpool kernel must be an odd integer in [1, 15]");
  if (numel(out) == 0) return THIN_OK;
  for (const thin_desc* d : {x, out})
    THIN_REQUIRE(d->strides[4] == 1 && (d->sizes[3] == 1 || d->strides[3] == 16) &&
                 reinterpret_cast<uintptr_t>(d->data) % 16 == 0 && d->strides[0] % 8 == 0 &&
                 d->strides[1] % 8 == 0 && d->strides[2] % 8 == 0, THIN_ERR_UNSUPPORTED,
                 "maxpool needs 16-byte aligned pixels (C0 dense, W stride 16)");
  THIN_REQUIRE(x->sizes[2] < (1 << 30) && x->sizes[3] < (1 << 30), THIN_ERR_UNSUPPORTED, "maxpool: plane too large");
  {
    // planes that fit one block's LDS: the whole-plane kernel with one pool
    // (SPPF k5 [32,256,20,20]: 5.2 us, against 7.5 us with row bands)
    if (sppf_whole_plane(x, out, kernel / 2)) return launch_sppf(x, kernel, 1, true, out, stream);
  }
  PoolPlan p;
  memset(&p, 0, sizeof p);
  p.x = static_cast<const char*>(x->data);
  p.y = static_cast<char*>(out->data);
  for (int d = 0; d < 4; ++d) {
    p.xs[d] = x->strides[d];
    p.ys[d] = out->strides[d];
  }
  p.xs[3] = p.ys[3] = 16;
  p.c = (uint32_t)x->sizes[1];
  p.h = (uint32_t)x->sizes[2];
  p.w = (uint32_t)x->sizes[3];
  p.parts = 2;
  return launch_pool<_Float16, 8>(p, (uint32_t)(x->sizes[0] * x->sizes[1]), kernel, stream);
}

extern "C" thin_status thin_sppf_nc1hwc0(const thin_desc* x, int32_t kernel, int32_t repeats, const thin_desc* out,
                                         hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(desc_valid(x) && desc_valid(out), THIN_ERR_INVALID, "sppf: invalid descriptor");
  THIN_REQUIRE(x->dtype == THIN_F16 && out->dtype == THIN_F16 && x->rank == 5 && out->rank == 5 &&
               x->sizes[4] == 16 && out->sizes[4] == 16, THIN_ERR_INVALID,
               "sppf expects float16 NC1HWC0 x and out");
  THIN_REQUIRE(pool_kernel_ok(kernel), THIN_ERR_INVALID, "sppf kernel must be an odd integer in [1, 15]");
  THIN_REQUIRE(repeats >= 1 && repeats <= 8, THIN_ERR_INVALID, "sppf repeats must be in [1, 8]");
  const int64_t N = x->sizes[0], C1 = x->sizes[1], H = x->sizes[2], W = x->sizes[3];
  THIN_REQUIRE(out->sizes[0] == N && out->sizes[1] == (repeats + 1) * C1 && out->sizes[2] == H && out->sizes[3] == W,
               THIN_ERR_INVALID, "sppf: out must be [N, (repeats + 1) * C1, H, W, 16] for x [N, C1, H, W, 16]");
  if (numel(out) == 0) return THIN_OK;
  for (const thin_desc* d : {x, out})
    THIN_REQUIRE(d->strides[4] == 1 && (d->sizes[3] == 1 || d->strides[3] == 16) &&
                 reinterpret_cast<uintptr_t>(d->data) % 16 == 0 && d->strides[0] % 8 == 0 &&
                 d->strides[1] % 8 == 0 && d->strides[2] % 8 == 0, THIN_ERR_UNSUPPORTED,
                 "sppf needs 16-byte aligned pixels (C0 dense, W stride 16)");
  THIN_REQUIRE(H < (1 << 30) && W < (1 << 30), THIN_ERR_UNSUPPORTED, "sppf: plane too large");
  if (!sppf_whole_plane(x, out, kernel / 2)) {
    // planes beyond one block's LDS: the copy and the chained pools, each
    // reading the previous output slot
    auto slot = [&](int r) {
      thin_desc d = *out;
      d.sizes[1] = C1;
      d.data = static_cast<char*>(out->data) + (int64_t)r * C1 * out->strides[1] * 2;
      return d;
    };
    thin_desc s0 = slot(0);
    thin_status st = thin_copy(x, &s0, stream);
    if (st != THIN_OK) return st;
    for (int r = 1; r <= repeats; ++r) {
      thin_desc a = slot(r - 1), b = slot(r);
      st = thin_maxpool_nc1hwc0(&a, kernel, &b, stream);
      if (st != THIN_OK) return st;
    }
    return THIN_OK;
  }
  return launch_sppf(x, kernel, repeats, false, out, stream);
}

extern "C" thin_status thin_maxpool2d_nchw(const thin_desc* x, int32_t kernel, const thin_desc* out,
                                           hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(desc_valid(x) && desc_valid(out), THIN_ERR_INVALID, "maxpool2d: invalid descriptor");
  THIN_REQUIRE((x->dtype == THIN_F16 || x->dtype == THIN_F32) && out->dtype == x->dtype && x->rank == 4 &&
               same_sizes(x, out), THIN_ERR_INVALID, "maxpool2d expects float16/float32 NCHW x and out of one shape");
  THIN_REQUIRE(pool_kernel_ok(kernel), THIN_ERR_INVALID, "maxpool2d kernel must be an odd integer in [1, 15]");
  if (numel(out) == 0) return THIN_OK;
  THIN_REQUIRE(x->sizes[0] * x->sizes[1] < (1ll << 31) && x->sizes[2] < (1 << 30) && x->sizes[3] < (1 << 30),
               THIN_ERR_UNSUPPORTED, "maxpool2d: tensor too large");
  PoolPlan p;
  memset(&p, 0, sizeof p);
  p.x = static_cast<const char*>(x->data);
  p.y = static_cast<char*>(out->data);
  for (int d = 0; d < 4; ++d) {
    p.xs[d] = x->strides[d];
    p.ys[d] = out->strides[d];
  }
  p.c = (uint32_t)x->sizes[1];
  p.h = (uint32_t)x->sizes[2];
  p.w = (uint32_t)x->sizes[3];
  p.parts = 1;
  const uint32_t planes = (uint32_t)(x->sizes[0] * x->sizes[1]);
  if (x->dtype == THIN_F16) return launch_pool<_Float16, 1>(p, planes, kernel, stream);
  return launch_pool<float, 1>(p, planes, kernel, stream);
}
