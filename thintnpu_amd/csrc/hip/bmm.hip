// Attention contractions: the batched fp16 product of strided or
// channel-blocked operands (with head groups and channel ranges) and the
// blocked channel gather that feeds it.
//
// The product keeps the reference's numerical contract: every output is the
// fp32 sum of its k products taken in reduction order 0, 1, ..., K-1 from a
// zero start, then one round-to-nearest-even cast to fp16.  fp16 x fp16
// products are exact in fp32 (22 significant bits, exponents far from the fp32
// limits), so fma(a, b, acc) rounds exactly like acc + a * b and the per-output
// chain of fmas reproduces the sequential sum bit for bit.  This rules out
// MFMA tiles (their internal summation order differs) and any split of the
// reduction; the parallelism is across outputs only.  The attention shapes are
// small (a [4, 64, 400] x [4, 400, 400] product is 41 M fmas), so a product
// is bound by the latency of its K-long dependent fma chains (about 32 cycles
// per dependent fp32 fma on gfx950) and by memory latency, not by VALU
// throughput.
#include "common.h"

#include <string.h>

namespace thin {
namespace {

// One axis of a logical matrix: index i sits at element offset
// (i / blk) * outer + (i % blk) * inner.
struct Axis {
  FastDiv blk;
  int64_t outer, inner;
  __device__ __forceinline__ int64_t at(uint32_t i) const {
    const uint32_t q = blk.div(i);
    return (int64_t)q * outer + (int64_t)(i - q * blk.d) * inner;
  }
};

// A logical [batch, rows, cols] matrix over fp16 storage (bmm_flow.cpp:19-33,
// 193-215): element (b, r, c) sits at b * batch + row.at(r + row_origin +
// b * row_group) + col.at(c + col_origin + b * col_group).  Head groups of a
// blocked operand have batch stride 0 and a per-group channel origin.
struct Mat {
  _Float16* p;
  int64_t batch;
  uint32_t row_origin, col_origin, row_group, col_group;
  Axis row, col;
  __device__ __forceinline__ int64_t at(uint32_t b, uint32_t r, uint32_t c) const {
    return (int64_t)b * batch + row.at(r + row_origin + b * row_group) + col.at(c + col_origin + b * col_group);
  }
};

constexpr uint32_t kBmmThreads = 256;  // 4 waves; wave w owns rows [w * RM, w * RM + RM) of the tile
constexpr uint32_t kBmmCols = 64;      // one output column per lane
constexpr uint32_t kBmmDepth = 32;     // reduction steps staged per LDS round

struct BmmPlan {
  Mat a, b, y;          // a: [batch, m, k], b: [batch, k, n], y: [batch, m, n]
  uint32_t m, n, k;
  uint32_t mtiles, ntiles;
  bool a_kfast, b_kfast;  // stage along k (the operand's smaller stride is on k)
  // streamed b: bytes from b.p to the end of its storage, vectors per
  // contiguous run along k (0 = one run) and the byte jump after a run
  uint32_t b_bytes, b_vrun, b_vjump;
  FastDiv div_mt, div_nt;  // streamed form: block index -> (batch, row tile, column tile)
};

// Output tile of 4 * RM rows x 64 columns per block.  A and B are staged as
// fp32 in LDS, kBmmDepth reduction steps at a time; each step is one LDS
// column read per lane, RM broadcast reads and RM fmas.
template <int RM>
__global__ __launch_bounds__(kBmmThreads) void bmm_kernel(BmmPlan p) {
  constexpr uint32_t TM = 4 * RM;
  constexpr uint32_t kAPitch = TM + 4;  // wave w's RM floats stay 4*RM-byte aligned
  constexpr uint32_t kBPitch = kBmmCols + 1;
  __shared__ __attribute__((aligned(16))) float As[kBmmDepth][kAPitch];
  __shared__ float Bs[kBmmDepth][kBPitch];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  uint32_t t = blockIdx.x;
  const uint32_t nt = t % p.ntiles;
  t /= p.ntiles;
  const uint32_t mt = t % p.mtiles;
  const uint32_t bt = t / p.mtiles;
  const uint32_t i0 = mt * TM, j0 = nt * kBmmCols;

  // B staging: each thread's columns are fixed for the whole block
  int64_t bcol[kBmmDepth * kBmmCols / kBmmThreads];
  constexpr uint32_t kBPer = kBmmDepth * kBmmCols / kBmmThreads;  // 8
#pragma unroll
  for (uint32_t s = 0; s < kBPer; ++s) {
    const uint32_t e = tid + s * kBmmThreads;
    const uint32_t jj = p.b_kfast ? e / kBmmDepth : e % kBmmCols;
    const uint32_t j = min(j0 + jj, p.n - 1);
    bcol[s] = (int64_t)bt * p.b.batch + p.b.col.at(j + p.b.col_origin + bt * p.b.col_group);
  }

  float acc[RM];
#pragma unroll
  for (int r = 0; r < RM; ++r) acc[r] = 0.f;

  for (uint32_t k0 = 0; k0 < p.k; k0 += kBmmDepth) {
    const uint32_t kc = min(kBmmDepth, p.k - k0);
    // all staging loads in flight at once: clamped addresses, then predicated
    // LDS stores
    constexpr uint32_t kAPer = (TM * kBmmDepth + kBmmThreads - 1) / kBmmThreads;
    _Float16 av[kAPer], bv[kBPer];
#pragma unroll
    for (uint32_t s = 0; s < kAPer; ++s) {
      const uint32_t e = min(tid + s * kBmmThreads, TM * kBmmDepth - 1);
      const uint32_t kk = p.a_kfast ? e % kBmmDepth : e / TM;
      const uint32_t ii = p.a_kfast ? e / kBmmDepth : e % TM;
      av[s] = p.a.p[p.a.at(bt, min(i0 + ii, p.m - 1), k0 + min(kk, kc - 1))];
    }
#pragma unroll
    for (uint32_t s = 0; s < kBPer; ++s) {
      const uint32_t e = tid + s * kBmmThreads;
      const uint32_t kk = p.b_kfast ? e % kBmmDepth : e / kBmmCols;
      bv[s] = p.b.p[bcol[s] + p.b.row.at(k0 + min(kk, kc - 1) + p.b.row_origin + bt * p.b.row_group)];
    }
#pragma unroll
    for (uint32_t s = 0; s < kAPer; ++s) {
      const uint32_t e = tid + s * kBmmThreads;
      const uint32_t kk = p.a_kfast ? e % kBmmDepth : e / TM;
      const uint32_t ii = p.a_kfast ? e / kBmmDepth : e % TM;
      if (e < TM * kBmmDepth && kk < kc) As[kk][ii] = (float)av[s];
    }
#pragma unroll
    for (uint32_t s = 0; s < kBPer; ++s) {
      const uint32_t e = tid + s * kBmmThreads;
      const uint32_t kk = p.b_kfast ? e % kBmmDepth : e / kBmmCols;
      const uint32_t jj = p.b_kfast ? e / kBmmDepth : e % kBmmCols;
      if (kk < kc) Bs[kk][jj] = (float)bv[s];
    }
    __syncthreads();
#pragma unroll 8
    for (uint32_t kk = 0; kk < kc; ++kk) {
      const float bv = Bs[kk][lane];
#pragma unroll
      for (int r = 0; r < RM; ++r) acc[r] = __builtin_fmaf(As[kk][wave * RM + r], bv, acc[r]);
    }
    __syncthreads();
  }
  const uint32_t j = j0 + lane;
  if (j >= p.n) return;
#pragma unroll
  for (int r = 0; r < RM; ++r) {
    const uint32_t i = i0 + wave * RM + r;
    if (i < p.m) p.y.p[p.y.at(bt, i, j)] = (_Float16)acc[r];
  }
}

// ---------------------------------------------------------------- streamed b
// When b holds every output column contiguously along k in 16-byte aligned
// runs of 8 or more elements (the probabilities of v p^T, the blocked keys of
// q^T k), lane j owns output column j and streams that column from memory with
// 16-byte loads: b needs no LDS and no block-wide staging.  A block is one
// wave; it stages its RM rows of a in LDS as fp32 (KS * 64 steps at a time)
// and each reduction step is RM fmas on LDS broadcasts.  The column is read in
// rounds of RV vectors (8 steps each): the first round is issued before the
// rows of a are staged, each later round loads while the previous one is
// consumed, and a whole round is consumed by straight-line code so that the
// LDS reads of one vector overlap the fmas of the previous one.  KS and RV
// are sized to K so that short reductions issue no surplus loads.
template <int RM, int KS, int RV>
__global__ __launch_bounds__(64) void bmm_stream_kernel(BmmPlan p) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  constexpr uint32_t kDepth = KS * 64;  // steps of a staged per round (a multiple of 8 * RV)
  __shared__ __attribute__((aligned(16))) float As[RM][kDepth];
  const uint32_t lane = threadIdx.x;
  uint32_t t = blockIdx.x;
  const uint32_t q = p.div_nt.div(t), nt = t - q * p.ntiles;  // no integer division sequence
  const uint32_t bt = p.div_mt.div(q), mt = q - bt * p.mtiles;
  const uint32_t i0 = mt * RM, j = nt * kBmmCols + lane;
  const _Float16* bcol = p.b.p + (int64_t)bt * p.b.batch +
                         p.b.col.at(min(j, p.n - 1) + p.b.col_origin + bt * p.b.col_group);
  const uint32_t rbase = p.b.row_origin + bt * p.b.row_group;
  // vector v of the column holds steps [8v, 8v + 8).  Loads go through a
  // buffer resource: the lane's column start is the vector offset, the step
  // offset is uniform (a scalar register) and advances by 16 bytes per vector
  // plus the run jump at each run end, so addressing costs a few scalar
  // operations per vector.  Loads past the last whole vector re-read it and
  // are not consumed.
  const uint32_t nvec = p.k / 8;
  const __amdgpu_buffer_rsrc_t brsrc = dev::buffer_rsrc(p.b.p, p.b_bytes);
  const uint32_t bvoff = (uint32_t)(bcol - p.b.p) * 2u;
  uint32_t bsoff = (uint32_t)p.b.row.at(rbase) * 2u;
  uint32_t rpos = p.b_vrun ? (rbase - p.b.row.blk.div(rbase) * p.b.row.blk.d) / 8u : 0u;
  uint32_t vaddr = 0;  // vector whose offset bsoff holds
  auto load_round = [&](h8 (&buf)[RV]) {
#pragma unroll
    for (int v = 0; v < RV; ++v) {
      buf[v] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(brsrc, bvoff, bsoff, 0));
      if (vaddr + 1 < nvec) {
        ++vaddr;
        bsoff += 16u;
        if (p.b_vrun && ++rpos == p.b_vrun) {
          rpos = 0;
          bsoff += p.b_vjump;
        }
      }
    }
  };
  h8 cur[RV], nxt[RV];
  if (nvec) load_round(cur);

  float acc[RM];
#pragma unroll
  for (int r = 0; r < RM; ++r) acc[r] = 0.f;
  typedef float f4 __attribute__((ext_vector_type(4)));
  // rows' steps kk..kk+7 of the staged a
  auto read_a = [&](f4 (&a)[RM][2], uint32_t kk) {
#pragma unroll
    for (int r = 0; r < RM; ++r) {
      a[r][0] = *reinterpret_cast<const f4*>(&As[r][kk]);
      a[r][1] = *reinterpret_cast<const f4*>(&As[r][kk + 4]);
    }
  };
  auto fmas = [&](const f4 (&a)[RM][2], const h8& v) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float bv = (float)v[q];
#pragma unroll
      for (int r = 0; r < RM; ++r) acc[r] = __builtin_fmaf(a[r][q / 4][q % 4], bv, acc[r]);
    }
  };
  auto consume = [&](const h8& v, uint32_t kk) {
    f4 a[RM][2];
    read_a(a, kk);
    fmas(a, v);
  };
  uint32_t vnext = 0;  // first vector not yet consumed (a multiple of RV between rounds)
  for (uint32_t k0 = 0; k0 < p.k; k0 += kDepth) {
    const uint32_t kc = min(kDepth, p.k - k0);
    if (k0) __syncthreads();  // the previous round's rows are no longer read
    {
      // every load of the round in flight at once: clamped addresses, then
      // predicated LDS stores
      int64_t colpart[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s)
        colpart[s] = p.a.col.at(k0 + min(lane + s * 64u, kc - 1) + p.a.col_origin + bt * p.a.col_group);
      _Float16 av[RM][KS];
#pragma unroll
      for (int r = 0; r < RM; ++r) {
        const _Float16* row = p.a.p + (int64_t)bt * p.a.batch +
                              p.a.row.at(min(i0 + r, p.m - 1) + p.a.row_origin + bt * p.a.row_group);
#pragma unroll
        for (int s = 0; s < KS; ++s) av[r][s] = row[colpart[s]];
      }
#pragma unroll
      for (int r = 0; r < RM; ++r)
#pragma unroll
        for (int s = 0; s < KS; ++s)
          if (lane + s * 64u < kc) As[r][lane + s * 64] = (float)av[r][s];
    }
    __syncthreads();
    const uint32_t vend = min(nvec, (k0 + kc) / 8);  // whole vectors inside this round
    // whole rounds: straight-line code
    while (vnext + RV <= vend) {
      const bool more = vnext + RV < nvec;
      if (more) load_round(nxt);
      // the a steps of vector v + 1 are read while vector v's fmas run
      f4 a0[RM][2], a1[RM][2];
      const uint32_t kb = vnext * 8 - k0;
      read_a(a0, kb);
#pragma unroll
      for (int v = 0; v < RV; v += 2) {
        read_a(a1, kb + (v + 1) * 8);
        fmas(a0, cur[v]);
        __builtin_amdgcn_sched_barrier(0);
        if (v + 2 < RV) read_a(a0, kb + (v + 2) * 8);
        fmas(a1, cur[v + 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (more) {
#pragma unroll
        for (int v = 0; v < RV; ++v) cur[v] = nxt[v];
      }
      vnext += RV;
    }
    // the last, partial round
    if (vnext < vend) {
#pragma unroll
      for (int v = 0; v < RV; ++v)
        if (vnext + v < vend) consume(cur[v], (vnext + v) * 8 - k0);
      vnext = vend;
    }
    // steps past the last whole vector
    for (uint32_t kk = max(k0, nvec * 8); kk < k0 + kc; ++kk) {
      const float bv = (float)bcol[p.b.row.at(rbase + kk)];
#pragma unroll
      for (int r = 0; r < RM; ++r) acc[r] = __builtin_fmaf(As[r][kk - k0], bv, acc[r]);
    }
  }
  if (j >= p.n) return;
#pragma unroll
  for (int r = 0; r < RM; ++r) {
    const uint32_t i = i0 + r;
    if (i < p.m) p.y.p[p.y.at(bt, i, j)] = (_Float16)acc[r];
  }
}

template <int RM>
void launch_stream(const BmmPlan& p, uint32_t grid, hipStream_t stream) {
  if (p.k <= 32)
    hipLaunchKernelGGL((bmm_stream_kernel<RM, 1, 4>), dim3(grid), dim3(64), 0, stream, p);
  else if (p.k <= 64)
    hipLaunchKernelGGL((bmm_stream_kernel<RM, 1, 8>), dim3(grid), dim3(64), 0, stream, p);
  else
    hipLaunchKernelGGL((bmm_stream_kernel<RM, 8, 8>), dim3(grid), dim3(64), 0, stream, p);
}

// ---------------------------------------------------------------- tiled b
// b streamable as above but with columns at least a cache line apart (the
// probabilities of v p^T: each column is a row of p): a lane that streams its
// own column touches a different line per lane and instruction, which
// saturates the L1 tag lookups.  Here a block of 4 waves computes 4 * RM rows
// x 64 columns and loads b in kTileDepth-step chunks with 8 lanes per column
// (one 128-byte line per 8 lanes), keeps them in LDS as fp16 step pairs, and
// each lane reads its column two steps at a time (one 32-bit LDS read for two
// fmas; the fp16 -> fp32 conversion folds into the fma).  The next chunk is
// loaded into registers while the current one is consumed.  K % 8 == 0.
//
// Each output is a chain of K dependent fmas, and a dependent fp32 fma takes
// about 32 cycles on gfx950 (measured), so a K = 400 product cannot finish in
// under ~5.6 us however it is tiled; the tile shape only has to keep every
// chain running.
constexpr uint32_t kTileDepth = 64;

template <int RM>
__global__ __launch_bounds__(kBmmThreads) void bmm_tile_kernel(BmmPlan p) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  constexpr uint32_t TM = 4 * RM;
  constexpr uint32_t kAPitch = TM + 4;
  constexpr uint32_t kBPitch = kBmmCols + 1;  // in step pairs
  constexpr uint32_t kAPer = TM * kTileDepth / kBmmThreads;  // a elements per thread per chunk
  __shared__ __attribute__((aligned(16))) float As[kTileDepth][kAPitch];
  __shared__ h2 Bs[kTileDepth / 2][kBPitch];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  uint32_t t = blockIdx.x;
  const uint32_t nt = t % p.ntiles;
  t /= p.ntiles;
  const uint32_t mt = t % p.mtiles;
  const uint32_t bt = t / p.mtiles;
  const uint32_t i0 = mt * TM, j0 = nt * kBmmCols;

  // b: thread handles vectors e = tid + 256 s: column jj = e / 8, steps
  // 8 * (e % 8) .. + 8 of the chunk
  const __amdgpu_buffer_rsrc_t brsrc = dev::buffer_rsrc(p.b.p, p.b_bytes);
  const uint32_t rbase = p.b.row_origin + bt * p.b.row_group;
  uint32_t bvoff[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const uint32_t jj = (tid + s * kBmmThreads) / 8u;
    bvoff[s] = (uint32_t)((int64_t)bt * p.b.batch +
                          p.b.col.at(min(j0 + jj, p.n - 1) + p.b.col_origin + bt * p.b.col_group)) * 2u;
  }
  const uint32_t kv = tid % 8u;
  h8 bv[2];
  _Float16 av[kAPer];
  auto load_chunk = [&](uint32_t k0, uint32_t kc) {
    // vectors past the chunk's end re-read its last vector (never consumed)
    const uint32_t kk = k0 + min(kv * 8u, kc - 8u);
    const uint32_t soff = (uint32_t)p.b.row.at(rbase + kk) * 2u;
#pragma unroll
    for (int s = 0; s < 2; ++s)
      bv[s] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(brsrc, bvoff[s] + soff, 0, 0));
#pragma unroll
    for (uint32_t s = 0; s < kAPer; ++s) {
      const uint32_t e = tid + s * kBmmThreads;
      const uint32_t kk2 = p.a_kfast ? e % kTileDepth : e / TM;
      const uint32_t ii = p.a_kfast ? e / kTileDepth : e % TM;
      av[s] = p.a.p[p.a.at(bt, min(i0 + ii, p.m - 1), k0 + min(kk2, kc - 1))];
    }
  };
  auto store_chunk = [&]() {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint32_t jj = (tid + s * kBmmThreads) / 8u;
#pragma unroll
      for (int q = 0; q < 4; ++q) Bs[kv * 4 + q][jj] = (h2){bv[s][2 * q], bv[s][2 * q + 1]};
    }
#pragma unroll
    for (uint32_t s = 0; s < kAPer; ++s) {
      const uint32_t e = tid + s * kBmmThreads;
      const uint32_t kk2 = p.a_kfast ? e % kTileDepth : e / TM;
      const uint32_t ii = p.a_kfast ? e / kTileDepth : e % TM;
      As[kk2][ii] = (float)av[s];
    }
  };

  float acc[RM];
#pragma unroll
  for (int r = 0; r < RM; ++r) acc[r] = 0.f;
  load_chunk(0, min(kTileDepth, p.k));
  for (uint32_t k0 = 0; k0 < p.k; k0 += kTileDepth) {
    const uint32_t kc = min(kTileDepth, p.k - k0);
    store_chunk();
    __syncthreads();
    if (k0 + kTileDepth < p.k) load_chunk(k0 + kTileDepth, min(kTileDepth, p.k - k0 - kTileDepth));
#pragma unroll 4
    for (uint32_t k2 = 0; k2 < kc / 2; ++k2) {
      const h2 b = Bs[k2][lane];
      const float b0 = (float)b[0], b1 = (float)b[1];
#pragma unroll
      for (int r = 0; r < RM; ++r) acc[r] = __builtin_fmaf(As[2 * k2][wave * RM + r], b0, acc[r]);
#pragma unroll
      for (int r = 0; r < RM; ++r) acc[r] = __builtin_fmaf(As[2 * k2 + 1][wave * RM + r], b1, acc[r]);
    }
    __syncthreads();
  }
  const uint32_t j = j0 + lane;
  if (j >= p.n) return;
#pragma unroll
  for (int r = 0; r < RM; ++r) {
    const uint32_t i = i0 + wave * RM + r;
    if (i < p.m) p.y.p[p.y.at(bt, i, j)] = (_Float16)acc[r];
  }
}

// ---------------------------------------------------------------- host

// b's columns run contiguously along k in 16-byte aligned groups of 8: unit
// step along k (a plain axis of stride 1, or a blocked axis of in-block stride
// 1 whose block is a multiple of 8 and whose block stride keeps 8-alignment),
// 8-aligned column, batch and group offsets, a 16-byte aligned base.
bool streamable_b(const Mat& b) {
  const Axis& k = b.row;
  const bool unit = (k.blk.d == 1 && k.outer == 1) || (k.blk.d % 8 == 0 && k.inner == 1 && k.outer % 8 == 0);
  const bool cols = b.col.outer % 8 == 0 && (b.col.blk.d == 1 || b.col.inner % 8 == 0);
  return unit && cols && reinterpret_cast<uintptr_t>(b.p) % 16 == 0 && b.batch % 8 == 0 && b.row_origin % 8 == 0 &&
         b.row_group % 8 == 0;
}

// Rows and columns of an operand before transposition (bmm_flow.cpp:280-281).
int64_t rows_of(const thin_desc* d) { return d->sizes[1] * (d->rank == 4 ? d->sizes[3] : 1); }

struct BmmShape {
  int64_t batch, m, k, n;
};

thin_status plan_shape(const thin_desc* a, const thin_desc* b, const thin_bmm_layout* L, BmmShape& s,
                       int64_t& a_rows, int64_t& b_rows) {
  THIN_REQUIRE(a && b && L && desc_valid(a) && desc_valid(b), THIN_ERR_INVALID, "bmm: invalid descriptor");
  THIN_REQUIRE(a->dtype == THIN_F16 && b->dtype == THIN_F16 && (a->rank == 3 || a->rank == 4) &&
                   (b->rank == 3 || b->rank == 4),
               THIN_ERR_INVALID, "bmm requires inference-only same-device FP16 rank-3 or channel-blocked rank-4 tensors");
  int64_t ar = rows_of(a), ac = a->sizes[2], br = rows_of(b), bc = b->sizes[2];
  THIN_REQUIRE(L->groups >= 0 && L->a_offset >= 0 && L->b_offset >= 0, THIN_ERR_INVALID, "invalid channel grouping");
  int64_t abatch = a->sizes[0], bbatch = b->sizes[0];
  for (int o = 0; o < 2; ++o) {
    const thin_desc* x = o ? b : a;
    int64_t& rows = o ? br : ar;
    int64_t& batches = o ? bbatch : abatch;
    if (L->groups && x->rank == 4) {
      THIN_REQUIRE(x->sizes[0] == 1 && rows % L->groups == 0, THIN_ERR_INVALID,
                   "grouped blocked operand requires N=1 and divisible channels");
      rows /= L->groups;
      batches = L->groups;
    }
  }
  const int64_t a_channels = L->a_channels < 0 ? ar - L->a_offset : L->a_channels;
  const int64_t b_channels = L->b_channels < 0 ? br - L->b_offset : L->b_channels;
  THIN_REQUIRE(a_channels > 0 && b_channels > 0 && L->a_offset + a_channels <= ar && L->b_offset + b_channels <= br,
               THIN_ERR_INVALID, "channel selection exceeds its group");
  a_rows = ar;
  b_rows = br;
  s.batch = abatch;
  s.m = L->transpose_a ? ac : a_channels;
  s.k = L->transpose_a ? a_channels : ac;
  const int64_t bk = L->transpose_b ? bc : b_channels;
  s.n = L->transpose_b ? b_channels : bc;
  THIN_REQUIRE(s.batch == bbatch && s.k == bk && s.batch > 0 && s.m > 0 && s.k > 0 && s.n > 0, THIN_ERR_INVALID,
               "bmm dimensions do not match or are empty");
  const int64_t np = (s.n + 15) / 16 * 16;
  THIN_REQUIRE(s.batch <= INT32_MAX && s.m <= INT32_MAX && s.k <= INT32_MAX && np <= INT32_MAX, THIN_ERR_INVALID,
               "bmm dimensions exceed kernel index range");
  THIN_REQUIRE(!L->blocked_output || (L->groups ? s.batch * s.m : s.m) % 16 == 0, THIN_ERR_INVALID,
               "blocked output requires C0-aligned channels");
  return THIN_OK;
}

Axis make_axis(int64_t blk, int64_t outer, int64_t inner) {
  Axis x;
  x.blk = FastDiv::make((uint32_t)blk);
  x.outer = outer;
  x.inner = inner;
  return x;
}

// Logical matrix of an input operand (bmm_flow.cpp:193-215): channels are the
// rows of a blocked operand, tokens its columns; groups split the channels of
// an N=1 blocked operand into heads; origin selects a channel range.
Mat make_input(const thin_desc* x, bool transpose, int64_t groups, int64_t origin) {
  Mat d;
  memset(&d, 0, sizeof d);
  d.p = static_cast<_Float16*>(x->data);
  d.batch = x->strides[0];
  const bool blocked = x->rank == 4;
  d.row = make_axis(blocked ? x->sizes[3] : 1, x->strides[1], blocked ? x->strides[3] : 0);
  d.col = make_axis(1, x->strides[2], 0);
  d.row_origin = (uint32_t)origin;
  if (groups > 0 && blocked) {
    d.batch = 0;
    d.row_group = (uint32_t)(x->sizes[1] * x->sizes[3] / groups);
  }
  if (transpose) {
    const Axis r = d.row;
    d.row = d.col;
    d.col = r;
    d.col_origin = d.row_origin;
    d.row_origin = 0;
    d.col_group = d.row_group;
    d.row_group = 0;
  }
  return d;
}

// Smallest element step along an axis (the in-block stride of a blocked axis).
int64_t unit_step(const Axis& x) { return x.blk.d > 1 ? x.inner : x.outer; }

thin_status check_out(const thin_desc* out, const BmmShape& s, const thin_bmm_layout* L) {
  THIN_REQUIRE(out && desc_valid(out) && out->dtype == THIN_F16, THIN_ERR_INVALID, "bmm: out must be float16");
  if (!L->blocked_output) {
    THIN_REQUIRE(out->rank == 3 && out->sizes[0] == s.batch && out->sizes[1] == s.m && out->sizes[2] == s.n,
                 THIN_ERR_INVALID, "bmm: out must be [%lld, %lld, %lld]", (long long)s.batch, (long long)s.m,
                 (long long)s.n);
  } else {
    const int64_t lead = L->groups ? 1 : s.batch, c1 = (L->groups ? s.batch * s.m : s.m) / 16;
    THIN_REQUIRE(out->rank == 4 && out->sizes[0] == lead && out->sizes[1] == c1 && out->sizes[2] == s.n &&
                     out->sizes[3] == 16,
                 THIN_ERR_INVALID, "bmm: blocked out must be [%lld, %lld, %lld, 16]", (long long)lead,
                 (long long)c1, (long long)s.n);
  }
  return THIN_OK;
}

}  // namespace
}  // namespace thin

using namespace thin;

extern "C" thin_status thin_layout_bmm_shape(const thin_desc* a, const thin_desc* b, const thin_bmm_layout* layout,
                                             int32_t* out_rank, int64_t* out_sizes) {
  clear_error();
  BmmShape s;
  int64_t ar, br;
  thin_status st = plan_shape(a, b, layout, s, ar, br);
  if (st != THIN_OK) return st;
  THIN_REQUIRE(out_rank && out_sizes, THIN_ERR_INVALID, "bmm: null output shape pointer");
  if (!layout->blocked_output) {
    *out_rank = 3;
    out_sizes[0] = s.batch;
    out_sizes[1] = s.m;
    out_sizes[2] = s.n;
  } else {
    *out_rank = 4;
    out_sizes[0] = layout->groups ? 1 : s.batch;
    out_sizes[1] = (layout->groups ? s.batch * s.m : s.m) / 16;
    out_sizes[2] = s.n;
    out_sizes[3] = 16;
  }
  return THIN_OK;
}

extern "C" thin_status thin_layout_bmm(const thin_desc* a, const thin_desc* b, const thin_bmm_layout* layout,
                                       const thin_desc* out, hipStream_t stream) {
  clear_error();
  BmmShape s;
  int64_t ar, br;
  thin_status st = plan_shape(a, b, layout, s, ar, br);
  if (st != THIN_OK) return st;
  st = check_out(out, s, layout);
  if (st != THIN_OK) return st;
  // every logical index the kernel forms (origin + group offset + index)
  // stays below the operand's own row / column count
  for (const thin_desc* x : {a, b, out})
    THIN_REQUIRE(x->sizes[1] * (x->rank == 4 ? x->sizes[3] : 1) < ((int64_t)1 << 31) &&
                     x->sizes[2] < ((int64_t)1 << 31),
                 THIN_ERR_UNSUPPORTED, "bmm: operand dimensions exceed the kernel index range");

  BmmPlan p;
  memset(&p, 0, sizeof p);
  p.a = make_input(a, layout->transpose_a, layout->groups, layout->a_offset);
  p.b = make_input(b, layout->transpose_b, layout->groups, layout->b_offset);
  Mat& y = p.y;
  y.p = static_cast<_Float16*>(out->data);
  if (!layout->blocked_output) {
    y.batch = out->strides[0];
    y.row = make_axis(1, out->strides[1], 0);
    y.col = make_axis(1, out->strides[2], 0);
  } else {
    // channel r of batch b is packed channel b * m + r of [lead, C1, n, 16]
    // (grouped), or channel r of image b (ungrouped; the two agree when the
    // ungrouped tensor is contiguous)
    y.row = make_axis(16, out->strides[1], out->strides[3]);
    y.col = make_axis(1, out->strides[2], 0);
    if (layout->groups) {
      y.batch = 0;
      y.row_group = (uint32_t)s.m;
    } else {
      y.batch = out->strides[0];
    }
  }
  p.m = (uint32_t)s.m;
  p.n = (uint32_t)s.n;
  p.k = (uint32_t)s.k;
  // k is the column axis of a and the row axis of b
  p.a_kfast = unit_step(p.a.col) <= unit_step(p.a.row);
  p.b_kfast = unit_step(p.b.row) <= unit_step(p.b.col);
  p.ntiles = (uint32_t)((s.n + kBmmCols - 1) / kBmmCols);
  int64_t b_extent = 1;  // elements from b's data pointer to its last element, + 1
  for (int d = 0; d < b->rank; ++d) b_extent += (b->sizes[d] - 1) * b->strides[d];
  if (streamable_b(p.b) && b_extent * 2 < ((int64_t)1 << 31)) {
    p.b_bytes = (uint32_t)(b_extent * 2);
    p.b_vrun = p.b.row.blk.d == 1 ? 0u : p.b.row.blk.d / 8u;
    p.b_vjump = p.b.row.blk.d == 1 ? 0u : (uint32_t)((p.b.row.outer - p.b.row.blk.d) * 2);
    if (p.k % 8 == 0 && p.b.col.blk.d == 1 && p.b.col.outer >= 64) {
      // columns a line or more apart: 64-column tiles staged through LDS
      auto blocks = [&](int rm) { return (uint64_t)s.batch * ((s.m + 4 * rm - 1) / (4 * rm)) * p.ntiles; };
      const int rm = blocks(4) * 4 >= 1024 ? 4 : blocks(2) * 4 >= 1024 ? 2 : 1;
      p.mtiles = (uint32_t)((s.m + 4 * rm - 1) / (4 * rm));
      const uint64_t grid = blocks(rm);
      THIN_REQUIRE(grid < ((uint64_t)1 << 31), THIN_ERR_UNSUPPORTED, "bmm: too many output tiles");
      if (rm == 4)
        hipLaunchKernelGGL(bmm_tile_kernel<4>, dim3((uint32_t)grid), dim3(kBmmThreads), 0, stream, p);
      else if (rm == 2)
        hipLaunchKernelGGL(bmm_tile_kernel<2>, dim3((uint32_t)grid), dim3(kBmmThreads), 0, stream, p);
      else
        hipLaunchKernelGGL(bmm_tile_kernel<1>, dim3((uint32_t)grid), dim3(kBmmThreads), 0, stream, p);
      THIN_LAUNCH_CHECK("bmm_tile_kernel");
      return THIN_OK;
    }
    // rows per wave: 2, which measured fastest for both attention products
    // (q^T k [4,400,32]x[4,32,400]: 6.3 us rotated against 6.9 with 4 rows and
    // 7.7 with 1); 1 when that leaves under half a wave per SIMD, 4 when it
    // would queue more than 8 waves per SIMD
    auto waves = [&](int rm) { return (uint64_t)s.batch * ((s.m + rm - 1) / rm) * p.ntiles; };
    const int rm = waves(2) < 512 ? 1 : waves(2) > 8192 ? 4 : 2;
    p.mtiles = (uint32_t)((s.m + rm - 1) / rm);
    p.div_mt = FastDiv::make(p.mtiles);
    p.div_nt = FastDiv::make(p.ntiles);
    const uint64_t grid = waves(rm);
    THIN_REQUIRE(grid < ((uint64_t)1 << 31), THIN_ERR_UNSUPPORTED, "bmm: too many output tiles");
    if (rm == 4)
      launch_stream<4>(p, (uint32_t)grid, stream);
    else if (rm == 2)
      launch_stream<2>(p, (uint32_t)grid, stream);
    else
      launch_stream<1>(p, (uint32_t)grid, stream);
    THIN_LAUNCH_CHECK("bmm_stream_kernel");
    return THIN_OK;
  }
  // rows per wave: the widest tile that still gives every SIMD about one wave
  auto blocks = [&](int rm) { return (uint64_t)s.batch * ((s.m + 4 * rm - 1) / (4 * rm)) * p.ntiles; };
  const int rm = blocks(4) * 4 >= 1024 ? 4 : blocks(2) * 4 >= 1024 ? 2 : 1;
  p.mtiles = (uint32_t)((s.m + 4 * rm - 1) / (4 * rm));
  const uint64_t grid = blocks(rm);
  THIN_REQUIRE(grid < ((uint64_t)1 << 31), THIN_ERR_UNSUPPORTED, "bmm: too many output tiles");
  if (rm == 4)
    hipLaunchKernelGGL(bmm_kernel<4>, dim3((uint32_t)grid), dim3(kBmmThreads), 0, stream, p);
  else if (rm == 2)
    hipLaunchKernelGGL(bmm_kernel<2>, dim3((uint32_t)grid), dim3(kBmmThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(bmm_kernel<1>, dim3((uint32_t)grid), dim3(kBmmThreads), 0, stream, p);
  THIN_LAUNCH_CHECK("bmm_kernel");
  return THIN_OK;
}

// ---------------------------------------------------------------- channel select

namespace thin {
namespace {

// out channel c of [1, C1o, T, 16] = x channel (c / count) * group + begin +
// c % count of [1, C1, T, 16] (bmm_flow.cpp:217-251); one thread per output
// element.
struct SelectPlan {
  const _Float16* x;
  _Float16* y;
  int64_t xs1, xs2, xs3, ys1, ys2, ys3;
  FastDiv tokens, count;
  uint32_t group, begin;
  uint64_t total;  // C1o * T * 16
};

__global__ __launch_bounds__(256) void channel_select_kernel(SelectPlan p) {
  // the plan in registers before the loop's bounds test: one round of scalar
  // loads (one asm statement: each is a scheduling boundary)
  __asm__ volatile("" ::"s"(p.x), "s"(p.y), "s"(p.xs1), "s"(p.xs2), "s"(p.xs3), "s"(p.ys1), "s"(p.ys2), "s"(p.ys3),
                   "s"(p.tokens.d), "s"(p.tokens.mul), "s"(p.tokens.shr), "s"(p.count.d), "s"(p.count.mul),
                   "s"(p.count.shr), "s"(p.group), "s"(p.begin), "s"(p.total));
  for (uint64_t e = (uint64_t)blockIdx.x * 256 + threadIdx.x; e < p.total; e += (uint64_t)gridDim.x * 256) {
    const uint32_t lane = (uint32_t)(e & 15u);
    const uint32_t rest = (uint32_t)(e >> 4);  // cb * T + t
    const uint32_t cb = p.tokens.div(rest), t = rest - cb * p.tokens.d;
    const uint32_t c = cb * 16u + lane;
    const uint32_t g = p.count.div(c);
    const uint32_t sc = g * p.group + p.begin + (c - g * p.count.d);
    const _Float16 v = p.x[(int64_t)(sc >> 4) * p.xs1 + (int64_t)t * p.xs2 + (int64_t)(sc & 15u) * p.xs3];
    p.y[(int64_t)cb * p.ys1 + (int64_t)t * p.ys2 + (int64_t)lane * p.ys3] = v;
  }
}

thin_status select_shape(const thin_desc* x, int64_t groups, int64_t begin, int64_t count, int64_t* sizes) {
  THIN_REQUIRE(x && desc_valid(x) && x->dtype == THIN_F16 && x->rank == 4 && x->sizes[0] == 1 && x->sizes[3] == 16,
               THIN_ERR_INVALID, "channel_select expects aligned N=1 FP16 blocked input");
  const int64_t channels = x->sizes[1] * 16;
  THIN_REQUIRE(groups > 0 && channels % groups == 0 && begin >= 0 && count > 0 && begin + count <= channels / groups &&
                   groups * count % 16 == 0,
               THIN_ERR_INVALID, "channel_select requires valid equal groups and C0-aligned total output channels");
  sizes[0] = 1;
  sizes[1] = groups * count / 16;
  sizes[2] = x->sizes[2];
  sizes[3] = 16;
  return THIN_OK;
}

}  // namespace
}  // namespace thin

extern "C" thin_status thin_channel_select_shape(const thin_desc* x, int64_t groups, int64_t begin, int64_t count,
                                                 int64_t* out_sizes) {
  clear_error();
  THIN_REQUIRE(out_sizes, THIN_ERR_INVALID, "channel_select: null output shape pointer");
  return select_shape(x, groups, begin, count, out_sizes);
}

extern "C" thin_status thin_channel_select(const thin_desc* x, int64_t groups, int64_t begin, int64_t count,
                                           const thin_desc* out, hipStream_t stream) {
  clear_error();
  int64_t sizes[4];
  thin_status st = select_shape(x, groups, begin, count, sizes);
  if (st != THIN_OK) return st;
  THIN_REQUIRE(out && desc_valid(out) && out->dtype == THIN_F16 && out->rank == 4 && out->sizes[0] == 1 &&
                   out->sizes[1] == sizes[1] && out->sizes[2] == sizes[2] && out->sizes[3] == 16,
               THIN_ERR_INVALID, "channel_select: out must be [1, %lld, %lld, 16] float16", (long long)sizes[1],
               (long long)sizes[2]);
  THIN_REQUIRE(x->sizes[1] * 16 < ((int64_t)1 << 31) && x->sizes[2] < ((int64_t)1 << 31) &&
                   sizes[1] * sizes[2] < ((int64_t)1 << 27),
               THIN_ERR_UNSUPPORTED, "channel_select: tensor too large");
  SelectPlan p;
  memset(&p, 0, sizeof p);
  p.x = static_cast<const _Float16*>(x->data);
  p.y = static_cast<_Float16*>(out->data);
  p.xs1 = x->strides[1];
  p.xs2 = x->strides[2];
  p.xs3 = x->strides[3];
  p.ys1 = out->strides[1];
  p.ys2 = out->strides[2];
  p.ys3 = out->strides[3];
  p.tokens = FastDiv::make((uint32_t)sizes[2]);
  p.count = FastDiv::make((uint32_t)count);
  p.group = (uint32_t)(x->sizes[1] * 16 / groups);
  p.begin = (uint32_t)begin;
  p.total = (uint64_t)sizes[1] * (uint64_t)sizes[2] * 16u;
  if (p.total == 0) return THIN_OK;
  hipLaunchKernelGGL(channel_select_kernel, dim3(grid_for(p.total, 256)), dim3(256), 0, stream, p);
  THIN_LAUNCH_CHECK("channel_select_kernel");
  return THIN_OK;
}
