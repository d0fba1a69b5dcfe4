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

#include <type_traits>

#include <string.h>

#include <algorithm>
#include <mutex>

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
// Wide form: a block covers 64 consecutive anchors (one per lane, so a wave
// reads 128 contiguous bytes per class in the production [B,4+nc,A] layout)
// and CG class groups (one per wave; group g scans classes g, g+CG, ...).  Each
// group keeps its first minimal key; merging the groups by (key, class) keeps
// the first class with the minimal key overall.
template <int CG>
__global__ __launch_bounds__(64 * CG) void class_max_wide_kernel(Layout L, int64_t batches, int64_t anchors,
                                                                  int64_t classes, uint16_t* bits1, int32_t* cls1,
                                                                  uint16_t* trace_max) {
  __shared__ uint32_t g_key[CG][64], g_bits[CG][64], g_cls[CG][64];
  const uint32_t lane = threadIdx.x & 63u, grp = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * 64 + lane;
  const bool live = t < batches * anchors;
  uint32_t bk = 0x10000u, bb = 0u, bc = 0xffffffffu;
  if (live) {
    const int64_t b = t / anchors, a = t - b * anchors;
    const uint16_t* row = L.x + b * L.sb + a * L.sa + 4 * L.sc;
#pragma unroll 4
    for (int64_t c = grp; c < classes; c += CG) {
      const uint32_t bits = row[c * L.sc];
      const uint32_t k = score_key(bits);
      if (k < bk) {
        bk = k;
        bb = bits;
        bc = (uint32_t)c;
      }
    }
  }
  g_key[grp][lane] = bk;
  g_bits[grp][lane] = bb;
  g_cls[grp][lane] = bc;
  __syncthreads();
  if (grp == 0 && live) {
#pragma unroll
    for (int g = 1; g < CG; ++g) {
      const uint32_t k = g_key[g][lane], c = g_cls[g][lane];
      if (k < bk || (k == bk && c < bc)) {
        bk = k;
        bb = g_bits[g][lane];
        bc = c;
      }
    }
    bits1[t] = (uint16_t)bb;
    cls1[t] = (int32_t)bc;
    if (trace_max) trace_max[t] = (uint16_t)bb;
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

// ---------------------------------------------------------------- register top-K
// One 1024-thread block per batch for up to 32768 candidates.  The candidate
// bits are staged in LDS with coalesced 16-byte loads (they also serve the
// packing step), then thread t takes candidates [t*KPT, t*KPT + KPT) into
// registers, so thread order is index order.  Radix select: per-wave LDS
// histograms of the high and then the low key byte, summed and scanned by 256
// threads, give the threshold key T and how many T-keyed candidates to keep; a
// block-wide exclusive scan of per-thread T counts ranks the T-keyed
// candidates in index order (lowest index kept).  The K selected records
// (key << 16 | index, unique) are ordered by rank counting (K <= 512, each
// record's rank summed over several threads) or an LDS bitonic sort.
// Modes: 0 writes the selected indices and the threshold key T; 1
// (class-agnostic anchors) and 2 (per-class pairs, whose scores a wide gather
// kernel collected) also pack the output rows and the trace stages.
//
// Mode 2 survivors: the K anchors of the first stage carry K pairs (their
// class maxima) keyed at most T1, the first stage's threshold, so the K-th
// best pair is keyed at most T1 and pairs keyed above it are never selected;
// they are dropped before the histograms.  Mode 2 with K <= 512 also fetches
// the first-stage anchors and their boxes into LDS while the selection runs.
constexpr uint32_t kRegThreads = 1024;
constexpr uint32_t kRegWaves = kRegThreads / 64;
constexpr uint32_t kRegMaxN = 32768;
constexpr uint32_t kRegMaxK = 8192;
constexpr uint32_t kRankSortMax = 512;

struct RegTopkPlan {
  const uint16_t* bits;   // candidate bits [B, n]
  Layout L;               // boxes for packing
  const int32_t* stage1;  // mode 2: first-stage anchors [B, K]
  uint32_t n, K;          // candidates and selections per batch
  FastDiv nc;             // classes (mode 2 pair index = rank * nc + class)
  int64_t anchors;        // row pitch of bits1 / cls1 (mode 1)
  int32_t* sel;           // mode 0: [B, K] selected candidate indices
  uint32_t* thresh;       // mode 0 writes, mode 2 reads (if set): threshold key per batch
  const int32_t* cls1;    // mode 1: class-max labels [B, A]
  uint32_t* out;          // modes 1, 2: [B, K, 6] fp32 bits
  thin_select_trace tr;
};

// LDS slot of candidate i.  Thread t reads its KPT keys as KPT/8 16-byte
// vectors at a stride of KPT*2 bytes; the vectors of one thread are permuted
// by a function of t so that the lanes of one read instruction fall on
// distinct bank groups for 128- and 256-byte LDS rows alike.
template <int KPT>
__device__ __forceinline__ uint32_t staged_vec(uint32_t g) {
  constexpr uint32_t VPT = KPT / 8;
  if constexpr (VPT == 1) {
    return g;
  } else {
    const uint32_t t = g / VPT, v = g % VPT;
    const uint32_t f = VPT == 4 ? ((t >> 1) ^ (t >> 3)) & 3u : ((t >> 2) ^ (t >> 3)) & 1u;
    return t * VPT + (v ^ f);
  }
}
template <int KPT>
__device__ __forceinline__ uint32_t staged_slot(uint32_t i) {
  return (staged_vec<KPT>(i >> 3) << 3) | (i & 7u);
}

// Exclusive block-wide prefix sum of v; `total` receives the block sum.
__device__ __forceinline__ uint32_t block_exclusive_sum(uint32_t v, uint32_t* wave_tot, uint32_t& total) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o);
    if (lane >= (uint32_t)o) x += y;
  }
  if (lane == 63u) wave_tot[wave] = x;
  __syncthreads();
  uint32_t before = 0;
  total = 0;
#pragma unroll
  for (uint32_t w = 0; w < kRegWaves; ++w) {
    const uint32_t t = wave_tot[w];
    before += w < wave ? t : 0u;
    total += t;
  }
  __syncthreads();
  return before + x - v;
}

// Sums the per-wave histograms and finds the bin q with
// base + count(< q) < need <= base + count(<= q); writes q and base + count(< q).
__device__ __forceinline__ void pick_bin(uint32_t (*hist)[256], uint32_t base, uint32_t need, uint32_t* wave_tot,
                                         uint32_t* result) {
  const uint32_t tid = threadIdx.x;
  uint32_t h = 0;
  if (tid < 256) {
#pragma unroll
    for (uint32_t w = 0; w < kRegWaves; ++w) h += hist[w][tid];
  }
  uint32_t total;
  const uint32_t excl = block_exclusive_sum(tid < 256 ? h : 0u, wave_tot, total);
  if (tid < 256 && base + excl < need && need <= base + excl + h) {
    result[0] = tid;
    result[1] = base + excl;
  }
  __syncthreads();
}

// First-stage anchors and their box bits, fetched into LDS by mode 2.
struct PairBoxes {
  int32_t anchor[kRankSortMax];
  uint16_t box[kRankSortMax][4];
};

// Output row r of batch b for selected candidate idx; `staged` holds the
// batch's candidate bits (the selected score's bits are at staged_slot(idx)).
template <int MODE, int KPT>
__device__ __forceinline__ void pack_row(const RegTopkPlan& p, const uint16_t* staged, const PairBoxes* pb,
                                         uint32_t b, uint32_t r, uint32_t idx) {
  int64_t a, label;
  const uint32_t sbits = staged[staged_slot<KPT>(idx)];
  uint32_t box[4];
  if (MODE == 1) {
    a = idx;
    label = p.cls1[(int64_t)b * p.anchors + a];
  } else {
    const uint32_t rank1 = p.nc.div(idx);
    label = idx - rank1 * p.nc.d;
    a = pb ? pb->anchor[rank1] : p.stage1[(size_t)b * p.K + rank1];
    if (pb) {
#pragma unroll
      for (int c = 0; c < 4; ++c) box[c] = pb->box[rank1][c];
    }
  }
  if (MODE == 1 || !pb) {
    const uint16_t* bx = p.L.x + b * p.L.sb + a * p.L.sa;
#pragma unroll
    for (int c = 0; c < 4; ++c) box[c] = bx[c * p.L.sc];
  }
  const size_t t = (size_t)b * p.K + r;
  uint32_t* o = p.out + t * 6;
#pragma unroll
  for (int c = 0; c < 4; ++c) o[c] = float_bits(box[c]);
  o[4] = float_bits(sbits);
  o[5] = __float_as_uint((float)label);
  if (p.tr.stage1) static_cast<int64_t*>(p.tr.stage1)[t] = MODE == 1 ? a : (int64_t)p.stage1[t];
  if (MODE == 2 && p.tr.stage2) static_cast<int64_t*>(p.tr.stage2)[t] = idx;
  if (p.tr.anchors) static_cast<int64_t*>(p.tr.anchors)[t] = a;
  if (p.tr.labels) static_cast<int64_t*>(p.tr.labels)[t] = label;
  if (p.tr.top_values) static_cast<uint16_t*>(p.tr.top_values)[t] = (uint16_t)sbits;
}

// Histogram update for a thread's keys: the high byte (hi == 0xffffffff) or
// the low byte of keys whose high byte is hi.  Equal bins of consecutive
// candidates are merged first, so skewed score distributions (most class
// maxima in one bin) cost one LDS atomic per run instead of one per key.
template <int KPT>
__device__ __forceinline__ void count_bins(uint32_t* hist, const uint32_t (&key)[KPT], uint32_t hi) {
  uint32_t cur = 0xffffffffu, run = 0;
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const bool in = hi == 0xffffffffu ? key[j] <= 0xffffu : (key[j] >> 8) == hi;
    if (!in) continue;
    const uint32_t bin = hi == 0xffffffffu ? key[j] >> 8 : key[j] & 0xffu;
    if (bin != cur) {
      if (run) atomicAdd(&hist[cur], run);
      cur = bin;
      run = 0;
    }
    ++run;
  }
  if (run) atomicAdd(&hist[cur], run);
}

// ranks[r] (zero on entry) += the number of records below rec[r], for
// r < count; rec[count, n16) are 0xffffffff pads and n16 <= 512 is a multiple
// of 16.  Records are unique, so the ranks are a permutation.  A record's rank
// is summed over kRegThreads / n16 threads, each comparing a slice of the
// records, 16 per step.  Ends with a block barrier.
__device__ __forceinline__ void rank_records(const uint32_t* rec, uint32_t n16, uint32_t count, uint32_t* ranks) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  const uint32_t tid = threadIdx.x;
  const uint32_t parts = kRegThreads / n16;  // >= 2 since n16 <= 512
  const uint32_t slice = ((n16 / 4 + parts - 1) / parts + 3) & ~3u;  // u4 records per thread
  const uint32_t r = tid % n16, part = tid / n16;
  if (part < parts) {
    const uint32_t mine = rec[r];
    const u4* r4 = reinterpret_cast<const u4*>(rec);
    const uint32_t lo = part * slice, hi = min(lo + slice, n16 / 4);
    uint32_t rank = 0;
    for (uint32_t u = lo; u < hi; u += 4) {
      u4 q[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) q[h] = r4[u + h];
#pragma unroll
      for (int h = 0; h < 4; ++h)
        rank += (q[h].x < mine) + (q[h].y < mine) + (q[h].z < mine) + (q[h].w < mine);
    }
    if (r < count && rank) atomicAdd(&ranks[r], rank);
  }
  __syncthreads();
}

// Radix-selects the K best candidates: thread t holds N keys (0xffffffff =
// absent) of candidates idx[j], and the block-wide order (t, j) is index
// order.  hist[0] and hist[1] must be zero.  Writes the K records
// (key << 16 | index) to recs[0, K) and returns the threshold key T.
template <int N>
__device__ __forceinline__ uint32_t radix_select(uint32_t (&key)[N], const uint32_t (&idx)[N], uint32_t K,
                                                 uint32_t (*hist)[kRegWaves][256], uint32_t* wave_tot,
                                                 uint32_t* result, uint32_t* recs) {
  const uint32_t wave = threadIdx.x >> 6;
  // level 1: high byte
  count_bins<N>(hist[0][wave], key, 0xffffffffu);
  __syncthreads();
  pick_bin(hist[0], 0, K, wave_tot, result);
  const uint32_t b1 = result[0], below1 = result[1];
  // level 2: low byte inside bucket b1
  count_bins<N>(hist[1][wave], key, b1);
  __syncthreads();
  pick_bin(hist[1], below1, K, wave_tot, result);
  const uint32_t T = (b1 << 8) | result[0];
  const uint32_t need = K - result[1];  // T-keyed candidates kept, lowest index first

  // rank the T-keyed candidates in index order, then place the selected ones
  uint32_t eq = 0;
#pragma unroll
  for (int j = 0; j < N; ++j) eq += key[j] == T ? 1u : 0u;
  uint32_t total;
  uint32_t eq_before = block_exclusive_sum(eq, wave_tot, total);
  uint32_t mine = 0;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const bool take = key[j] < T || (key[j] == T && eq_before < need);
    eq_before += key[j] == T ? 1u : 0u;
    key[j] = take ? key[j] : 0xffffffffu;  // reuse: 0xffffffff = not selected
    mine += take ? 1u : 0u;
  }
  uint32_t pos = block_exclusive_sum(mine, wave_tot, total);
#pragma unroll
  for (int j = 0; j < N; ++j)
    if (key[j] != 0xffffffffu) recs[pos++] = (key[j] << 16) | idx[j];
  return T;
}

template <int MODE, int KPT>
__global__ __launch_bounds__(kRegThreads) void topk_reg_kernel(RegTopkPlan p) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(16))) uint16_t staged[kRegMaxN];
  __shared__ uint32_t hist[2][kRegWaves][256];
  __shared__ __attribute__((aligned(16))) uint32_t recs[kRegMaxK];
  __shared__ uint32_t ranks[kRankSortMax];
  __shared__ __attribute__((aligned(16))) uint32_t surv[MODE == 2 ? kRegThreads : 16];
  __shared__ PairBoxes pbox;
  __shared__ uint32_t wave_tot[kRegWaves];
  __shared__ uint32_t result[2];
  const uint32_t b = blockIdx.x, tid = threadIdx.x;
  const uint32_t n = p.n, K = p.K;
  const uint32_t first = tid * KPT;
  const bool prefetch = MODE == 2 && K <= kRankSortMax;

  // mode 2: the first-stage anchors, then (below) their boxes, into LDS
  if (prefetch && tid < K) pbox.anchor[tid] = p.stage1[(size_t)b * K + tid];
  // stage the batch's candidate bits in LDS (coalesced), clear both
  // histograms and the partial ranks
  const uint16_t* src = p.bits + (size_t)b * n;
  uint32_t head = 0;
  if ((reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
    head = n & ~7u;
    for (uint32_t v = tid; v < head / 8; v += kRegThreads)
      reinterpret_cast<u4*>(staged)[staged_vec<KPT>(v)] = reinterpret_cast<const u4*>(src)[v];
  }
  for (uint32_t i = head + tid; i < n; i += kRegThreads) staged[staged_slot<KPT>(i)] = src[i];
  for (uint32_t q = tid; q < 2 * kRegWaves * 256; q += kRegThreads) (&hist[0][0][0])[q] = 0;
  for (uint32_t q = tid; q < kRankSortMax; q += kRegThreads) ranks[q] = 0;
  const uint32_t t1 = MODE == 2 && p.thresh ? p.thresh[b] : 0xffffu;
  __syncthreads();
  // box bits of the first-stage anchors: the loads stay in flight during the
  // selection and land in LDS just before the packing
  uint32_t box_bits[4] = {0u, 0u, 0u, 0u};
  if (prefetch && tid < K) {
    const uint16_t* bx = p.L.x + b * p.L.sb + (int64_t)pbox.anchor[tid] * p.L.sa;
#pragma unroll
    for (int c = 0; c < 4; ++c) box_bits[c] = bx[c * p.L.sc];
  }
  uint32_t key[KPT], idx[KPT];
#pragma unroll
  for (int v = 0; v < KPT / 8; ++v) {
    const u4 w = reinterpret_cast<const u4*>(staged)[staged_vec<KPT>(tid * (KPT / 8) + v)];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      key[v * 8 + 2 * h] = w[h] & 0xffffu;
      key[v * 8 + 2 * h + 1] = w[h] >> 16;
    }
  }
  uint32_t survivors = 0;
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const uint32_t k = first + j < n ? score_key(key[j]) : 0xffffffffu;
    key[j] = k <= t1 ? k : 0xffffffffu;  // mode 2: pairs keyed above T1 are never selected
    idx[j] = first + j;
    survivors += key[j] != 0xffffffffu ? 1u : 0u;
  }

  uint32_t T = 0;
  bool compact = false;
  if constexpr (MODE == 2) {
    // few survivors: move their records (in index order) to LDS
    uint32_t count;
    uint32_t at = block_exclusive_sum(survivors, wave_tot, count);
    compact = count <= kRegThreads;
    if (compact) {
#pragma unroll
      for (int j = 0; j < KPT; ++j)
        if (key[j] != 0xffffffffu) surv[at++] = (key[j] << 16) | (first + j);
      const uint32_t C16 = (count + 15u) & ~15u;
      if (count <= kRankSortMax && tid >= count && tid < C16) surv[tid] = 0xffffffffu;
      __syncthreads();
      if (count <= kRankSortMax) {
        // at most 512: a survivor's rank among all survivors (records are
        // unique) is its output row; ranks below K are the selection, sorted
        rank_records(surv, C16, count, ranks);
        if (tid < count && ranks[tid] < K) recs[ranks[tid]] = surv[tid];
        if (prefetch && tid < K) {
#pragma unroll
          for (int c = 0; c < 4; ++c) pbox.box[tid][c] = (uint16_t)box_bits[c];
        }
        __syncthreads();
        if (tid < K) pack_row<MODE, KPT>(p, staged, &pbox, b, tid, recs[tid] & 0xffffu);
        return;
      }
      uint32_t k1[1] = {tid < count ? surv[tid] >> 16 : 0xffffffffu};
      const uint32_t i1[1] = {tid < count ? surv[tid] & 0xffffu : 0u};
      T = radix_select<1>(k1, i1, K, hist, wave_tot, result, recs);
    }
  }
  if (!compact) T = radix_select<KPT>(key, idx, K, hist, wave_tot, result, recs);
  if (MODE == 0 && p.thresh && tid == 0) p.thresh[b] = T;
  const uint32_t K16 = (K + 15u) & ~15u;
  if (K <= kRankSortMax && tid >= K && tid < K16) recs[tid] = 0xffffffffu;
  if (prefetch && tid < K) {
#pragma unroll
    for (int c = 0; c < 4; ++c) pbox.box[tid][c] = (uint16_t)box_bits[c];
  }
  __syncthreads();

  const PairBoxes* pb = prefetch ? &pbox : nullptr;
  if (K <= kRankSortMax) {
    rank_records(recs, K16, K, ranks);
    if (tid < K) {
      const uint32_t idx = recs[tid] & 0xffffu;
      if (MODE == 0) p.sel[(size_t)b * K + ranks[tid]] = (int32_t)idx;
      else pack_row<MODE, KPT>(p, staged, pb, b, ranks[tid], idx);
    }
    return;
  }
  uint32_t P = 1;
  while (P < K) P <<= 1;
  for (uint32_t i = K + tid; i < P; i += kRegThreads) recs[i] = 0xffffffffu;
  __syncthreads();
  for (uint32_t size = 2; size <= P; size <<= 1) {
    for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
      for (uint32_t i = tid; i < P; i += kRegThreads) {
        const uint32_t l = i ^ stride;
        if (l > i) {
          const uint32_t x = recs[i], y = recs[l];
          const bool up = (i & size) == 0;
          if ((x > y) == up) {
            recs[i] = y;
            recs[l] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  for (uint32_t r = tid; r < K; r += kRegThreads) {
    const uint32_t idx = recs[r] & 0xffffu;
    if (MODE == 0) p.sel[(size_t)b * K + r] = (int32_t)idx;
    else pack_row<MODE, KPT>(p, staged, pb, b, r, idx);
  }
}

template <int MODE>
void launch_reg_topk(const RegTopkPlan& p, int64_t B, hipStream_t stream) {
  if (p.n <= 8u * kRegThreads)
    hipLaunchKernelGGL((topk_reg_kernel<MODE, 8>), dim3((uint32_t)B), dim3(kRegThreads), 0, stream, p);
  else if (p.n <= 16u * kRegThreads)
    hipLaunchKernelGGL((topk_reg_kernel<MODE, 16>), dim3((uint32_t)B), dim3(kRegThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((topk_reg_kernel<MODE, 32>), dim3((uint32_t)B), dim3(kRegThreads), 0, stream, p);
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

// ---------------------------------------------------------------- split selection
// The selection spread over many workgroups, for one image or a few.  Records
// are 32-bit (key << 16 | index): the stage-1 index is the anchor, the stage-2
// index the flat pair index rank * nc + class; both fit 16 bits here, keys
// never reach 0xffff (the largest is -inf's 0xfc00), so 0xffffffff pads.
//
//   slice  (grid lists x B): class max of kSlice anchors, then the slice's
//          records sorted -> lists1[b][p], bits1 / cls1.
//   merge1 (grid kMergeBlocks x B): the stage-1 top K of the sorted slices;
//          writes stage1[b][rank] and the threshold key T1 (class-agnostic:
//          packs the output rows instead).
//   pairs  (grid pair blocks x B): block p takes stage-1 ranks [p*RB, ...),
//          gathers their nc scores, keeps pairs keyed at most T1 (the K
//          class-max pairs of the stage-1 anchors are among them, so the
//          K-th best pair is keyed at most T1) and writes them sorted, at most
//          K, to lists2[b][p].
//   merge2 (grid kMergeBlocks x B): the top K of the pair lists; packs rows.
//
// Merging sorted lists.  With q such that the first min(q, n_p) records of
// the lists number at least K, every record above R = max_p
// list_p[min(q, n_p) - 1] has at least K records below it, so only records up
// to R are candidates.  A candidate at position i of list p has rank i plus,
// for every other list, the number of its candidates below it.  Each merge
// block ranks a share of the candidates; the ranks are a permutation, so the
// shares write disjoint rows.
//
// These kernels avoid long chains of dependent LDS accesses (about 130 cycles
// each on gfx950): sorts are rank counts (every record compared with every
// other, independent vector loads), and list counts are vector scans of the
// short candidate prefixes.
constexpr uint32_t kSlice = 256;         // anchors per stage-1 list
constexpr uint32_t kMaxLists = 64;       // lists per batch and stage
constexpr uint32_t kMergeBlocks = 32;    // merge workgroups per batch
constexpr uint32_t kSplitMaxK = 1024;
constexpr uint32_t kPairCap = 4096;      // gathered pairs per pairs block
constexpr uint32_t kMerge2Words = 16384; // pair lists per batch: pair_blocks * K records
constexpr uint32_t kPad = 0xffffffffu;
// Every split kernel runs 1024-thread workgroups.  Device code uses these
// constants rather than blockDim / gridDim, which are read from the dispatch's
// implicit arguments in memory (a dependent load on the critical path).
constexpr uint32_t kSplitThreads = 1024;
constexpr uint32_t kSliceThreads = 1024;  // slice_kernel workgroups
// LDS pitch of a stage-1 list: 260 words puts list l's vectors on banks 4l
// mod 64 (a 256-word pitch would put every list on the same banks, and the
// lanes that scan different lists would serialise).
constexpr uint32_t kSliceLds = kSlice + 4;

typedef uint32_t u4v __attribute__((ext_vector_type(4)));

struct SplitPlan {
  Layout L;
  uint32_t A, nc, K;
  uint32_t lists1;        // stage-1 lists per batch: ceil(A / kSlice)
  uint32_t q1;            // stage-1 prefix length (host: depends on A and K only)
  uint32_t pair_blocks;   // stage-2 lists per batch
  uint32_t ranks_per;     // stage-1 ranks per pairs block
  uint32_t pitch2;        // words per pair list: K rounded up to a multiple of 4
  uint32_t lds_pitch2;    // the same list's LDS pitch, 4 mod 64 words (see kSliceLds)
  int32_t agnostic;
  int32_t vec_classes;    // anchors contiguous in aligned 16-byte groups (slice_kernel)
  uint16_t* bits1;        // [B, A]
  int32_t* cls1;          // [B, A]
  uint32_t* lists1_rec;   // [B, lists1, kSlice]
  int32_t* stage1;        // [B, K]
  uint32_t* thresh;       // [B]: T1
  uint32_t* lists2_rec;   // [B, pair_blocks, pitch2]
  uint32_t* count2;       // [B, pair_blocks]
  uint32_t* out;          // [B, K, 6] fp32 bits
  thin_select_trace tr;
};

// Number of records in buf[0, n) below x, buf 16-byte aligned with kPad up to
// the next multiple of 4 (vector loads, no dependent chain).
__device__ __forceinline__ uint32_t count_below(const uint32_t* buf, uint32_t n, uint32_t x) {
  const u4v* v = reinterpret_cast<const u4v*>(buf);
  const uint32_t n4 = (n + 3) / 4;
  uint32_t c = 0;
  for (uint32_t u = 0; u < n4; u += 4) {  // four independent loads per step
    u4v q[4];
#pragma unroll
    for (uint32_t h = 0; h < 4; ++h) q[h] = u + h < n4 ? v[u + h] : (u4v)kPad;
#pragma unroll
    for (uint32_t h = 0; h < 4; ++h) c += (q[h].x < x) + (q[h].y < x) + (q[h].z < x) + (q[h].w < x);
  }
  return c;
}

// Sorts the n unique records of buf (kPad up to a multiple of 4) by rank
// counting: out[rank] = record for ranks below `keep`.  Each record is
// compared by max(1, BD / n) threads (BD: the block size), each over a slice
// of buf; their
// counts meet in ranks[] (n words, LDS).  Every thread of the block calls it;
// ends with a block barrier.
template <uint32_t BD>
__device__ __forceinline__ void rank_sort(const uint32_t* buf, uint32_t n, uint32_t keep, uint32_t* ranks,
                                          uint32_t* out) {
  const uint32_t tid = threadIdx.x, bd = BD;
  for (uint32_t i = tid; i < n; i += bd) ranks[i] = 0;
  __syncthreads();
  const uint32_t n4 = (n + 3) / 4;
  const uint32_t parts = n ? max(1u, bd / n) : 1u;
  const uint32_t per = (n4 + parts - 1) / parts;
  const u4v* v = reinterpret_cast<const u4v*>(buf);
  for (uint32_t w = tid; w < n * parts; w += bd) {
    const uint32_t part = w / n, r = w - part * n;
    const uint32_t mine = buf[r];
    uint32_t c = 0;
    const uint32_t hi = min(n4, part * per + per);
    for (uint32_t u = part * per; u < hi; u += 4) {  // four independent loads per step
      u4v q[4];
#pragma unroll
      for (uint32_t h = 0; h < 4; ++h) q[h] = u + h < hi ? v[u + h] : (u4v)kPad;
#pragma unroll
      for (uint32_t h = 0; h < 4; ++h) c += (q[h].x < mine) + (q[h].y < mine) + (q[h].z < mine) + (q[h].w < mine);
    }
    if (c) atomicAdd(&ranks[r], c);
  }
  __syncthreads();
  for (uint32_t i = tid; i < n; i += bd)
    if (ranks[i] < keep) out[ranks[i]] = buf[i];
  __syncthreads();
}

// Class max of one slice, then the slice's records sorted.  Two load forms:
// scalar (any strides: a lane per anchor, four class groups per anchor) and,
// when anchors are contiguous in 16-byte groups (the production [B,4+nc,A]
// layout read through its [B,A,4+nc] view), a 16-byte load of eight anchors
// per lane and class, 32 class groups per octet of anchors.  The class groups
// meet in LDS, where the packed (key << 16 | class) minimum keeps the first
// class with the best key.
__global__ __launch_bounds__(kSliceThreads) void slice_kernel(SplitPlan p) {
  constexpr uint32_t kTiles = kSlice / 64;                  // scalar form: 64-anchor tiles
  constexpr uint32_t kGroups = kSliceThreads / kSlice;      // scalar form: class groups per anchor
  constexpr uint32_t kUnroll = 16;      // scalar form: class loads in flight per lane
  constexpr uint32_t kOctets = kSlice / 8;
  constexpr uint32_t kVGroups = kSliceThreads / kOctets;   // vector form: class groups per octet
  constexpr uint32_t kVUnroll = 4;      // vector form: 16-byte loads in flight per lane
  __shared__ uint32_t g_kc[kVGroups * kSlice];
  __shared__ uint16_t g_bits[kVGroups * kSlice];
  __shared__ __attribute__((aligned(16))) uint32_t recs[kSlice];
  __shared__ uint32_t ranks[kSlice], sorted[kSlice];
  const uint32_t b = blockIdx.y, slice = blockIdx.x, tid = threadIdx.x;
  const uint16_t* img = p.L.x + b * p.L.sb;
  const uint32_t sc = (uint32_t)p.L.sc;
  uint32_t groups;
  if (p.vec_classes) {
    const uint32_t o = tid % kOctets, g = tid / kOctets;
    const uint32_t a0 = slice * kSlice + o * 8u;
    uint32_t kc[8], bits[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      kc[j] = kPad;
      bits[j] = 0;
    }
    if (a0 < p.A) {  // A % 8 == 0: the octet is whole
      for (uint32_t c0 = g; c0 < p.nc; c0 += kVGroups * kVUnroll) {
        u4v v[kVUnroll];
#pragma unroll
        for (uint32_t u = 0; u < kVUnroll; ++u) {
          const uint32_t c = c0 + u * kVGroups;
          v[u] = c < p.nc ? *reinterpret_cast<const u4v*>(img + (4u + c) * sc + a0) : (u4v)0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < kVUnroll; ++u) {
          const uint32_t c = c0 + u * kVGroups;
          if (c < p.nc) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              const uint32_t h = (v[u][j / 2] >> (16 * (j & 1))) & 0xffffu;
              const uint32_t k = (score_key(h) << 16) | c;
              if (k < kc[j]) {
                kc[j] = k;
                bits[j] = h;
              }
            }
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      g_kc[g * kSlice + o * 8 + j] = kc[j];
      g_bits[g * kSlice + o * 8 + j] = (uint16_t)bits[j];
    }
    groups = kVGroups;
  } else {
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t local = (wave % kTiles) * 64u + lane, grp = wave / kTiles;
    const uint32_t a = slice * kSlice + local;
    uint32_t best = kPad, bb = 0u;
    if (a < p.A) {
      // one image spans fewer than 2^31 elements (checked on the host)
      const uint32_t row = a * (uint32_t)p.L.sa + 4u * sc;
      for (uint32_t c0 = grp; c0 < p.nc; c0 += kGroups * kUnroll) {
        uint32_t bits[kUnroll];
#pragma unroll
        for (uint32_t u = 0; u < kUnroll; ++u) {
          const uint32_t c = c0 + u * kGroups;
          bits[u] = c < p.nc ? img[row + c * sc] : 0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < kUnroll; ++u) {
          const uint32_t c = c0 + u * kGroups;
          const uint32_t k = c < p.nc ? (score_key(bits[u]) << 16) | c : kPad;
          if (k < best) {
            best = k;
            bb = bits[u];
          }
        }
      }
    }
    g_kc[grp * kSlice + local] = best;
    g_bits[grp * kSlice + local] = (uint16_t)bb;
    groups = kGroups;
  }
  __syncthreads();
  // Minimum over the class groups of each anchor.  Keys carry their class in
  // the low bits, so every key of an anchor is distinct and any reduction
  // order gives the same minimum (and its score bits).  The vector form's 32
  // groups reduce in two levels with every load of a level in flight at once
  // (a serial loop of 31 dependent LDS reads cost ~3 us per slice).
  constexpr uint32_t kParts = kSliceThreads / kSlice;  // 4
  __shared__ uint32_t part_kc[kParts * kSlice];
  __shared__ uint16_t part_bits[kParts * kSlice];
  auto reduce = [&](const uint32_t* kcs, const uint16_t* bitss, auto count, uint32_t first, uint32_t& best,
                    uint32_t& bb) {
    constexpr uint32_t N = decltype(count)::value;
    uint32_t k[N], h[N];
#pragma unroll
    for (uint32_t g = 0; g < N; ++g) {
      k[g] = kcs[(first + g) * kSlice];
      h[g] = bitss[(first + g) * kSlice];
    }
    best = k[0];
    bb = h[0];
#pragma unroll
    for (uint32_t g = 1; g < N; ++g)
      if (k[g] < best) {
        best = k[g];
        bb = h[g];
      }
  };
  uint32_t best = kPad, bb = 0u;
  if (groups == kVGroups) {
    static_assert(kVGroups == kParts * 8, "two-level group reduction");
    const uint32_t x = tid % kSlice, q = tid / kSlice;
    reduce(g_kc + x, g_bits + x, std::integral_constant<uint32_t, 8>(), q * 8u, best, bb);
    part_kc[q * kSlice + x] = best;
    part_bits[q * kSlice + x] = (uint16_t)bb;
    __syncthreads();
    if (tid < kSlice)
      reduce(part_kc + tid, part_bits + tid, std::integral_constant<uint32_t, kParts>(), 0u, best, bb);
  } else if (tid < kSlice) {
    static_assert(kGroups == kParts, "scalar form: one group per part");
    reduce(g_kc + tid, g_bits + tid, std::integral_constant<uint32_t, kGroups>(), 0u, best, bb);
  }
  if (tid < kSlice) {
    const uint32_t a = slice * kSlice + tid;
    uint32_t rec = kPad;
    if (a < p.A) {
      const size_t t = (size_t)b * p.A + a;
      p.bits1[t] = (uint16_t)bb;
      p.cls1[t] = (int32_t)(best & 0xffffu);
      if (p.tr.class_max) static_cast<uint16_t*>(p.tr.class_max)[t] = (uint16_t)bb;
      rec = (best & 0xffff0000u) | a;
    }
    recs[tid] = rec;
  }
  __syncthreads();
  const uint32_t n = min(kSlice, p.A - slice * kSlice);
  rank_sort<kSliceThreads>(recs, n, n, ranks, sorted);
  if (tid < kSlice) p.lists1_rec[((size_t)b * p.lists1 + slice) * kSlice + tid] = tid < n ? sorted[tid] : kPad;
}

// Wave-wide max and inclusive prefix sum by DPP row operations and the
// gfx950 permlane swaps (VALU only; a ds_bpermute shuffle costs ~150 cycles
// per dependent step, these a few each).
__device__ __forceinline__ uint32_t xor16(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return (threadIdx.x & 16u) ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t xor32(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (threadIdx.x & 32u) ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true));   // xor 1
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true));   // xor 2
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xF, 0xF, true));  // row_ror:4
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, true));  // row_ror:8
  v = max(v, xor16(v));
  return max(v, xor32(v));
}
// Inclusive prefix sum across the wave's 64 lanes.
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t v) {
  const uint32_t lane = threadIdx.x & 63u;
  // within rows of 16: shifts by 1, 2, 4, 8 (lanes shifted in from outside the row add 0)
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);  // row_shr:8
  // across rows: add the total of every earlier row
  const uint32_t row_total = (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
  const uint32_t t1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 31);
  const uint32_t t2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 47);
  v += lane >= 16 ? row_total : 0u;
  v += lane >= 32 ? t1 : 0u;
  v += lane >= 48 ? t2 : 0u;
  return v;
}

// Merge candidates of `nl` sorted lists held in LDS (list l at lists + l *
// pitch, length len[l], kPad beyond): cnt[l] records of list l are at most R
// (see above); they are copied to cand[off[l] ...], their list to from[...];
// off[nl] is the total.  q: the prefix length (0: choose it here).  Ends with
// a block barrier.
__device__ __forceinline__ void merge_candidates(const uint32_t* lists, uint32_t pitch, const uint32_t* len,
                                                 uint32_t nl, uint32_t K, uint32_t q, uint32_t* cnt, uint32_t* off,
                                                 uint32_t* cand, uint8_t* from) {
  const uint32_t tid = threadIdx.x;
  if (tid < 64) {  // wave 0; lane t handles lists t and t + 64
    if (q == 0) {
      // lane i tries q0 + i * step (q0 = ceil(K / nl)); the first lane whose
      // prefixes hold K records wins.  Lane 63 tries q >= K, which always holds.
      const uint32_t q0 = (K + nl - 1) / nl;
      const uint32_t step = max(1u, (K - min(K, q0) + 62u) / 63u);
      const uint32_t qi = min(K, q0 + tid * step);
      uint32_t sum = 0;
      for (uint32_t l = 0; l < nl; ++l) sum += min(qi, len[l]);
      const uint64_t ok = __ballot(sum >= K);
      q = (uint32_t)__shfl((int)qi, __builtin_ctzll(ok), 64);
    }
    // the bound R: the largest prefix end
    uint32_t m[2], R = 0;
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) {
      const uint32_t l = tid + 64 * h;
      m[h] = l < nl ? min(q, len[l]) : 0u;
      if (m[h]) R = max(R, lists[l * pitch + m[h] - 1]);
    }
    R = wave_max_u32(R);
    // cnt: records <= R, at least m; scan 16 at a time past the prefix
    uint32_t c[2];
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) {
      const uint32_t l = tid + 64 * h;
      c[h] = m[h];
      if (l < nl) {
        const uint32_t* lp = lists + l * pitch;
        const uint32_t n = len[l];
        for (;;) {
          const uint32_t c4 = c[h] & ~3u;
          uint32_t hit = 0;
#pragma unroll
          for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t at = c4 + 4 * u;
            const u4v v = at < n ? reinterpret_cast<const u4v*>(lp)[at / 4] : (u4v)kPad;
            hit += (v.x <= R) + (v.y <= R) + (v.z <= R) + (v.w <= R);
          }
          const uint32_t before = c[h] - c4;  // records of the first vector already counted
          const uint32_t found = hit - min(hit, before);
          c[h] += found;
          if (found < 16 - before || c[h] >= n) break;
        }
        c[h] = min(c[h], n);
        cnt[l] = c[h];
      }
    }
    const uint32_t incl0 = wave_scan_u32(c[0]);
    const uint32_t total0 = (uint32_t)__builtin_amdgcn_readlane((int)incl0, 63);
    const uint32_t incl1 = wave_scan_u32(c[1]) + total0;
    if (tid < nl) off[tid] = incl0 - c[0];
    if (tid + 64 < nl) off[tid + 64] = incl1 - c[1];
    if (tid == 63) off[nl] = incl1;
  }
  __syncthreads();
  // copy each list's candidates; wave w takes lists w, w + 16, ...
  const uint32_t lane = tid & 63u;
  for (uint32_t l = tid >> 6; l < nl; l += kSplitThreads >> 6)
    for (uint32_t i = lane; i < cnt[l]; i += 64) {
      cand[off[l] + i] = lists[l * pitch + i];
      from[off[l] + i] = (uint8_t)l;
    }
  __syncthreads();
}

// Sum over aligned groups of 8 lanes, every lane gets its group's total: xor
// 1 and 2 by quad permutes, xor 4 by row shifts (DPP, no LDS round trip).
__device__ __forceinline__ uint32_t group8_sum(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true);  // quad_perm [1,0,3,2]
  v += (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true);  // quad_perm [2,3,0,1]
  const uint32_t up = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x104, 0xF, 0xF, true);    // row_shl:4
  const uint32_t down = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x114, 0xF, 0xF, true);  // row_shr:4
  return v + ((threadIdx.x & 4u) ? down : up);
}

// Ranks this block's share of the candidates.  A group of 8 lanes takes one
// candidate; lane o counts the candidates below it in lists o, o + 8, ...
// (its own list: its position), and the counts add up across the group to
// the candidate's rank.  Calls emit(rank, rec) for ranks below K.  Rounds are
// wave-uniform, so the cross-lane sums always see their whole group.
template <typename Emit>
__device__ __forceinline__ void rank_candidates(const uint32_t* lists, uint32_t pitch, const uint32_t* cnt,
                                                const uint32_t* off, const uint32_t* cand, const uint8_t* from,
                                                uint32_t nl, uint32_t K, Emit emit) {
  constexpr uint32_t G = 8;
  const uint32_t C = off[nl];
  const uint32_t share = (C + kMergeBlocks - 1) / kMergeBlocks;
  const uint32_t j0 = blockIdx.x * share, j1 = min(C, j0 + share);
  const uint32_t groups = kSplitThreads / G, group = threadIdx.x / G, o0 = threadIdx.x % G;
  for (uint32_t base = j0; base < j1; base += groups) {
    const uint32_t j = base + group;
    const bool valid = j < j1;
    uint32_t rec = 0, below = 0;
    if (valid) {
      rec = cand[j];
      const uint32_t l = from[j];
      for (uint32_t o = o0; o < nl; o += G)
        below += o == l ? j - off[l] : count_below(lists + o * pitch, cnt[o], rec);
    }
    below = group8_sum(below);
    if (valid && o0 == 0 && below < K) emit(below, rec);
  }
}

// Output row r of batch b: anchor a, label, score bits.
// All loads come before any store: a wave waits for its stores as well as its
// loads when it needs a load result, so interleaving them would serialise on
// store completion.
// Row t of out (fp32 bits: box, score, label) and its trace entries.
__device__ __forceinline__ void put_row(uint32_t* out, const thin_select_trace& tr, size_t t, const uint32_t (&box)[4],
                                        int64_t a, int64_t label, uint32_t sbits, int64_t stage2) {
  uint32_t* o = out + t * 6;
#pragma unroll
  for (int c = 0; c < 4; ++c) o[c] = float_bits(box[c]);
  o[4] = float_bits(sbits);
  o[5] = __float_as_uint((float)label);
  if (tr.stage2 && stage2 >= 0) static_cast<int64_t*>(tr.stage2)[t] = stage2;
  if (tr.anchors) static_cast<int64_t*>(tr.anchors)[t] = a;
  if (tr.labels) static_cast<int64_t*>(tr.labels)[t] = label;
  if (tr.top_values) static_cast<uint16_t*>(tr.top_values)[t] = (uint16_t)sbits;
}

__device__ __forceinline__ void pack_out(const SplitPlan& p, uint32_t b, uint32_t r, int64_t a, int64_t label,
                                         uint32_t sbits, int64_t stage2) {
  const uint16_t* bx = p.L.x + b * p.L.sb + a * p.L.sa;
  uint32_t box[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) box[c] = bx[c * p.L.sc];
  put_row(p.out, p.tr, (size_t)b * p.K + r, box, a, label, sbits, stage2);
}

__global__ __launch_bounds__(kSplitThreads) void merge1_kernel(SplitPlan p) {
  __shared__ __attribute__((aligned(16))) uint32_t lists[kMaxLists * kSliceLds];
  __shared__ uint32_t cand[kMaxLists * kSlice];
  __shared__ uint8_t from[kMaxLists * kSlice];
  __shared__ uint32_t len[kMaxLists], cnt[kMaxLists], off[kMaxLists + 1];
  const uint32_t b = blockIdx.y, tid = threadIdx.x;
  const uint32_t nl = p.lists1, total = nl * kSlice;
  const u4v* src = reinterpret_cast<const u4v*>(p.lists1_rec + (size_t)b * total);
  for (uint32_t v = tid; v < total / 4; v += kSplitThreads) {
    const uint32_t l = v / (kSlice / 4), i4 = v - l * (kSlice / 4);
    reinterpret_cast<u4v*>(lists)[l * (kSliceLds / 4) + i4] = src[v];
  }
  if (tid < nl) len[tid] = min(kSlice, p.A - tid * kSlice);
  __syncthreads();
  merge_candidates(lists, kSliceLds, len, nl, p.K, p.q1, cnt, off, cand, from);
  rank_candidates(lists, kSliceLds, cnt, off, cand, from, nl, p.K, [&](uint32_t rank, uint32_t rec) {
    const uint32_t a = rec & 0xffffu;
    const size_t t = (size_t)b * p.K + rank;
    if (p.tr.stage1) static_cast<int64_t*>(p.tr.stage1)[t] = a;
    if (p.agnostic) {
      const size_t ba = (size_t)b * p.A + a;
      pack_out(p, b, rank, a, p.cls1[ba], p.bits1[ba], -1);
    } else {
      p.stage1[t] = (int32_t)a;
      if (rank == p.K - 1) p.thresh[b] = rec >> 16;
    }
  });
}

__global__ __launch_bounds__(kSplitThreads) void pairs_kernel(SplitPlan p) {
  __shared__ __attribute__((aligned(16))) uint32_t surv[kPairCap];
  __shared__ uint32_t ranks[kPairCap];
  __shared__ uint32_t sorted[kSplitMaxK];
  __shared__ int32_t anchors[kSplitMaxK];
  __shared__ uint32_t s_count;
  const uint32_t b = blockIdx.y, tid = threadIdx.x;
  const uint32_t r0 = blockIdx.x * p.ranks_per, r1 = min(p.K, r0 + p.ranks_per);
  const uint32_t nr = r1 > r0 ? r1 - r0 : 0u;
  const uint32_t T1 = p.thresh[b];
  if (tid == 0) s_count = 0;
  for (uint32_t r = tid; r < nr; r += kSplitThreads) anchors[r] = p.stage1[(size_t)b * p.K + r0 + r];
  __syncthreads();
  const uint32_t pairs = nr * p.nc;
  for (uint32_t j = tid; j < pairs; j += kSplitThreads) {
    const uint32_t rr = j / p.nc, c = j - rr * p.nc;
    const uint32_t bits = p.L.x[b * p.L.sb + (int64_t)anchors[rr] * p.L.sa + (int64_t)(4 + c) * p.L.sc];
    const uint32_t flat = (r0 + rr) * p.nc + c;
    if (p.tr.gathered) static_cast<uint16_t*>(p.tr.gathered)[(size_t)b * p.K * p.nc + flat] = (uint16_t)bits;
    const uint32_t k = score_key(bits);
    if (k <= T1) surv[atomicAdd(&s_count, 1u)] = (k << 16) | flat;
  }
  __syncthreads();
  const uint32_t n = s_count, keep = min(n, p.K);
  if (tid < 4 && n + tid < kPairCap) surv[n + tid] = kPad;  // pad to a whole vector
  __syncthreads();
  rank_sort<kSplitThreads>(surv, n, keep, ranks, sorted);
  uint32_t* dst = p.lists2_rec + ((size_t)b * p.pair_blocks + blockIdx.x) * p.pitch2;
  for (uint32_t i = tid; i < keep; i += kSplitThreads) dst[i] = sorted[i];
  if (tid == 0) p.count2[(size_t)b * p.pair_blocks + blockIdx.x] = keep;
}

__global__ __launch_bounds__(kSplitThreads) void merge2_kernel(SplitPlan p) {
  __shared__ __attribute__((aligned(16))) uint32_t lists[kMerge2Words];
  __shared__ uint32_t cand[kMerge2Words];
  __shared__ uint8_t from[kMerge2Words];
  __shared__ uint32_t len[kMaxLists], cnt[kMaxLists], off[kMaxLists + 1];
  __shared__ int32_t anchors[kSplitMaxK];
  const uint32_t b = blockIdx.y, tid = threadIdx.x;
  const uint32_t nl = p.pair_blocks, pl = p.lds_pitch2;
  const uint32_t* src = p.lists2_rec + (size_t)b * nl * p.pitch2;
  if (tid < nl) len[tid] = p.count2[(size_t)b * nl + tid];
  for (uint32_t r = tid; r < p.K; r += kSplitThreads) anchors[r] = p.stage1[(size_t)b * p.K + r];
  __syncthreads();
  for (uint32_t v = tid; v < nl * pl; v += kSplitThreads) {
    const uint32_t l = v / pl, i = v - l * pl;
    lists[v] = i < len[l] ? src[l * p.pitch2 + i] : kPad;
  }
  __syncthreads();
  merge_candidates(lists, pl, len, nl, p.K, 0, cnt, off, cand, from);
  rank_candidates(lists, pl, cnt, off, cand, from, nl, p.K, [&](uint32_t rank, uint32_t rec) {
    const uint32_t flat = rec & 0xffffu;
    const uint32_t r1 = flat / p.nc, c = flat - r1 * p.nc;
    const int64_t a = anchors[r1];
    const uint32_t sbits = p.L.x[b * p.L.sb + a * p.L.sa + (int64_t)(4 + c) * p.L.sc];
    pack_out(p, b, rank, a, c, sbits, flat);
  });
}

// ---------------------------------------------------------------- two-launch selection
// The selection in two launches, for one image or a few:
//
//   runs   (grid runs x B, 512 threads): per anchor of kRun, the three
//          smallest (key << 16 | class) over the classes; the run's
//          (key << 16 | anchor) records sorted (a bitonic network over two
//          waves) -> runs_rec, with each record's row key (below) ->
//          runs_side; per anchor a 16-byte info record (box, class-max score
//          bits and class, second key and class) -> info.
//   finish (grid B, 1024 threads): the stage-1 candidates of the sorted runs
//          (the prefix bound of the split kernels), sorted, while the info of
//          every candidate and the score rows of the few candidates whose
//          third key could reach the bound are in flight; stage 2 from the K
//          class-max pairs, the second pairs and those rows; rows packed
//          from LDS.
//
// Stage 2 is the top K of the stage-1 anchors' pairs keyed at most T1 (the K
// class-max pairs are among them): the class-max pairs (key_r, r * nc +
// class_r), the second pair of every anchor whose second key is at most T1,
// and, for an anchor whose third key is at most T1, every pair of its row.
// T1 is at most the candidate bound, so those rows are among the prefetched
// ones.  A second pair's score bits follow from its key, except for NaN and
// zero keys (several encodings each): rows with such a second key are
// prefetched too.  A run record's row key is the smallest key that makes its
// row needed: the third key, or the second key when that is NaN or zero.  When the rows do not fit (thousands of tied scores), or a
// trace of the gathered scores is asked for, every stage-1 row is gathered
// into an LDS table instead, and ties beyond kSortCap survivors go through a
// radix select of the K-th smallest pair.
//
// Sorting in one workgroup is a bitonic network over at most kSortCap
// records, held by four waves (E records per thread for n = 256E; smaller n a
// record per thread): exchanges within a thread in registers, within a wave
// by DPP and permlane swaps, between waves through LDS.  More stage-1
// candidates than kSortCap go through an exact radix select of the K-th
// smallest record first (four 8-bit digits, LDS histograms), so only K
// records are sorted.  Records are unique, so the network's order is the
// stable (key, index) order.
constexpr uint32_t kRun = 128;             // anchors per sorted run
constexpr uint32_t kRunThreads = 512;      // runs_kernel workgroups
constexpr uint32_t kMaxRuns = 128;         // runs per image (A <= 16384)
constexpr uint32_t kRunPitch = kRun + 4;   // finish LDS words per run list (run l on banks 4l mod 64)
constexpr uint32_t kSidePitch = kRun + 8;  // finish LDS halves per run row-key list (16-byte rows)
constexpr uint32_t kFinishThreads = 1024;  // finish_kernel workgroups
constexpr uint32_t kSortCap = 1024;        // records one bitonic sort holds
constexpr uint32_t kPairTable = 32768;     // K * nc limit: every stage-1 row in LDS (fallback)
constexpr uint32_t kGatherBatch = 32;      // fallback gather: pair loads in flight per thread
constexpr uint32_t kMaxX = 256;            // prefetched candidate rows
constexpr uint32_t kXTable = 16384;        // their fp16 scores in LDS
constexpr uint32_t kXBatch = 8;            // prefetched row loads per thread
constexpr uint32_t kNoX = 0xffffu;
// finish_kernel's reused LDS region (32-bit words): the runs and their side
// keys, then the candidate tables, then (fallback) the pair table; info1
// lies past the pair table and survives it.
constexpr uint32_t kRegSide = kMaxRuns * kRunPitch;            // runs: row keys (u16)
constexpr uint32_t kRegWords = kRegSide + kMaxRuns * kSidePitch / 2;
constexpr uint32_t kRegInfoSlot = 8192;                        // u4v [kSortCap]: info per slot
constexpr uint32_t kRegXTable = kRegInfoSlot + 4 * kSortCap;   // u16 [kXTable]
constexpr uint32_t kRegInfo1 = kRegXTable + kXTable / 2;       // u4v [kSplitMaxK]: info per stage-1 rank
static_assert(kRegInfo1 + 4 * kSplitMaxK <= kRegWords, "finish LDS region");
static_assert(kPairTable / 2 <= kRegInfo1 && kMaxRuns * kRun / 2 <= kRegInfoSlot, "finish LDS aliasing");

struct RunsPlan {
  Layout L;
  uint32_t A, nc, K;
  uint32_t runs;          // runs per image: ceil(A / kRun)
  uint32_t q;             // prefix length whose run prefixes hold K records (host: A and K only)
  uint32_t rows_per;      // finish: stage-1 ranks per gather pass, kFinishThreads / nc
  int32_t agnostic;
  int32_t vec_classes;    // anchors contiguous in aligned 16-byte groups
  int32_t row_classes;    // classes contiguous, rows in aligned 8-byte chunks, nc % 4 == 0
  uint32_t* runs_rec;     // [B, runs, kRun]: sorted records
  uint16_t* runs_side;    // [B, runs, kRun]: row key of each record's anchor
  u4v* info;              // [B, A] halves: box[4], class-max bits, class, second key, second class
  uint32_t* out;          // [B, K, 6] fp32 bits
  thin_select_trace tr;
};

// The middle of three (a v_med3_u32).
__device__ __forceinline__ uint32_t umed3(uint32_t a, uint32_t b, uint32_t c) {
  return max(min(a, b), min(max(a, b), c));
}
__device__ __forceinline__ uint32_t half_of(const u4v& v, uint32_t i) { return (v[i / 2] >> (16 * (i & 1))) & 0xffffu; }
// Key 0 (NaN) and 0x7fff (zero) stand for several encodings; every other
// key is one fp16 encoding, run_key's inverse.
__device__ __forceinline__ bool key_ambiguous(uint32_t k) { return k == 0u || k == 0x7fffu; }
__device__ __forceinline__ uint32_t key_bits(uint32_t k) { return k > 0x7fffu ? k + 1u : 0x7fffu - k; }

// One bitonic exchange with the lane J away (J < 64): the lower lane of the
// pair keeps the minimum when `up`, the maximum otherwise.  Whole waves only.
template <uint32_t J>
__device__ __forceinline__ uint32_t bitonic_xchg(uint32_t x, bool up) {
  const uint32_t p = dev::lane_xor_bits<J>(x);
  const bool keep_min = ((threadIdx.x & J) == 0) == up;
  return keep_min ? min(x, p) : max(x, p);
}
// The in-wave end of a bitonic merge: exchanges at J, J / 2, ..., 1.
template <uint32_t J>
__device__ __forceinline__ uint32_t bitonic_tail(uint32_t x, bool up) {
  if constexpr (J == 0) {
    return x;
  } else {
    return bitonic_tail<J / 2>(bitonic_xchg<J>(x, up), up);
  }
}
// Sorts the wave's 64 records, ascending where bit 6 of n (the record's index
// in the block's sequence) is clear and descending where it is set: the
// first six merges of a bitonic sort of the whole sequence.
template <uint32_t K = 2>
__device__ __forceinline__ uint32_t bitonic_wave(uint32_t x, uint32_t n) {
  if constexpr (K > 64) {
    return x;
  } else {
    return bitonic_wave<K * 2>(bitonic_tail<K / 2>(x, (n & K) == 0), n);
  }
}

// Sorts buf[0, n) ascending, n a power of two in [64, 256], thread i holding
// record i; exchanges of 64 and more go through xch (2 x kSortCap words,
// alternate halves, so one barrier per stage).  Every thread of the block
// calls it after a barrier that published buf; ends with a barrier.
__device__ __forceinline__ void block_sort1(uint32_t* buf, uint32_t n, uint32_t* xch) {
  const uint32_t tid = threadIdx.x;
  const bool live = tid < n;  // whole waves
  uint32_t x = kPad;
  if (live) x = bitonic_wave(buf[tid], tid);
  uint32_t half = 0;
  for (uint32_t k = 128; k <= n; k <<= 1) {
    const bool up = (tid & k) == 0;
    for (uint32_t j = k >> 1; j >= 64; j >>= 1) {
      uint32_t* s = xch + half;
      half ^= kSortCap;
      if (live) s[tid] = x;
      __syncthreads();
      if (live) {
        const uint32_t p = s[tid ^ j];
        const bool keep_min = ((tid & j) == 0) == up;
        x = keep_min ? min(x, p) : max(x, p);
      }
    }
    if (live) x = bitonic_tail<32>(x, up);
  }
  if (live) buf[tid] = x;
  __syncthreads();
}

// One stage (merge size K, distance J) of a bitonic sort of 256 * E records,
// thread t < 256 holding records t * E .. t * E + E - 1 in x.
template <uint32_t E, uint32_t K, uint32_t J>
__device__ __forceinline__ void bitonic_stage(uint32_t (&x)[E], bool live, uint32_t* xch, uint32_t& half) {
  const uint32_t tid = threadIdx.x;
  if constexpr (J < E) {  // within the thread
    if (live) {
#pragma unroll
      for (uint32_t e = 0; e < E; ++e)
        if ((e & J) == 0) {
          const bool up = ((tid * E + e) & K) == 0;  // constant when K <= E
          const uint32_t lo = min(x[e], x[e | J]), hi = max(x[e], x[e | J]);
          x[e] = up ? lo : hi;
          x[e | J] = up ? hi : lo;
        }
    }
  } else if constexpr (J < 64 * E) {  // within the wave: lane xor J / E
    if (live) {
      const bool up = ((tid * E) & K) == 0;
      const bool keep_min = ((tid & (J / E)) == 0) == up;
#pragma unroll
      for (uint32_t e = 0; e < E; ++e) {
        const uint32_t p = dev::lane_xor_bits<J / E>(x[e]);
        x[e] = keep_min ? min(x[e], p) : max(x[e], p);
      }
    }
  } else {  // between waves, through LDS
    uint32_t* s = xch + half;
    half ^= kSortCap;
    if (live) {
#pragma unroll
      for (uint32_t e = 0; e < E; ++e) s[tid * E + e] = x[e];
    }
    __syncthreads();
    if (live) {
      const bool up = ((tid * E) & K) == 0;
#pragma unroll
      for (uint32_t e = 0; e < E; ++e) {
        const uint32_t n = tid * E + e;
        const uint32_t p = s[n ^ J];
        const bool keep_min = ((n & J) == 0) == up;
        x[e] = keep_min ? min(x[e], p) : max(x[e], p);
      }
    }
  }
}
template <uint32_t E, uint32_t K, uint32_t J>
__device__ __forceinline__ void bitonic_merge(uint32_t (&x)[E], bool live, uint32_t* xch, uint32_t& half) {
  if constexpr (J >= 1) {
    bitonic_stage<E, K, J>(x, live, xch, half);
    bitonic_merge<E, K, J / 2>(x, live, xch, half);
  }
}
template <uint32_t E, uint32_t K = 2>
__device__ __forceinline__ void bitonic_sort(uint32_t (&x)[E], bool live, uint32_t* xch, uint32_t& half) {
  if constexpr (K <= 256 * E) {
    bitonic_merge<E, K, K / 2>(x, live, xch, half);
    bitonic_sort<E, K * 2>(x, live, xch, half);
  }
}
// Sorts buf[0, 256 * E) ascending; same contract as block_sort1.
template <uint32_t E>
__device__ __forceinline__ void block_sort_e(uint32_t* buf, uint32_t* xch) {
  const uint32_t tid = threadIdx.x;
  const bool live = tid < 256;  // waves 0-3
  uint32_t x[E];
  if (live) {
#pragma unroll
    for (uint32_t e = 0; e < E; ++e) x[e] = buf[tid * E + e];
  }
  uint32_t half = 0;
  bitonic_sort<E>(x, live, xch, half);
  if (live) {
#pragma unroll
    for (uint32_t e = 0; e < E; ++e) buf[tid * E + e] = x[e];
  }
  __syncthreads();
}
// Sorts buf[0, n) ascending, n a power of two in [64, kSortCap].
__device__ __forceinline__ void block_sort(uint32_t* buf, uint32_t n, uint32_t* xch) {
  if (n <= 256) block_sort1(buf, n, xch);
  else if (n == 512) block_sort_e<2>(buf, xch);
  else block_sort_e<4>(buf, xch);
}

__device__ __forceinline__ uint32_t pow2_at_least(uint32_t n) {
  uint32_t p = 64;
  while (p < n) p <<= 1;
  return p;
}

// The K-th smallest (K >= 1) of the unique records a traversal visits, by
// four 8-bit digits, most significant first: each pass counts the digits of
// the records that match the digits chosen so far (a wave whose matching
// lanes share one digit adds once), and wave 0 finds the digit where the
// running count reaches K.  visit(f) calls f(rec) on the calling thread's
// share of the records.  Every thread of the block calls it; hist: 256 words
// of LDS, sel: 2.
template <typename Visit>
__device__ uint32_t radix_select(Visit visit, uint32_t K, uint32_t* hist, uint32_t* sel) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  uint32_t prefix = 0, kk = K;
  for (int shift = 24; shift >= 0; shift -= 8) {
    const uint32_t hi = shift == 24 ? 0u : ~0u << (shift + 8);
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    visit([&](uint32_t rec) {
      const bool match = (rec & hi) == (prefix & hi);
      const uint32_t d = (rec >> shift) & 255u;
      const uint64_t act = __ballot(match);
      if (!act) return;
      const uint32_t first = (uint32_t)__builtin_ctzll(act);
      const uint32_t d0 = (uint32_t)__builtin_amdgcn_readlane((int)d, (int)first);
      const uint64_t same = __ballot(match && d == d0);
      if (same == act) {
        if (lane == first) atomicAdd(&hist[d0], (uint32_t)__popcll(act));
      } else if (match) {
        atomicAdd(&hist[d], 1u);
      }
    });
    __syncthreads();
    if (tid < 64) {
      uint32_t h[4], s = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h[i] = hist[tid * 4 + i];
        s += h[i];
      }
      const uint32_t incl = wave_scan_u32(s);
      uint32_t cum = incl - s;
      if (cum < kk && kk <= incl) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (kk <= cum + h[i]) {
            sel[0] = tid * 4 + i;
            sel[1] = kk - cum;
            break;
          }
          cum += h[i];
        }
      }
    }
    __syncthreads();
    prefix |= sel[0] << shift;
    kk = sel[1];
  }
  return prefix;
}

// The two-launch selection's key: score_key's order (NaN first, then
// descending value, +0 and -0 equal) as 0x7fff - |h| for positive h and
// 0x7fff + |h| for negative h, NaN -> 0.  It differs from score_key only in
// its values for negative scores (one less), which never meet score_key's:
// every key of this path comes from run_key / run_key2 and turns back into
// bits through key_bits.
__device__ __forceinline__ uint32_t run_key(uint32_t h) {
  const uint32_t m = h & 0x7fffu;
  if (m > 0x7c00u) return 0u;
  return (h & 0x8000u) ? 0x7fffu + m : 0x7fffu - m;
}
// run_key of both fp16 halves of w at once (16-bit packed arithmetic).
__device__ __forceinline__ uint32_t run_key2(uint32_t w) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  typedef short i16x2 __attribute__((ext_vector_type(2)));
  const uint32_t m = w & 0x7fff7fffu;
  const u16x2 mv = __builtin_bit_cast(u16x2, m);
  const uint32_t pos = m ^ 0x7fff7fffu;  // 0x7fff - |h|
  const uint32_t neg = __builtin_bit_cast(uint32_t, mv + (u16x2)0x7fff);
  const uint32_t sign = __builtin_bit_cast(uint32_t, __builtin_bit_cast(i16x2, w) >> (i16x2)15);
  const uint32_t key = (neg & sign) | (pos & ~sign);
  // |h| - 0x7c01 is negative exactly for the non-NaN halves
  const i16x2 t = __builtin_bit_cast(i16x2, m) - (i16x2)0x7c01;
  return key & __builtin_bit_cast(uint32_t, t >> (i16x2)15);
}

// Folds (key << 16 | class) k of a later class, score bits h, into the three
// smallest so far (b < s < t; kPad where missing): every key is distinct, so
// the new third is the middle of (s, k, t) and the new second the middle of
// (b, k, s).
__device__ __forceinline__ void fold3(uint32_t& b, uint32_t& s, uint32_t& t, uint32_t& bits, uint32_t k, uint32_t h) {
  t = umed3(s, k, t);
  s = umed3(b, k, s);
  if (k < b) {
    b = k;
    bits = h;
  }
}

// Class keys of kRun anchors (the two load forms of slice_kernel, and a row
// form for rows of contiguous classes) and their box channels; then the
// run's records sorted: waves 0 and 1 sort 64 each (ascending, descending),
// one LDS exchange at distance 64 and the in-wave end of the last merge.
__global__ __launch_bounds__(kRunThreads) void runs_kernel(RunsPlan p) {
  constexpr uint32_t kTiles = kRun / 64;                  // scalar form: 64-anchor tiles
  constexpr uint32_t kGroups = kRunThreads / kRun;        // scalar form: class groups per anchor
  constexpr uint32_t kUnroll = 16;                        // scalar form: class loads in flight per lane
  constexpr uint32_t kOctets = kRun / 8;
  constexpr uint32_t kVGroups = kRunThreads / kOctets;    // vector form: class groups per octet
  constexpr uint32_t kVUnroll = 4;                        // vector form: 16-byte loads in flight per lane
  constexpr uint32_t kRUnroll = 6;                        // row form: 8-byte loads in flight per lane
  static_assert(kRunThreads == 4 * kRun, "row form: four lanes per anchor");
  constexpr uint32_t kParts = kRunThreads / kRun;         // group-reduction parts per anchor
  static_assert(kVGroups == kParts * 8 && kGroups == kParts && kGroups == 4, "group reduction shape");
  // per class group and anchor: the three smallest (key << 16 | class), best bits
  __shared__ uint32_t g_b[kVGroups * kRun], g_s[kVGroups * kRun], g_t[kVGroups * kRun];
  __shared__ uint16_t g_bits[kVGroups * kRun];
  __shared__ uint32_t part_b[kParts * kRun], part_s[kParts * kRun], part_t[kParts * kRun];
  __shared__ uint16_t part_bits[kParts * kRun];
  __shared__ uint16_t box[4 * kRun];
  __shared__ uint16_t side_of[kRun];
  __shared__ uint32_t xch[kRun];
  const uint32_t b = blockIdx.y, run = blockIdx.x, tid = threadIdx.x;
  const uint16_t* img = p.L.x + b * p.L.sb;
  const uint32_t sc = (uint32_t)p.L.sc;
  if (p.vec_classes) {
    const uint32_t o = tid % kOctets, g = tid / kOctets;
    const uint32_t a0 = run * kRun + o * 8u;
    uint32_t kb[8], ks[8], kt[8], bits[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      kb[j] = kPad;
      ks[j] = kPad;
      kt[j] = kPad;
      bits[j] = 0;
    }
    if (a0 < p.A) {  // A % 8 == 0: the octet is whole
      // box channel g of the octet (groups 0-3), in flight with the classes
      const u4v bv = *reinterpret_cast<const u4v*>(img + min(g, 3u) * sc + a0);
      for (uint32_t c0 = g; c0 < p.nc; c0 += kVGroups * kVUnroll) {
        u4v v[kVUnroll];
#pragma unroll
        for (uint32_t u = 0; u < kVUnroll; ++u) {
          const uint32_t c = c0 + u * kVGroups;
          v[u] = c < p.nc ? *reinterpret_cast<const u4v*>(img + (4u + c) * sc + a0) : (u4v)0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < kVUnroll; ++u) {
          const uint32_t c = c0 + u * kVGroups;
          if (c < p.nc) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {  // two anchors per 32-bit word
              const uint32_t w = v[u][q], kw = run_key2(w);
              fold3(kb[2 * q], ks[2 * q], kt[2 * q], bits[2 * q], (kw << 16) | c, w & 0xffffu);
              fold3(kb[2 * q + 1], ks[2 * q + 1], kt[2 * q + 1], bits[2 * q + 1], (kw & 0xffff0000u) | c, w >> 16);
            }
          }
        }
      }
      if (g < 4) {
#pragma unroll
        for (int j = 0; j < 8; ++j) box[g * kRun + o * 8 + j] = (uint16_t)half_of(bv, j);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t at = g * kRun + o * 8 + j;
      g_b[at] = kb[j];
      g_s[at] = ks[j];
      g_t[at] = kt[j];
      g_bits[at] = (uint16_t)bits[j];
    }
  } else if (p.row_classes) {
    // four lanes per anchor: lane g reads the anchor's 8-byte class chunks g,
    // g + 4, ... (lane 0 also the box chunk before them), then the quad merges
    // its four triples in two exchanges, leaving the anchor's three in every lane
    typedef uint32_t u2v __attribute__((ext_vector_type(2)));
    const uint32_t local = tid / 4u, g = tid % 4u, a = run * kRun + local, nch = p.nc / 4u;
    uint32_t kb = kPad, ks = kPad, kt = kPad, bb = 0u;
    u2v bx = (u2v)0u;
    if (a < p.A) {
      // one image spans fewer than 2^31 elements (checked on the host)
      const u2v* row = reinterpret_cast<const u2v*>(img + a * (uint32_t)p.L.sa);
      if (g == 0) bx = row[0];
      for (uint32_t j0 = g; j0 < nch; j0 += 4u * kRUnroll) {
        u2v v[kRUnroll];
#pragma unroll
        for (uint32_t u = 0; u < kRUnroll; ++u) {
          const uint32_t j = j0 + 4u * u;
          v[u] = j < nch ? row[1u + j] : (u2v)0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < kRUnroll; ++u) {
          const uint32_t j = j0 + 4u * u;
          if (j < nch) {
#pragma unroll
            for (uint32_t q = 0; q < 2; ++q) {  // classes 4j + 2q and 4j + 2q + 1
              const uint32_t w = v[u][q], kw = run_key2(w), c = 4u * j + 2u * q;
              fold3(kb, ks, kt, bb, (kw << 16) | c, w & 0xffffu);
              fold3(kb, ks, kt, bb, (kw & 0xffff0000u) | (c + 1u), w >> 16);
            }
          }
        }
      }
    }
    auto merge = [&](uint32_t pb, uint32_t ps, uint32_t pt, uint32_t ph) {
      uint32_t unused = 0;
      fold3(kb, ks, kt, bb, pb, ph);
      fold3(kb, ks, kt, unused, ps, 0u);  // never below the partner's best, so bits stay
      fold3(kb, ks, kt, unused, pt, 0u);
    };
    merge(dev::lane_xor_bits<1>(kb), dev::lane_xor_bits<1>(ks), dev::lane_xor_bits<1>(kt),
          dev::lane_xor_bits<1>(bb));
    merge(dev::lane_xor_bits<2>(kb), dev::lane_xor_bits<2>(ks), dev::lane_xor_bits<2>(kt),
          dev::lane_xor_bits<2>(bb));
    if (g == 0) {
      g_b[local] = kb;
      g_s[local] = ks;
      g_t[local] = kt;
      g_bits[local] = (uint16_t)bb;
#pragma unroll
      for (uint32_t c = 0; c < 4; ++c) box[c * kRun + local] = (uint16_t)(bx[c / 2] >> (16 * (c & 1)));
    }
  } else {
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t local = (wave % kTiles) * 64u + lane, grp = wave / kTiles;
    const uint32_t a = run * kRun + local;
    uint32_t kb = kPad, ks = kPad, kt = kPad, bb = 0u;
    if (a < p.A) {
      // one image spans fewer than 2^31 elements (checked on the host)
      const uint32_t base = a * (uint32_t)p.L.sa;
      const uint32_t bxv = img[base + grp * sc];  // box channel grp
      const uint32_t row = base + 4u * sc;
      for (uint32_t c0 = grp; c0 < p.nc; c0 += kGroups * kUnroll) {
        uint32_t bits[kUnroll];
#pragma unroll
        for (uint32_t u = 0; u < kUnroll; ++u) {
          const uint32_t c = c0 + u * kGroups;
          bits[u] = c < p.nc ? img[row + c * sc] : 0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < kUnroll; ++u) {
          const uint32_t c = c0 + u * kGroups;
          if (c < p.nc) fold3(kb, ks, kt, bb, (run_key(bits[u]) << 16) | c, bits[u]);
        }
      }
      box[grp * kRun + local] = (uint16_t)bxv;
    }
    const uint32_t at = grp * kRun + local;
    g_b[at] = kb;
    g_s[at] = ks;
    g_t[at] = kt;
    g_bits[at] = (uint16_t)bb;
  }
  __syncthreads();
  // The three smallest over the class groups of each anchor (all keys
  // distinct, so any merge order gives the same three); the vector form's 32
  // groups reduce in two levels.
  auto reduce = [&](const uint32_t* bs, const uint32_t* ss, const uint32_t* ts, const uint16_t* hs, auto count,
                    uint32_t first, uint32_t& kb, uint32_t& ks, uint32_t& kt, uint32_t& bb) {
    constexpr uint32_t N = decltype(count)::value;
    uint32_t vb[N], vs[N], vt[N], vh[N];
#pragma unroll
    for (uint32_t g = 0; g < N; ++g) {
      const uint32_t at = (first + g) * kRun;
      vb[g] = bs[at];
      vs[g] = ss[at];
      vt[g] = ts[at];
      vh[g] = hs[at];
    }
    kb = vb[0];
    ks = vs[0];
    kt = vt[0];
    bb = vh[0];
#pragma unroll
    for (uint32_t g = 1; g < N; ++g) {
      fold3(kb, ks, kt, bb, vb[g], vh[g]);
      uint32_t unused = 0;
      fold3(kb, ks, kt, unused, vs[g], 0u);  // never below the group's best, so bits stay
      fold3(kb, ks, kt, unused, vt[g], 0u);
    }
  };
  uint32_t kb = kPad, ks = kPad, kt = kPad, bb = 0u;
  if (p.vec_classes) {
    const uint32_t x = tid % kRun, q = tid / kRun;
    reduce(g_b + x, g_s + x, g_t + x, g_bits + x, std::integral_constant<uint32_t, 8>(), q * 8u, kb, ks, kt, bb);
    part_b[q * kRun + x] = kb;
    part_s[q * kRun + x] = ks;
    part_t[q * kRun + x] = kt;
    part_bits[q * kRun + x] = (uint16_t)bb;
    __syncthreads();
    if (tid < kRun)
      reduce(part_b + tid, part_s + tid, part_t + tid, part_bits + tid, std::integral_constant<uint32_t, kParts>(), 0u,
             kb, ks, kt, bb);
  } else if (p.row_classes) {
    if (tid < kRun) {
      kb = g_b[tid];
      ks = g_s[tid];
      kt = g_t[tid];
      bb = g_bits[tid];
    }
  } else if (tid < kRun) {
    reduce(g_b + tid, g_s + tid, g_t + tid, g_bits + tid, std::integral_constant<uint32_t, kGroups>(), 0u, kb, ks, kt,
           bb);
  }
  uint32_t rec = kPad;
  if (tid < kRun) {
    const uint32_t a = run * kRun + tid;
    if (a < p.A) {
      const size_t t = (size_t)b * p.A + a;
      u4v iv;
      iv[0] = box[tid] | ((uint32_t)box[kRun + tid] << 16);
      iv[1] = box[2 * kRun + tid] | ((uint32_t)box[3 * kRun + tid] << 16);
      iv[2] = bb | (kb << 16);                    // class-max bits, class
      iv[3] = (ks >> 16) | (ks << 16);            // second key, second class (0xffff, 0xffff: none)
      p.info[t] = iv;
      if (p.tr.class_max) static_cast<uint16_t*>(p.tr.class_max)[t] = (uint16_t)bb;
      rec = (kb & 0xffff0000u) | a;
    }
    const uint32_t sk = ks >> 16;
    side_of[tid] = (uint16_t)min(kt >> 16, key_ambiguous(sk) ? sk : 0xffffu);
    rec = bitonic_wave(rec, tid);
    xch[tid] = rec;
  }
  __syncthreads();
  if (tid < kRun) {
    const uint32_t o = xch[tid ^ 64u];
    rec = (tid & 64u) ? max(rec, o) : min(rec, o);
    rec = bitonic_tail<32>(rec, true);
    const size_t at = ((size_t)b * p.runs + run) * kRun + tid;
    p.runs_rec[at] = rec;
    p.runs_side[at] = rec == kPad ? (uint16_t)0xffffu : side_of[(rec & 0xffffu) - run * kRun];
  }
}

// Stage-1 candidates, their sort, stage 2 and the rows, for image blockIdx.x.
__global__ __launch_bounds__(kFinishThreads) void finish_kernel(RunsPlan p) {
  __shared__ __attribute__((aligned(16))) uint32_t region[kRegWords];
  __shared__ uint32_t sortbuf[kSortCap], s2buf[kSortCap + 64];  // s2buf: K pairs and up to 64 extras
  __shared__ uint32_t xch[2 * kSortCap];
  __shared__ uint16_t anchor_of[kSortCap], xslot[kSortCap], xlist[kMaxX], xrank[kSortCap], anchors1[kSplitMaxK],
      x1[kSplitMaxK];
  __shared__ uint32_t cnt[kMaxRuns], off[kMaxRuns + 1];
  __shared__ uint32_t hist[256], sel[2], bound, count, count2, nx, nxr;
  const uint32_t b = blockIdx.x, tid = threadIdx.x, nl = p.runs, K = p.K, nc = p.nc;
  const uint16_t* img = p.L.x + b * p.L.sb;
  const uint32_t sa = (uint32_t)p.L.sa, sc = (uint32_t)p.L.sc;
  uint32_t* lists = region;
  uint16_t* lside = reinterpret_cast<uint16_t*>(region + kRegSide);
  u4v* info_slot = reinterpret_cast<u4v*>(region + kRegInfoSlot);
  uint16_t* xtable = reinterpret_cast<uint16_t*>(region + kRegXTable);
  u4v* info1 = reinterpret_cast<u4v*>(region + kRegInfo1);
  uint16_t* table = reinterpret_cast<uint16_t*>(region);  // fallback: [K * nc]
  const u4v* info_g = p.info + (size_t)b * p.A;

  // the runs and their row keys into LDS: every 16-byte load issued before
  // any is stored
  {
    constexpr uint32_t kV = kRun / 4, kPer = kMaxRuns * kV / kFinishThreads;
    constexpr uint32_t kSV = kRun / 8, kSPer = kMaxRuns * kSV / kFinishThreads;
    const uint32_t total = nl * kV, stotal = nl * kSV;
    const u4v* src = reinterpret_cast<const u4v*>(p.runs_rec + (size_t)b * nl * kRun);
    const u4v* ssrc = reinterpret_cast<const u4v*>(p.runs_side + (size_t)b * nl * kRun);
    u4v v[kPer], sv[kSPer];
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i)
      if (tid + i * kFinishThreads < total) v[i] = src[tid + i * kFinishThreads];
#pragma unroll
    for (uint32_t i = 0; i < kSPer; ++i)
      if (tid + i * kFinishThreads < stotal) sv[i] = ssrc[tid + i * kFinishThreads];
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t e = tid + i * kFinishThreads;
      if (e < total) reinterpret_cast<u4v*>(lists)[(e / kV) * (kRunPitch / 4) + e % kV] = v[i];
    }
#pragma unroll
    for (uint32_t i = 0; i < kSPer; ++i) {
      const uint32_t e = tid + i * kFinishThreads;
      if (e < stotal) reinterpret_cast<u4v*>(lside)[(e / kSV) * (kSidePitch / 8) + e % kSV] = sv[i];
    }
  }
  if (tid == 0) {
    count = 0;
    count2 = 0;
    nx = 0;
    nxr = 0;
  }
  __syncthreads();

  // Candidates: records up to R, the largest of the prefix ends (the first
  // min(q, len) records of each run hold at least K records, so the K-th
  // smallest is at most R).  Wave 0, lane t: runs t and t + 64; the count
  // past the prefix scans 16 records a step.
  if (tid < 64) {
    uint32_t len[2], m[2], R = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t l = tid + 64u * h;
      len[h] = l < nl ? min(kRun, p.A - l * kRun) : 0u;
      m[h] = min(p.q, len[h]);
      if (m[h]) R = max(R, lists[l * kRunPitch + m[h] - 1]);
    }
    R = wave_max_u32(R);
    uint32_t c[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t* lp = lists + (tid + 64u * h) * kRunPitch;
      const uint32_t n = len[h];
      c[h] = m[h];  // the first m records are at most R
      while (c[h] < n) {
        const uint32_t c4 = c[h] & ~3u;
        uint32_t hit = 0;
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
          const uint32_t at = c4 + 4 * u;
          const u4v v = at < n ? reinterpret_cast<const u4v*>(lp)[at / 4] : (u4v)kPad;
          hit += (v.x <= R) + (v.y <= R) + (v.z <= R) + (v.w <= R);
        }
        const uint32_t before = c[h] - c4;  // records of the first vector already counted
        const uint32_t found = hit - min(hit, before);
        c[h] = min(c[h] + found, n);
        if (found < 16 - before) break;
      }
    }
    const uint32_t incl0 = wave_scan_u32(c[0]);
    const uint32_t total0 = (uint32_t)__builtin_amdgcn_readlane((int)incl0, 63);
    const uint32_t incl1 = wave_scan_u32(c[1]) + total0;
    if (tid < nl) {
      cnt[tid] = c[0];
      off[tid] = incl0 - c[0];
    }
    if (tid + 64 < nl) {
      cnt[tid + 64] = c[1];
      off[tid + 64] = incl1 - c[1];
    }
    if (tid == 63) {
      off[kMaxRuns] = incl1;
      bound = R;
    }
  }
  __syncthreads();
  const uint32_t C = off[kMaxRuns], Rkey = bound >> 16;
  // eight threads per run walk its candidates
  auto candidates = [&](auto&& f) {
    const uint32_t l = tid >> 3;
    if (l < nl) {
      const uint32_t n = cnt[l], at = off[l];
      for (uint32_t k = tid & 7u; k < n; k += 8) f(lists[l * kRunPitch + k], lside[l * kSidePitch + k], at + k);
    }
  };
  const bool few = C <= kSortCap;
  uint32_t n1 = pow2_at_least(K);
  if (few) {
    // Candidate slots in (run, position) order, sorted as (key << 16 | slot):
    // runs cover increasing anchor ranges and sort equal keys by anchor, so
    // slot order among equal keys is anchor order and the sort gives the
    // stage-1 order.  Rows to prefetch: a row key at most the bound.
    candidates([&](uint32_t rec, uint32_t rk, uint32_t at) {
      sortbuf[at] = (rec & 0xffff0000u) | at;
      anchor_of[at] = (uint16_t)(rec & 0xffffu);
      uint32_t x = kNoX;
      if (!p.agnostic && rk <= Rkey) {
        x = atomicAdd(&nx, 1u);
        if (x < kMaxX) xlist[x] = (uint16_t)at;
        else x = kNoX;
      }
      xslot[at] = (uint16_t)x;
    });
    n1 = pow2_at_least(C);
    for (uint32_t i = C + tid; i < n1; i += kFinishThreads) sortbuf[i] = kPad;
  } else {
    const uint32_t T = radix_select(
        [&](auto&& f) { candidates([&](uint32_t rec, uint32_t, uint32_t) { f(rec); }); }, K, hist, sel);
    candidates([&](uint32_t rec, uint32_t, uint32_t) {
      if (rec <= T) {
        const uint32_t slot = atomicAdd(&count, 1u);
        if (slot < kSortCap) sortbuf[slot] = rec;  // exactly K (records are unique)
      }
    });
    for (uint32_t i = K + tid; i < n1; i += kFinishThreads) sortbuf[i] = kPad;
  }
  __syncthreads();
  const uint32_t G = p.rows_per, cls = p.agnostic ? 0u : tid % nc, grow = p.agnostic ? 0u : tid / nc;
  const uint32_t NX = nx;
  const bool fast = few && !p.agnostic && NX <= kMaxX && NX <= kXBatch * G && NX * nc <= kXTable && !p.tr.gathered;
  u4v my_info = (u4v)0u;
  uint32_t xr[kXBatch];
  if (few) {
    // In flight across the sort (nothing reads them before it ends): the
    // info of candidate slot tid and the prefetched rows (thread (grow, cls):
    // class cls of rows grow, grow + G, ...).
    if (tid < C) my_info = info_g[min((uint32_t)anchor_of[tid], p.A - 1)];
    if (fast && grow < G) {
#pragma unroll
      for (uint32_t i = 0; i < kXBatch; ++i) {
        const uint32_t x = grow + i * G;
        if (x < NX) xr[i] = img[min((uint32_t)anchor_of[xlist[x]], p.A - 1) * sa + (4u + cls) * sc];
      }
    }
  }
  block_sort(sortbuf, n1, xch);

  if (few) {
    // the runs are dead: the slot tables take their place
    if (tid < C) info_slot[tid] = my_info;
    if (fast && grow < G) {
#pragma unroll
      for (uint32_t i = 0; i < kXBatch; ++i) {
        const uint32_t x = grow + i * G;
        if (x < NX) xtable[x * nc + cls] = (uint16_t)xr[i];
      }
    }
    __syncthreads();
  }
  // stage 1: ranks 0..K-1 (at least K real records were sorted; the clamps
  // only keep addresses in bounds)
  const uint32_t T1 = sortbuf[K - 1] >> 16;
  for (uint32_t r = tid; r < K; r += kFinishThreads) {
    const uint32_t rec = sortbuf[r];
    u4v iv;
    uint32_t a, x = kNoX;
    if (few) {
      const uint32_t s = min(rec & 0xffffu, C - 1);
      a = anchor_of[s];
      iv = info_slot[s];
      x = xslot[s];
    } else {
      a = min(rec & 0xffffu, p.A - 1);
      iv = info_g[a];  // many tied candidates: one more round of loads
    }
    anchors1[r] = (uint16_t)a;
    if (p.tr.stage1) static_cast<int64_t*>(p.tr.stage1)[(size_t)b * K + r] = a;
    info1[r] = iv;
    x1[r] = (uint16_t)x;
    if (fast) {
      s2buf[r] = (rec & 0xffff0000u) | (r * nc + half_of(iv, 5));  // the class-max pair
      const uint32_t sk = half_of(iv, 6);
      if (sk <= T1) {
        if (x != kNoX) {
          xrank[atomicAdd(&nxr, 1u)] = (uint16_t)r;  // its row holds the extra pairs
        } else {
          const uint32_t slot = atomicAdd(&count2, 1u);  // the second pair only (third key above T1)
          if (K + slot < kSortCap + 64) s2buf[K + slot] = (sk << 16) | (r * nc + half_of(iv, 7));
        }
      }
    }
  }
  __syncthreads();

  if (p.agnostic) {
    for (uint32_t i = tid; i < K; i += kFinishThreads) {
      const u4v iv = info1[i];
      const uint32_t bx[4] = {half_of(iv, 0), half_of(iv, 1), half_of(iv, 2), half_of(iv, 3)};
      put_row(p.out, p.tr, (size_t)b * K + i, bx, anchors1[i], half_of(iv, 5), half_of(iv, 4), -1);
    }
    return;
  }

  if (fast) {
    // the other pairs of the prefetched rows keyed at most T1
    const uint32_t NE = nxr;
    if (grow < G) {
      for (uint32_t e = grow; e < NE; e += G) {
        const uint32_t r = xrank[e];
        const uint32_t x = min((uint32_t)x1[r], kMaxX - 1);
        if (cls != half_of(info1[r], 5)) {
          const uint32_t key = run_key(xtable[x * nc + cls]);
          if (key <= T1) {
            const uint32_t slot = atomicAdd(&count2, 1u);
            if (K + slot < kSortCap + 64) s2buf[K + slot] = (key << 16) | (r * nc + cls);
          }
        }
      }
    }
    __syncthreads();
    const uint32_t E2 = count2, S = K + E2;
    // row i of the output: pair record rec
    auto emit = [&](uint32_t i, uint32_t rec) {
      const uint32_t f = min(rec & 0xffffu, K * nc - 1);  // a pair index (clamp: LDS bounds only)
      const uint32_t r = f / nc, c = f - r * nc;
      const u4v iv = info1[r];
      const uint32_t x = x1[r];
      const uint32_t sbits = c == half_of(iv, 5) ? half_of(iv, 4)
                             : x != kNoX        ? xtable[min(x, kMaxX - 1) * nc + c]
                                                : key_bits(half_of(iv, 6));  // the second pair
      const uint32_t bx[4] = {half_of(iv, 0), half_of(iv, 1), half_of(iv, 2), half_of(iv, 3)};
      put_row(p.out, p.tr, (size_t)b * K + i, bx, anchors1[r], c, sbits, f);
    };
    if (E2 <= 64) {
      // The class-max pairs s2buf[0, K) are in order already (keys follow the
      // stage-1 ranks, and so do the pair indices of equal keys).  A record's
      // row is the records below it: its index among the class-max pairs
      // plus the extras below it (a count over the few extras), or, for an
      // extra, the extras below it plus the class-max pairs below it (a
      // binary search).
      const uint32_t* ext = s2buf + K;
      for (uint32_t i = tid; i < K + E2; i += kFinishThreads) {
        const uint32_t rec = s2buf[i];
        uint32_t row = i < K ? i : 0u;
        for (uint32_t j = 0; j < E2; ++j) row += ext[j] < rec;
        if (i >= K) {
          uint32_t lo = 0, hi = K;
          while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (s2buf[mid] < rec) lo = mid + 1;
            else hi = mid;
          }
          row += lo;
        }
        if (row < K) emit(row, rec);
      }
      return;
    }
    if (S <= kSortCap) {
      const uint32_t n2 = pow2_at_least(S);
      for (uint32_t i = S + tid; i < n2; i += kFinishThreads) s2buf[i] = kPad;
      __syncthreads();
      block_sort(s2buf, n2, xch);
      for (uint32_t i = tid; i < K; i += kFinishThreads) emit(i, s2buf[i]);
      return;
    }
  }

  // Fallback: every stage-1 row into the LDS table (thread (grow, cls): class
  // cls of ranks grow, grow + G, ...); pairs keyed at most T1 survive.
  if (tid == 0) count = 0;
  __syncthreads();
  if (grow < G) {
    for (uint32_t r0 = grow; r0 < K; r0 += G * kGatherBatch) {
      uint32_t h[kGatherBatch];
#pragma unroll
      for (uint32_t u = 0; u < kGatherBatch; ++u) {
        const uint32_t r = min(r0 + u * G, K - 1);
        h[u] = img[(uint32_t)anchors1[r] * sa + (4u + cls) * sc];
      }
#pragma unroll
      for (uint32_t u = 0; u < kGatherBatch; ++u) {
        const uint32_t r = r0 + u * G;
        if (r < K) {
          const uint32_t f = r * nc + cls;
          table[f] = (uint16_t)h[u];
          if (p.tr.gathered) static_cast<uint16_t*>(p.tr.gathered)[(size_t)b * K * nc + f] = (uint16_t)h[u];
          const uint32_t key = run_key(h[u]);
          if (key <= T1) {
            const uint32_t slot = atomicAdd(&count, 1u);
            if (slot < kSortCap) s2buf[slot] = (key << 16) | f;
          }
        }
      }
    }
  }
  __syncthreads();
  // the survivors sorted, or (more than kSortCap: ties) the K-th smallest pair
  // record selected over the whole table and the K records up to it sorted
  const uint32_t S = count;
  uint32_t have2 = K;
  if (S <= kSortCap) {
    have2 = S;
  } else {
    const uint32_t total = K * nc;
    if (tid == 0) count2 = 0;
    const uint32_t T = radix_select(
        [&](auto&& f) {
          for (uint32_t i = tid; i < total; i += kFinishThreads) f((run_key(table[i]) << 16) | i);
        },
        K, hist, sel);
    for (uint32_t i = tid; i < total; i += kFinishThreads) {
      const uint32_t rec = (run_key(table[i]) << 16) | i;
      if (rec <= T) {
        const uint32_t slot = atomicAdd(&count2, 1u);
        if (slot < kSortCap) s2buf[slot] = rec;  // exactly K
      }
    }
  }
  const uint32_t n2 = pow2_at_least(have2);
  for (uint32_t i = have2 + tid; i < n2; i += kFinishThreads) s2buf[i] = kPad;
  __syncthreads();
  block_sort(s2buf, n2, xch);
  for (uint32_t i = tid; i < K; i += kFinishThreads) {
    const uint32_t f = min(s2buf[i] & 0xffffu, K * nc - 1);
    const uint32_t r = f / nc, c = f - r * nc;
    const u4v iv = info1[r];
    const uint32_t bx[4] = {half_of(iv, 0), half_of(iv, 1), half_of(iv, 2), half_of(iv, 3)};
    put_row(p.out, p.tr, (size_t)b * K + i, bx, anchors1[r], c, table[f], f);
  }
}

// ---------------------------------------------------------------- host

// Shape of the split selection for these sizes; ok == false leaves them to
// the one-workgroup-per-batch path (more anchors than 64 lists of kSlice,
// K above kSplitMaxK, or pair indices / pair lists too large).
struct SplitShape {
  bool ok;
  uint32_t lists1, q1, pair_blocks, ranks_per, pitch2, lds_pitch2;
};

SplitShape split_shape(int64_t B, int64_t A, int64_t nc, int64_t K, bool agnostic, int64_t image_extent) {
  SplitShape sh;
  memset(&sh, 0, sizeof sh);
  if (K < 1 || K > (int64_t)kSplitMaxK || A > (int64_t)(kMaxLists * kSlice) || B > 65535 ||
      image_extent >= ((int64_t)1 << 31))
    return sh;
  sh.lists1 = (uint32_t)((A + kSlice - 1) / kSlice);
  // q1: the smallest prefix length whose lists' prefixes hold K records
  for (uint32_t q = 1; q <= kSlice; ++q) {
    int64_t sum = 0;
    for (uint32_t l = 0; l < sh.lists1; ++l) sum += std::min<int64_t>(q, A - (int64_t)l * kSlice);
    if (sum >= K) {
      sh.q1 = q;
      break;
    }
  }
  if (!agnostic) {
    if (K * nc > 65536) return sh;
    const int64_t per = std::max<int64_t>(1, std::min<int64_t>(K, 2048 / nc));
    if (per * nc > (int64_t)kPairCap) return sh;
    sh.ranks_per = (uint32_t)per;
    sh.pair_blocks = (uint32_t)((K + per - 1) / per);
    sh.pitch2 = (uint32_t)((K + 3) & ~(int64_t)3);
    sh.lds_pitch2 = (uint32_t)(((K + 63) & ~(int64_t)63) + 4);
    if (sh.pair_blocks > kMaxLists || (int64_t)sh.pair_blocks * sh.lds_pitch2 > (int64_t)kMerge2Words) return sh;
  }
  sh.ok = true;
  return sh;
}

// Shape of the two-launch selection; ok == false leaves the sizes to the
// split kernels or the one-workgroup-per-batch path (K above kSplitMaxK, more
// than kMaxRuns runs, more classes than finish_kernel threads, or K * nc pair
// scores beyond its LDS table).
struct RunsShape {
  bool ok;
  uint32_t runs, q, rows_per;
};

RunsShape runs_shape(int64_t B, int64_t A, int64_t nc, int64_t K, bool agnostic, int64_t image_extent) {
  RunsShape r;
  memset(&r, 0, sizeof r);
  if (K < 1 || K > (int64_t)kSplitMaxK || A > (int64_t)(kMaxRuns * kRun) || B > 65535 ||
      image_extent >= ((int64_t)1 << 31))
    return r;
  if (!agnostic && (nc > (int64_t)kFinishThreads || K * nc > (int64_t)kPairTable)) return r;
  r.runs = (uint32_t)((A + kRun - 1) / kRun);
  // q: the smallest prefix length whose run prefixes hold K records (every
  // run holds kRun anchors but the last, which holds `last`)
  const int64_t last = A - (int64_t)(r.runs - 1) * kRun;
  const int64_t q = (K + r.runs - 1) / r.runs;
  r.q = (uint32_t)(q <= last ? q : (K - last + r.runs - 2) / (r.runs - 1));
  r.rows_per = agnostic ? 0u : (uint32_t)(kFinishThreads / nc);
  r.ok = true;
  return r;
}

struct WsLayout {
  size_t bits1, cls1, stage1, gathered, stage2, thresh, recs, lists1, lists2, count2, runs, runs_side, info, total;
  uint32_t recs_pitch;  // P for the large-K path (0 = not needed)
  SplitShape split;
  RunsShape two;        // the two-launch selection (taken before split when ok)
};

size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

// image_extent: elements one image of `decoded` spans (its largest offset + 1);
// -1 when unknown (workspace queries size for the split path whenever it
// could apply).
WsLayout ws_layout(int64_t B, int64_t A, int64_t nc, int64_t max_det, bool agnostic, int64_t image_extent = -1) {
  WsLayout w;
  memset(&w, 0, sizeof w);
  const int64_t K = max_det < A ? max_det : A;
  w.two = runs_shape(B, A, nc, K, agnostic, image_extent < 0 ? 0 : image_extent);
  if (!w.two.ok) w.split = split_shape(B, A, nc, K, agnostic, image_extent < 0 ? 0 : image_extent);
  size_t off = 0;
  w.bits1 = off; off += up256((size_t)(B * A) * 2);
  w.cls1 = off; off += up256((size_t)(B * A) * 4);
  w.stage1 = off; off += up256((size_t)(B * K) * 4);
  if (!agnostic) {
    w.gathered = off; off += up256((size_t)(B * K * nc) * 2);
    w.stage2 = off; off += up256((size_t)(B * K) * 4);
    w.thresh = off; off += up256((size_t)B * 4);
  }
  if (w.two.ok) {
    w.runs = off; off += up256((size_t)B * w.two.runs * kRun * 4);
    w.runs_side = off; off += up256((size_t)B * w.two.runs * kRun * 2);
    w.info = off; off += up256((size_t)(B * A) * 16);
  }
  if (w.split.ok) {
    w.lists1 = off; off += up256((size_t)B * w.split.lists1 * kSlice * 4);
    if (!agnostic) {
      w.lists2 = off; off += up256((size_t)B * w.split.pair_blocks * (size_t)w.split.pitch2 * 4);
      w.count2 = off; off += up256((size_t)B * w.split.pair_blocks * 4);
    }
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

namespace thin {
namespace {

// Elements one image of decoded [B, A, 4+nc] spans: its largest offset + 1.
int64_t image_extent(const thin_desc* d) {
  return 1 + (d->sizes[1] - 1) * d->strides[1] + (d->sizes[2] - 1) * d->strides[2];
}

// Argument checks shared by both entry points.  Sets *skip when the call has
// nothing to launch (empty batch or anchors, or K == 0 without a class_max
// trace: selection_flow.cpp:436-439).
thin_status select_validate(const thin_desc* decoded, int64_t max_det, void* out, const thin_select_trace* trace,
                            bool* skip) {
  *skip = false;
  THIN_REQUIRE(desc_valid(decoded), THIN_ERR_INVALID, "detection_select: invalid descriptor");
  THIN_REQUIRE(decoded->dtype == THIN_F16 && decoded->rank == 3, THIN_ERR_INVALID,
               "detection_select expects float16 [B,A,4+nc]");
  THIN_REQUIRE(decoded->sizes[2] > 4 && max_det >= 0, THIN_ERR_INVALID,
               "detection_select requires nc > 0 and max_det >= 0");
  const int64_t B = decoded->sizes[0], A = decoded->sizes[1], nc = decoded->sizes[2] - 4;
  const int64_t K = max_det < A ? max_det : A;
  if (B == 0 || A == 0 || (K == 0 && !(trace && trace->class_max))) {
    *skip = true;
    return THIN_OK;
  }
  THIN_REQUIRE(out != nullptr || K == 0, THIN_ERR_INVALID, "detection_select: null output");
  THIN_REQUIRE(A < ((int64_t)1 << 31) && K * nc < ((int64_t)1 << 31), THIN_ERR_UNSUPPORTED,
               "detection_select: candidate count exceeds 2^31");
  return THIN_OK;
}

// Enqueues the selection kernels over a validated call; `ws` holds w.total
// bytes, 256-byte aligned.  Every workspace region is written before it is
// read within the call, so no region needs clearing.
thin_status select_run(const thin_desc* decoded, int64_t max_det, bool agn, void* out, char* ws, const WsLayout& w,
                       const thin_select_trace* trace, hipStream_t stream) {
  const int64_t B = decoded->sizes[0], A = decoded->sizes[1], nc = decoded->sizes[2] - 4;
  const int64_t K = max_det < A ? max_det : A;
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
  const bool vec_classes = decoded->strides[1] == 1 && A % 8 == 0 && decoded->strides[2] % 8 == 0 &&
                           (B == 1 || decoded->strides[0] % 8 == 0) &&
                           reinterpret_cast<uintptr_t>(decoded->data) % 16 == 0;
  if (w.two.ok) {
    RunsPlan rp;
    memset(&rp, 0, sizeof rp);
    rp.L = L;
    rp.A = (uint32_t)A;
    rp.nc = (uint32_t)nc;
    rp.K = (uint32_t)K;
    rp.runs = w.two.runs;
    rp.q = w.two.q;
    rp.rows_per = w.two.rows_per;
    rp.agnostic = agn ? 1 : 0;
    rp.vec_classes = vec_classes ? 1 : 0;
    rp.row_classes = !vec_classes && decoded->strides[2] == 1 && decoded->strides[1] % 4 == 0 && nc % 4 == 0 &&
                             (B == 1 || decoded->strides[0] % 4 == 0) &&
                             reinterpret_cast<uintptr_t>(decoded->data) % 8 == 0
                         ? 1
                         : 0;
    rp.runs_rec = reinterpret_cast<uint32_t*>(ws + w.runs);
    rp.runs_side = reinterpret_cast<uint16_t*>(ws + w.runs_side);
    rp.info = reinterpret_cast<u4v*>(ws + w.info);
    rp.out = static_cast<uint32_t*>(out);
    rp.tr = tr;
    hipLaunchKernelGGL(runs_kernel, dim3(rp.runs, (uint32_t)B), dim3(kRunThreads), 0, stream, rp);
    THIN_LAUNCH_CHECK("select_runs");
    hipLaunchKernelGGL(finish_kernel, dim3((uint32_t)B), dim3(kFinishThreads), 0, stream, rp);
    THIN_LAUNCH_CHECK("select_finish");
    return THIN_OK;
  }
  if (w.split.ok) {
    SplitPlan sp;
    memset(&sp, 0, sizeof sp);
    sp.L = L;
    sp.A = (uint32_t)A;
    sp.nc = (uint32_t)nc;
    sp.K = (uint32_t)K;
    sp.lists1 = w.split.lists1;
    sp.q1 = w.split.q1;
    sp.pair_blocks = w.split.pair_blocks;
    sp.ranks_per = w.split.ranks_per;
    sp.pitch2 = w.split.pitch2;
    sp.lds_pitch2 = w.split.lds_pitch2;
    sp.agnostic = agn ? 1 : 0;
    sp.vec_classes = vec_classes ? 1 : 0;
    sp.bits1 = bits1;
    sp.cls1 = cls1;
    sp.lists1_rec = reinterpret_cast<uint32_t*>(ws + w.lists1);
    sp.stage1 = stage1;
    sp.thresh = agn ? nullptr : reinterpret_cast<uint32_t*>(ws + w.thresh);
    sp.lists2_rec = agn ? nullptr : reinterpret_cast<uint32_t*>(ws + w.lists2);
    sp.count2 = agn ? nullptr : reinterpret_cast<uint32_t*>(ws + w.count2);
    sp.out = static_cast<uint32_t*>(out);
    sp.tr = tr;
    const uint32_t nb = (uint32_t)B;
    hipLaunchKernelGGL(slice_kernel, dim3(sp.lists1, nb), dim3(kSliceThreads), 0, stream, sp);
    THIN_LAUNCH_CHECK("select_slice");
    hipLaunchKernelGGL(merge1_kernel, dim3(kMergeBlocks, nb), dim3(kSplitThreads), 0, stream, sp);
    THIN_LAUNCH_CHECK("select_merge1");
    if (agn) return THIN_OK;
    hipLaunchKernelGGL(pairs_kernel, dim3(sp.pair_blocks, nb), dim3(kSplitThreads), 0, stream, sp);
    THIN_LAUNCH_CHECK("select_pairs");
    hipLaunchKernelGGL(merge2_kernel, dim3(kMergeBlocks, nb), dim3(kSplitThreads), 0, stream, sp);
    THIN_LAUNCH_CHECK("select_merge2");
    return THIN_OK;
  }
  constexpr int kGroups = 16;
  hipLaunchKernelGGL((class_max_wide_kernel<kGroups>), dim3((uint32_t)((B * A + 63) / 64)), dim3(64 * kGroups), 0,
                     stream, L, B, A, nc, bits1, cls1, static_cast<uint16_t*>(tr.class_max));
  THIN_LAUNCH_CHECK("class_max");
  if (K == 0) return THIN_OK;
  RegTopkPlan rp;
  memset(&rp, 0, sizeof rp);
  rp.L = L;
  rp.K = (uint32_t)K;
  rp.nc = FastDiv::make((uint32_t)nc);
  rp.anchors = A;
  rp.out = static_cast<uint32_t*>(out);
  rp.tr = tr;
  const bool reg1 = A <= (int64_t)kRegMaxN && K <= (int64_t)kRegMaxK;
  const bool reg2 = K * nc <= (int64_t)kRegMaxN && K <= (int64_t)kRegMaxK;
  if (agn && reg1) {  // one launch: select anchors by their class max and pack
    rp.bits = bits1;
    rp.n = (uint32_t)A;
    rp.cls1 = cls1;
    launch_reg_topk<1>(rp, B, stream);
    THIN_LAUNCH_CHECK("topk_pack");
    return THIN_OK;
  }
  thin_status s;
  if (reg1) {
    rp.bits = bits1;
    rp.n = (uint32_t)A;
    rp.sel = stage1;
    rp.thresh = agn ? nullptr : reinterpret_cast<uint32_t*>(ws + w.thresh);  // T1 for the pair survivors
    launch_reg_topk<0>(rp, B, stream);
    THIN_LAUNCH_CHECK("topk_stage1");
  } else {
    s = topk(bits1, B, A, K, stage1, recs, w.recs_pitch, stream);
    if (s) return s;
  }
  if (!agn) {
    hipLaunchKernelGGL(gather_kernel, dim3(blocks_for((uint64_t)(B * K * nc))), dim3(kThreads), 0, stream, L, B, K,
                       nc, stage1, gathered, static_cast<uint16_t*>(tr.gathered));
    THIN_LAUNCH_CHECK("gather");
    if (reg2) {  // select pairs over the gathered scores and pack
      rp.bits = gathered;
      rp.stage1 = stage1;
      rp.n = (uint32_t)(K * nc);
      rp.sel = nullptr;
      launch_reg_topk<2>(rp, B, stream);
      THIN_LAUNCH_CHECK("topk_stage2");
      return THIN_OK;
    }
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

}  // namespace
}  // namespace thin

extern "C" thin_status thin_detection_select(const thin_desc* decoded, int64_t max_det, int32_t agnostic, void* out,
                                             void* workspace, size_t workspace_bytes,
                                             const thin_select_trace* trace, hipStream_t stream) {
  clear_error();
  bool skip = false;
  thin_status s = select_validate(decoded, max_det, out, trace, &skip);
  if (s != THIN_OK || skip) return s;
  const bool agn = agnostic != 0;
  const WsLayout w = ws_layout(decoded->sizes[0], decoded->sizes[1], decoded->sizes[2] - 4, max_det, agn,
                               image_extent(decoded));
  THIN_REQUIRE(workspace != nullptr && workspace_bytes >= w.total, THIN_ERR_WORKSPACE,
               "detection_select: workspace of %zu bytes needed, %zu given", w.total, workspace_bytes);
  THIN_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, THIN_ERR_WORKSPACE,
               "detection_select: workspace must be 256-byte aligned");
  return select_run(decoded, max_det, agn, out, static_cast<char*>(workspace), w, trace, stream);
}

// ---------------------------------------------------------------- allocation-free variant
// The workspace of thin_detection_select_noalloc lives in a static device
// array of this library (one copy per GPU, held until the process ends).  In
// host code `scratch` names a host-side shadow, not device memory: its device
// address comes from hipGetSymbolAddress, taken once per device on the first
// call with that device current, and only that address reaches the kernels.
namespace thin {
namespace {

constexpr int kScratchDevices = 64;
static __device__ __align__(256) unsigned char scratch[THIN_SELECT_SCRATCH_BYTES];

std::mutex g_scratch_mutex;
void* g_scratch_addr[kScratchDevices];

thin_status scratch_address(void** addr) {
  int device = -1;
  THIN_HIP_CHECK(hipGetDevice(&device));
  THIN_REQUIRE(device >= 0 && device < kScratchDevices, THIN_ERR_UNSUPPORTED,
               "detection_select_noalloc: device index %d beyond %d", device, kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_addr[device]) {
    void* p = nullptr;
    THIN_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    THIN_REQUIRE(p != nullptr && reinterpret_cast<uintptr_t>(p) % 256 == 0, THIN_ERR_HIP,
                 "detection_select_noalloc: scratch address %p is not 256-byte aligned", p);
    g_scratch_addr[device] = p;
  }
  *addr = g_scratch_addr[device];
  return THIN_OK;
}

}  // namespace
}  // namespace thin

extern "C" thin_status thin_detection_select_noalloc(const thin_desc* decoded, int64_t max_det, int32_t agnostic,
                                                     void* out, const thin_select_trace* trace, hipStream_t stream) {
  clear_error();
  bool skip = false;
  thin_status s = select_validate(decoded, max_det, out, trace, &skip);
  if (s != THIN_OK || skip) return s;
  const bool agn = agnostic != 0;
  const WsLayout w = ws_layout(decoded->sizes[0], decoded->sizes[1], decoded->sizes[2] - 4, max_det, agn,
                               image_extent(decoded));
  THIN_REQUIRE(w.total <= (size_t)THIN_SELECT_SCRATCH_BYTES, THIN_ERR_WORKSPACE,
               "detection_select_noalloc: these sizes need %zu bytes of scratch, the static scratch holds %zu "
               "(use thin_detection_select with a workspace)",
               w.total, (size_t)THIN_SELECT_SCRATCH_BYTES);
  void* ws = nullptr;
  s = scratch_address(&ws);
  if (s != THIN_OK) return s;
  return select_run(decoded, max_det, agn, out, static_cast<char*>(ws), w, trace, stream);
}
