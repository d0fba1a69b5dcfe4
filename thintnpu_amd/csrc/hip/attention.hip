// Fused blocked attention of the C2PSA block: the chain from the head-grouped
// blocked QKV tensor to the mixed values (whole_blocked.py:91-103) in one
// launch, with the bits of that chain:
//
//   Q-prescaled:  q'     = fp16(q * scale)                 channel_select, mul
//                 s[i,j] = fp16(sum_c q'[c,i] k[c,j])      layout_bmm (q^T k)
//   post-scale:   s[i,j] = fp16(fp16(sum_c q[c,i] k[c,j]) * scale)
//   both:         p[i,:] = softmax(s[i,:])                 row softmax
//                 o[c,i] = fp16(sum_t v[c,t] p[i,t])       layout_bmm (v p^T), blocked
//
// Each sum is thin_layout_bmm's sequential fp32 fma chain (reduction order
// 0..K-1 from +0, one rounding), and the softmax is the row kernel's fp16 core
// (dev::softmax_row_h8) with the reduction tree row_tree() picks for the
// [heads, T, T] scores, so the output equals the unfused chain bit for bit.
//
// One block per (head, 8 query rows), G / 8 waves (G lanes per softmax row,
// 64 / G rows per wave); the block's scores and probabilities never leave
// LDS:
//   1. q rows go to LDS (fp16) and each thread loads the k columns it owns.
//      v of the head is loaded into registers as 8-channel x 8-token tiles
//      after the scores, in flight through the softmax (issued first, its
//      51 KB a block queued ahead of q and k: 8.8 against 8.5 us).
//   2. scores, 8 rows x T columns: a thread owns one or two columns, 8 chains
//      of Dk fmas each.
//   3. softmax: G lanes per row, in place.
//   4. the v tiles, transposed to [T/8][Dv (+1 pad)][8], go to LDS.
//   5. mixed values: lane c owns channel c (and c + 64), one chain of T fmas
//      per row of its wave; v by 16-byte LDS reads per 8 steps, p by
//      broadcast reads, loaded four steps ahead.
#include "common.h"

#include <string.h>

namespace thin {
namespace {

using dev::h8;
typedef float f4 __attribute__((ext_vector_type(4)));

// Query rows per block (4 with one row per wave measured slower at 400 tokens
// x 4 heads: 11.0 against 8.9 us, though two blocks then share a CU).
constexpr uint32_t kAttnRows = 8;
constexpr uint32_t kAttnMaxTokens = 512;  // at most two score columns per thread
constexpr uint32_t kAttnVTiles = 512;     // at most this many 8x8 v tiles per head
constexpr uint32_t kAttnMaxLds = 64u * 1024u;
constexpr uint32_t kAttnStepsPerChunk = 4;  // 8-token steps of v p^T per LDS round (one row, one channel group)

struct AttnPlan {
  const _Float16* x;  // qkv [1, C1, T, 16]: token stride 16, in-block stride 1
  _Float16* y;        // out [1, heads * Dv / 16, T, 16]: same
  int64_t xs1, ys1;   // 16-channel block strides (elements)
  uint32_t T, Dv, group;  // tokens, value channels per head, channels per head group
  uint32_t row_blocks, grid;
  float scale;
  uint32_t prescale;
  uint32_t s_off, v_off;  // byte offsets of the score and v regions in LDS (q rows at 0)
};

// G lanes per softmax row, so 64 / G rows per wave and G / 8 waves per block
// of kAttnRows rows.
template <int DK, int G, int KPT, int CG>
__global__ __launch_bounds__(kAttnRows * G) void attention_kernel(AttnPlan p) {
  constexpr int RW = 64 / G;  // rows per wave
  constexpr int BI = (int)kAttnRows;
  constexpr uint32_t NT = kAttnRows * G;       // threads
  constexpr uint32_t VR = kAttnVTiles / NT;     // v tiles per thread
  constexpr uint32_t NCOL = kAttnMaxTokens / NT < 2 ? 1 : 2;  // score columns per thread
  constexpr uint32_t PF = RW * CG >= (int)kAttnStepsPerChunk ? 1u : kAttnStepsPerChunk / (RW * CG);
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  _Float16* Qs = reinterpret_cast<_Float16*>(lds);               // [BI][DK]
  _Float16* Ss = reinterpret_cast<_Float16*>(lds + p.s_off);     // [BI][T]
  h8* Vt = reinterpret_cast<h8*>(lds + p.v_off);                  // [T / 8][Dv + 1]
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t T = p.T, Dv = p.Dv, vpitch = Dv + 1u;  // the pad vector spreads v's LDS writes over the banks

  // blocks of one head on one XCD (dispatch deals blocks round-robin over 8)
  uint32_t b = blockIdx.x;
  if (p.grid % 8u == 0) b = (b % 8u) * (p.grid / 8u) + b / 8u;
  const uint32_t h = b / p.row_blocks;
  const uint32_t i0 = (b - h * p.row_blocks) * BI;
  const uint32_t ch0 = h * p.group;  // first channel of the head group (a multiple of 16)

  // 1. the q values and the thread's k columns j = tid + r * NT in flight
  //    together.  Every thread issues the same loads (indexes clamped in
  //    range, surplus values unused), so the compiler can count them: with
  //    loads under a branch its wait counts turn conservative.
  constexpr uint32_t QR = (BI * DK + NT - 1) / NT;  // q values per thread
  _Float16 qraw[QR];
#pragma unroll
  for (uint32_t r = 0; r < QR; ++r) {
    const uint32_t e = min(tid + r * NT, (uint32_t)(BI * DK) - 1u), i = e / DK, c = e % DK, t = min(i0 + i, T - 1);
    qraw[r] = p.x[(int64_t)((ch0 + c) >> 4) * p.xs1 + (int64_t)t * 16 + (c & 15u)];
  }
  h8 kc[NCOL][DK / 8];
#pragma unroll
  for (uint32_t r = 0; r < NCOL; ++r) {
    const uint32_t j = min(tid + r * NT, T - 1);
#pragma unroll
    for (int kb = 0; kb < DK / 16; ++kb) {
      const _Float16* src = p.x + (int64_t)((ch0 + DK) / 16u + kb) * p.xs1 + (int64_t)j * 16;
      kc[r][2 * kb] = *reinterpret_cast<const h8*>(src);
      kc[r][2 * kb + 1] = *reinterpret_cast<const h8*>(src + 8);
    }
  }
  // q rows into LDS, prescaled as the unfused chain's mul rounds them (fp16
  // values either way)
#pragma unroll
  for (uint32_t r = 0; r < QR; ++r) {
    const uint32_t e = tid + r * NT;
    if (e < (uint32_t)(BI * DK)) Qs[e] = p.prescale ? dev::to_half((float)qraw[r] * p.scale) : qraw[r];
  }
  __syncthreads();

  // 2. scores of the thread's columns: per row, the sequential chain over the
  //    key channels.  The q values of channel group c8 + 1 are read while
  //    group c8's fmas run (the compiler barriers keep it from hoisting every
  //    q read of the loop, which would exhaust the registers).
  {
    float acc[NCOL][BI];
#pragma unroll
    for (uint32_t r = 0; r < NCOL; ++r)
#pragma unroll
      for (int i = 0; i < BI; ++i) acc[r][i] = 0.f;
    h8 qa[BI], qb[BI];
    auto read_q = [&](h8 (&q)[BI], int c8) {
#pragma unroll
      for (int i = 0; i < BI; ++i) q[i] = *reinterpret_cast<const h8*>(&Qs[i * DK + 8 * c8]);
    };
    auto fmas = [&](const h8 (&q)[BI], int c8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
#pragma unroll
        for (uint32_t r = 0; r < NCOL; ++r) {
          const float k = (float)kc[r][c8][u];
#pragma unroll
          for (int i = 0; i < BI; ++i) acc[r][i] = __builtin_fmaf((float)q[i][u], k, acc[r][i]);
        }
      }
    };
    // pins the chains' values here: the fmas before, the next q reads after
    auto fence = [&]() {
#pragma unroll
      for (uint32_t r = 0; r < NCOL; ++r)
#pragma unroll
        for (int i = 0; i < BI; ++i) asm volatile("" : "+v"(acc[r][i])::"memory");
    };
    read_q(qa, 0);
#pragma unroll
    for (int c8 = 0; c8 < DK / 8; c8 += 2) {
      read_q(qb, c8 + 1);
      fmas(qa, c8);
      fence();
      if (c8 + 2 < DK / 8) read_q(qa, c8 + 2);
      fmas(qb, c8 + 1);
      fence();
    }
#pragma unroll
    for (uint32_t r = 0; r < NCOL; ++r) {
      const uint32_t j = tid + r * NT;
      if (j < T) {
#pragma unroll
        for (int i = 0; i < BI; ++i) {
          _Float16 s = dev::to_half(acc[r][i]);
          if (!p.prescale) s = dev::to_half((float)s * p.scale);
          Ss[i * T + j] = s;
        }
      }
    }
  }
  __syncthreads();

  // the v tiles (8 channels x 8 tokens), loaded under the softmax
  const uint32_t vcols = Dv / 8u, vtiles = vcols * (T / 8u);
  h8 vraw[VR][8];
#pragma unroll
  for (uint32_t r = 0; r < VR; ++r) {
    const uint32_t e = min(tid + r * NT, vtiles - 1u);
    const uint32_t tg = e / vcols, c = ch0 + 2u * DK + (e - tg * vcols) * 8u;
    const _Float16* src = p.x + (int64_t)(c >> 4) * p.xs1 + (c & 15u) + (int64_t)tg * 128;
#pragma unroll
    for (int u = 0; u < 8; ++u) vraw[r][u] = *reinterpret_cast<const h8*>(src + u * 16);
  }

  // 3. softmax of the wave's rows, in place
  {
    const uint32_t i = wave * RW + lane / G, g = lane % G, chunks = T / 8u;
    const bool live = i0 + i < T;
    h8 raw[KPT], out[KPT];
    bool have[KPT];
#pragma unroll
    for (int k = 0; k < KPT; ++k) {
      const uint32_t c = g + G * k;
      have[k] = live && c < chunks;
      if (have[k]) raw[k] = *reinterpret_cast<const h8*>(&Ss[i * T + 8u * c]);
    }
    dev::softmax_row_h8<G, KPT>(raw, have, out);
#pragma unroll
    for (int k = 0; k < KPT; ++k)
      if (have[k]) *reinterpret_cast<h8*>(&Ss[i * T + 8u * (g + G * k)]) = out[k];
  }

  // the v tiles, transposed to Vt[tg][c] = v[c][8 tg .. 8 tg + 7], into LDS
#pragma unroll
  for (uint32_t r = 0; r < VR; ++r) {
    const uint32_t e = tid + r * NT;
    if (e < vtiles) {
      const uint32_t tg = e / vcols, c = (e - tg * vcols) * 8u;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        h8 o;
#pragma unroll
        for (int u = 0; u < 8; ++u) o[u] = vraw[r][u][k];
        Vt[tg * vpitch + c + k] = o;
      }
    }
  }
  __syncthreads();

  // 4. mixed values: the sequential chain over the tokens.  v and p are read
  //    from LDS PF steps at a time, the next chunk while the current one is
  //    consumed.
  float acc[CG][RW];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg)
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) acc[cg][rr] = 0.f;
  uint32_t cl[CG];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) cl[cg] = min(lane + 64u * cg, Dv - 1u);
  const _Float16* prow = Ss + wave * RW * T;
  const uint32_t steps = T / 8u;
  struct Chunk {
    h8 v[PF][CG], p[PF][RW];
  };
  auto load = [&](Chunk& ch, uint32_t tg0) {
#pragma unroll
    for (uint32_t s = 0; s < PF; ++s) {
      const uint32_t tg = min(tg0 + s, steps - 1u);  // steps past the end re-read the last (not consumed)
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) ch.v[s][cg] = Vt[tg * vpitch + cl[cg]];
#pragma unroll
      for (int rr = 0; rr < RW; ++rr) ch.p[s][rr] = *reinterpret_cast<const h8*>(prow + rr * T + 8u * tg);
    }
  };
  auto consume = [&](const Chunk& ch, uint32_t count) {
#pragma unroll
    for (uint32_t s = 0; s < PF; ++s) {
      if (s < count) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
          for (int rr = 0; rr < RW; ++rr)
#pragma unroll
            for (int cg = 0; cg < CG; ++cg)
              acc[cg][rr] = __builtin_fmaf((float)ch.v[s][cg][u], (float)ch.p[s][rr][u], acc[cg][rr]);
      }
    }
  };
  Chunk ca, cb;
  load(ca, 0);
  for (uint32_t tg0 = 0;;) {
    if (tg0 + PF >= steps) {
      consume(ca, steps - tg0);
      break;
    }
    load(cb, tg0 + PF);
    consume(ca, PF);
    tg0 += PF;
    if (tg0 + PF >= steps) {
      consume(cb, steps - tg0);
      break;
    }
    load(ca, tg0 + PF);
    consume(cb, PF);
    tg0 += PF;
  }
#pragma unroll
  for (int rr = 0; rr < RW; ++rr) {
    const uint32_t t = i0 + wave * RW + rr;
    if (t >= T) continue;
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
      const uint32_t c = lane + 64u * cg;
      if (c < Dv) {
        const uint32_t oc = h * Dv + c;
        p.y[(int64_t)(oc >> 4) * p.ys1 + (int64_t)t * 16 + (oc & 15u)] = dev::to_half(acc[cg][rr]);
      }
    }
  }
}

template <int DK, int G, int KPT>
void launch_cg(const AttnPlan& p, uint32_t lds, hipStream_t stream) {
  if (p.Dv <= 64)
    hipLaunchKernelGGL((attention_kernel<DK, G, KPT, 1>), dim3(p.grid), dim3(kAttnRows * G), lds, stream, p);
  else
    hipLaunchKernelGGL((attention_kernel<DK, G, KPT, 2>), dim3(p.grid), dim3(kAttnRows * G), lds, stream, p);
}

template <int DK>
void launch_tree(const AttnPlan& p, RowTree tree, uint32_t lds, hipStream_t stream) {
  if (tree.lanes == 64) launch_cg<DK, 64, 1>(p, lds, stream);
  else if (tree.lanes == 32) launch_cg<DK, 32, 2>(p, lds, stream);
  else launch_cg<DK, 16, 2>(p, lds, stream);
}

}  // namespace
}  // namespace thin

using namespace thin;

extern "C" thin_status thin_attention(const thin_desc* qkv, int64_t heads, int64_t key_dim, int64_t head_dim,
                                      float scale, int32_t prescale, const thin_desc* out, hipStream_t stream) {
  clear_error();
  THIN_REQUIRE(qkv && out && desc_valid(qkv) && desc_valid(out), THIN_ERR_INVALID, "attention: invalid descriptor");
  THIN_REQUIRE(qkv->dtype == THIN_F16 && qkv->rank == 4 && qkv->sizes[0] == 1 && qkv->sizes[3] == 16,
               THIN_ERR_INVALID, "attention: qkv must be an N=1 FP16 blocked tensor [1, C1, T, 16]");
  const int64_t channels = qkv->sizes[1] * 16, T = qkv->sizes[2];
  THIN_REQUIRE(heads > 0 && channels % heads == 0 && key_dim > 0 && head_dim > 0 &&
                   2 * key_dim + head_dim <= channels / heads && heads * head_dim % 16 == 0,
               THIN_ERR_INVALID, "attention: %lld heads of %lld + %lld + %lld channels do not fit %lld channels",
               (long long)heads, (long long)key_dim, (long long)key_dim, (long long)head_dim, (long long)channels);
  THIN_REQUIRE(out->dtype == THIN_F16 && out->rank == 4 && out->sizes[0] == 1 &&
                   out->sizes[1] == heads * head_dim / 16 && out->sizes[2] == T && out->sizes[3] == 16,
               THIN_ERR_INVALID, "attention: out must be [1, %lld, %lld, 16] float16",
               (long long)(heads * head_dim / 16), (long long)T);
  // what the fused kernel covers; other shapes run the op chain
  const int64_t group = channels / heads;
  const RowTree tree = row_tree(T / 8, (uint64_t)(heads * T));
  THIN_REQUIRE(qkv->strides[3] == 1 && qkv->strides[2] == 16 && qkv->strides[1] % 8 == 0 &&
                   reinterpret_cast<uintptr_t>(qkv->data) % 16 == 0 && out->strides[3] == 1 &&
                   out->strides[2] == 16,
               THIN_ERR_UNSUPPORTED, "attention: qkv and out need packed 16-channel blocks (16-byte aligned qkv)");
  THIN_REQUIRE((key_dim == 16 || key_dim == 32 || key_dim == 64) && head_dim % 16 == 0 && head_dim <= 128 &&
                   group % 16 == 0,
               THIN_ERR_UNSUPPORTED, "attention: key_dim must be 16, 32 or 64 and head_dim a multiple of 16 up to 128");
  THIN_REQUIRE(T % 8 == 0 && T > 128 && T <= kAttnMaxTokens && (tree.lanes == 64 || tree.lanes == 32 ||
                                                                  tree.lanes == 16),
               THIN_ERR_UNSUPPORTED, "attention: tokens must be a multiple of 8 in (128, %u]", kAttnMaxTokens);
  const uint32_t bi = kAttnRows;
  const uint32_t q_bytes = bi * (uint32_t)key_dim * 2u, s_bytes = bi * (uint32_t)T * 2u;
  const uint32_t v_bytes = (uint32_t)(T / 8 * (head_dim + 1) * 16);
  const uint32_t lds = q_bytes + s_bytes + v_bytes;  // each part a multiple of 16 bytes
  THIN_REQUIRE(lds <= kAttnMaxLds && (uint64_t)(head_dim / 8) * (T / 8) <= kAttnVTiles,
               THIN_ERR_UNSUPPORTED, "attention: %lld tokens x %lld value channels exceed the fused kernel's LDS",
               (long long)T, (long long)head_dim);
  THIN_REQUIRE(qkv->strides[1] < ((int64_t)1 << 31) && out->strides[1] < ((int64_t)1 << 31),
               THIN_ERR_UNSUPPORTED, "attention: tensor too large");

  AttnPlan p;
  memset(&p, 0, sizeof p);
  p.x = static_cast<const _Float16*>(qkv->data);
  p.y = static_cast<_Float16*>(out->data);
  p.xs1 = qkv->strides[1];
  p.ys1 = out->strides[1];
  p.T = (uint32_t)T;
  p.Dv = (uint32_t)head_dim;
  p.group = (uint32_t)group;
  p.row_blocks = ((uint32_t)T + bi - 1) / bi;
  p.grid = (uint32_t)heads * p.row_blocks;
  p.scale = scale;
  p.prescale = prescale ? 1u : 0u;
  p.s_off = q_bytes;
  p.v_off = q_bytes + s_bytes;
  THIN_REQUIRE(heads * (int64_t)p.row_blocks < ((int64_t)1 << 31), THIN_ERR_UNSUPPORTED, "attention: too many heads");
  if (key_dim == 16) launch_tree<16>(p, tree, lds, stream);
  else if (key_dim == 32) launch_tree<32>(p, tree, lds, stream);
  else launch_tree<64>(p, tree, lds, stream);
  THIN_LAUNCH_CHECK("attention_kernel");
  return THIN_OK;
}
