// Device helpers of the router shared by the standalone router kernels and the fused
// decode front end: wave-wide reductions and the top-k of one logits row.
#pragma once

#include <math.h>

#include "common.h"

namespace mxmoe {

constexpr int kMaxEPerLane = 16;  // E <= 1024

// Wave-wide reductions through DPP lane moves (VALU latency, no LDS crossbar): within
// each row of 16 lanes quad swaps, half-row and row mirrors; then row_bcast15/31 fold
// rows 0..3 into lane 63, whose value is read into a scalar register (every lane gets
// the same result).  Lanes a move has no source for keep the identity.
#define MXMOE_DPP_STEP(T, OP, V, IDENT, CTRL, ROWS)                                            \
  V = OP(V, __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, IDENT), \
                                                              __builtin_bit_cast(int, V),     \
                                                              CTRL, ROWS, 0xf, false)))
#define MXMOE_WAVE_REDUCE(T, OP, V, IDENT)                                                   \
  do {                                                                                   \
    MXMOE_DPP_STEP(T, OP, V, IDENT, 0xB1, 0xf);  /* quad_perm [1,0,3,2] */              \
    MXMOE_DPP_STEP(T, OP, V, IDENT, 0x4E, 0xf);  /* quad_perm [2,3,0,1] */              \
    MXMOE_DPP_STEP(T, OP, V, IDENT, 0x141, 0xf); /* row_half_mirror */                   \
    MXMOE_DPP_STEP(T, OP, V, IDENT, 0x140, 0xf); /* row_mirror */                        \
    MXMOE_DPP_STEP(T, OP, V, IDENT, 0x142, 0xa); /* row_bcast15 into rows 1, 3 */        \
    MXMOE_DPP_STEP(T, OP, V, IDENT, 0x143, 0xc); /* row_bcast31 into rows 2, 3 */        \
  } while (0)

__device__ __forceinline__ float fmax_op(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ float fadd_op(float a, float b) { return a + b; }

__device__ __forceinline__ float wave_max(float v) {
  MXMOE_WAVE_REDUCE(float, fmax_op, v, -INFINITY);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_sum(float v) {
  MXMOE_WAVE_REDUCE(float, fadd_op, v, 0.0f);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// The same reductions over each row of 16 lanes (the first four DPP moves): every
// lane of a row ends with its row's result.
#define MXMOE_ROW_REDUCE(T, OP, V, IDENT)                                                    \
  do {                                                                                   \
    MXMOE_DPP_STEP(T, OP, V, IDENT, 0xB1, 0xf);                                          \
    MXMOE_DPP_STEP(T, OP, V, IDENT, 0x4E, 0xf);                                          \
    MXMOE_DPP_STEP(T, OP, V, IDENT, 0x141, 0xf);                                         \
    MXMOE_DPP_STEP(T, OP, V, IDENT, 0x140, 0xf);                                         \
  } while (0)

__device__ __forceinline__ float row16_max(float v) {
  MXMOE_ROW_REDUCE(float, fmax_op, v, -INFINITY);
  return v;
}

__device__ __forceinline__ float row16_sum(float v) {
  MXMOE_ROW_REDUCE(float, fadd_op, v, 0.0f);
  return v;
}

// Reductions over a group of W lanes (the wave, or a row of 16).
template <int W>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (W == 64) return wave_max(v);
  else return row16_max(v);
}
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (W == 64) return wave_sum(v);
  else return row16_sum(v);
}

// Max of 64-bit keys over a group of W lanes (row moves, then for W = 64 the row
// broadcasts and lane 63); lanes a move has no source for keep key 0.
template <int W>
__device__ __forceinline__ uint64_t group_max_key(uint64_t v) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
#define MXMOE_KEY_STEP(CTRL, ROWS)                                                        \
  {                                                                                       \
    const uint32_t l2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, CTRL, ROWS, 0xf, false); \
    const uint32_t h2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, CTRL, ROWS, 0xf, false); \
    const uint64_t a = ((uint64_t)hi << 32) | lo, b = ((uint64_t)h2 << 32) | l2;            \
    const uint64_t m = b > a ? b : a;                                                     \
    lo = (uint32_t)m;                                                                     \
    hi = (uint32_t)(m >> 32);                                                             \
  }
  MXMOE_KEY_STEP(0xB1, 0xf)
  MXMOE_KEY_STEP(0x4E, 0xf)
  MXMOE_KEY_STEP(0x141, 0xf)
  MXMOE_KEY_STEP(0x140, 0xf)
  if constexpr (W == 64) {
    MXMOE_KEY_STEP(0x142, 0xa)
    MXMOE_KEY_STEP(0x143, 0xc)
    lo = (uint32_t)__builtin_amdgcn_readlane((int)lo, 63);
    hi = (uint32_t)__builtin_amdgcn_readlane((int)hi, 63);
  }
#undef MXMOE_KEY_STEP
  return ((uint64_t)hi << 32) | lo;
}

// Selection key of (score, expert e): the score's bits mapped to an unsigned order
// (larger score, larger key; -0 counts as +0) in the high word and ~e in the low word,
// so the largest key is the largest score with the lowest expert id.  NaN scores and
// experts past E get key 0 and are never selected.
__device__ __forceinline__ uint64_t topk_key(float v, int e, int E) {
  const uint32_t b = __float_as_uint(v + 0.0f);
  const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  const uint64_t k = ((uint64_t)o << 32) | (uint32_t)~e;
  return (e < E && !(v != v)) ? k : 0ull;
}

__device__ __forceinline__ float topk_key_value(uint64_t k) {
  const uint32_t o = (uint32_t)(k >> 32);
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

// A row of E <= 64*PER logits into one wave: lane l holds experts l, l+64, ...
template <int PER>
__device__ __forceinline__ void load_row_wave(const float* __restrict__ row, int E,
                                              float (&v)[PER]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? row[e] : -INFINITY;
  }
}

// Top-k of one row (as load_row_wave holds it) by one wave, router.py:383-565
// semantics: act_first = 0: top-k on the logits (descending, equal values -> lower
// expert id), then the activation over the k selected values; act_first = 1: the
// activation over all E logits, then top-k.  renorm divides the k values by (their
// sum + eps).  rnd (a Dt) is the precision of the reference's computation dtype: every
// activation output, the renorm sum and quotient are rounded to it, as the torch ops of
// router.py:383-503 round each result of a half-precision tensor op (fp32 arithmetic,
// one rounding per op).  Every lane returns the same sel_idx[0..K) and out[0..K).
// topk_row_group<W, PER> does the same for a group of W lanes (W = 64: the wave; W = 16:
// a row of 16 lanes, lane j of the row holding experts j, j+16, ...).
template <int W, int PER>
__device__ __forceinline__ void topk_row_group(const float (&vals)[PER], int E, int K, int act,
                                               int act_first, int renorm, float renorm_eps,
                                               int rnd, int (&sel_idx)[8], float (&out)[8]) {
  const int lane = threadIdx.x & (W - 1);
  float score[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) score[i] = vals[i];
  if (act_first) {
    if (act == MXMOE_ROUTER_SOFTMAX) {
      float m = score[0];
#pragma unroll
      for (int i = 1; i < PER; ++i) m = fmaxf(m, score[i]);
      m = group_max<W>(m);
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        score[i] = lane + W * i < E ? expf(score[i] - m) : 0.f;
        s += score[i];
      }
      s = group_sum<W>(s);
#pragma unroll
      for (int i = 0; i < PER; ++i)
        score[i] = lane + W * i < E ? round_to(score[i] / s, rnd) : -INFINITY;
    } else {
#pragma unroll
      for (int i = 0; i < PER; ++i)
        score[i] = lane + W * i < E ? round_to(sigmoid_f32(score[i]), rnd) : -INFINITY;
    }
  }
  // k rounds of arg-max over the selection keys (descending score, equal scores ->
  // lower expert id); selected keys are knocked out.  With no candidate left a round
  // yields index 0x7fffffff and value -inf.
  uint64_t key[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) key[i] = topk_key(score[i], lane + W * i, E);
  float sel_val[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    sel_idx[k] = 0;
    sel_val[k] = 0.f;
    if (k >= K) continue;
    uint64_t best = key[0];
#pragma unroll
    for (int i = 1; i < PER; ++i) best = key[i] > best ? key[i] : best;
    best = group_max_key<W>(best);
    sel_idx[k] = best ? (int)~(uint32_t)best : 0x7fffffff;
    sel_val[k] = best ? topk_key_value(best) : -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; ++i) key[i] = key[i] == best ? 0ull : key[i];
  }
  // Activation over the selected values unless it came first, then optional renorm.
#pragma unroll
  for (int k = 0; k < 8; ++k) out[k] = sel_val[k];
  if (!act_first) {
    if (act == MXMOE_ROUTER_SOFTMAX) {
      const float m = sel_val[0];
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k < K) {
          out[k] = expf(sel_val[k] - m);
          s += out[k];
        }
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k < K) out[k] = round_to(out[k] / s, rnd);
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k < K) out[k] = round_to(sigmoid_f32(sel_val[k]), rnd);
    }
  }
  if (renorm) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < K) s += out[k];
    s = round_to(s, rnd) + renorm_eps;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < K) out[k] = round_to(out[k] / s, rnd);
  }
}

template <int PER>
__device__ __forceinline__ void topk_row_wave(const float (&vals)[PER], int E, int K, int act,
                                              int act_first, int renorm, float renorm_eps,
                                              int rnd, int (&sel_idx)[8], float (&out)[8]) {
  topk_row_group<64, PER>(vals, E, K, act, act_first, renorm, renorm_eps, rnd, sel_idx, out);
}

// Values per lane for E experts: the template argument of topk_row_wave.
inline int topk_per_lane(int E) {
  const int per = (E + 63) / 64;
  return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : 16;
}

// Lane k < K of the wave writes the k-th selection of a row.
__device__ __forceinline__ void store_topk_wave(const int (&sel_idx)[8], const float (&out)[8],
                                                int K, int32_t* __restrict__ idx_row,
                                                float* __restrict__ val_row) {
  const int lane = threadIdx.x & 63;
  if (lane < K) {
    int si = 0;
    float so = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k == lane) {
        si = sel_idx[k];
        so = out[k];
      }
    idx_row[lane] = si;
    val_row[lane] = so;
  }
}


// One wave's share of router logits (router_logits_kernel and the fused prefill router):
// acc[e][t] = sum over the wave's 128-wide K chunks c = kw, kw + NW, kw + 2 NW, ... (in
// that order, four MFMA steps each) of expert rows e0 + 16 e + (lane % 16) (A operand)
// times token rows t0 + 16 t + (lane % 16) (B operand); rows past E or T re-read the last
// one.  Summing the NW waves' results in wave order gives the logits, with the same
// arithmetic whatever the tile shape TT x ET.  Operand modes as router_logits_kernel.
template <int TT, int ET, int NW, bool XF16, bool WF16, int OP>
__device__ __forceinline__ void router_partial_logits(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w, int T,
                                                      int H, int E, int t0, int e0, int kw,
                                                      f32x4 (&acc)[ET][TT]) {
  const int nc = (H + 127) / 128;
  const int tail_q = (H % 128) / 32;  // blocks of 32 in a partial last chunk

  const int lane = threadIdx.x & 63, q = lane >> 4, r16 = lane & 15;
  const uint16_t* xr[TT];
  const uint16_t* wr[ET];
#pragma unroll
  for (int t = 0; t < TT; ++t) xr[t] = x + (size_t)min(t0 + 16 * t + r16, T - 1) * H;
#pragma unroll
  for (int e = 0; e < ET; ++e) wr[e] = w + (size_t)min(e0 + 16 * e + r16, E - 1) * H;

#pragma unroll
  for (int e = 0; e < ET; ++e)
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[e][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  // Chunk c's operands (lanes past K in a partial last chunk feed zeros; every lane runs
  // the MFMAs), loaded one chunk ahead of their MFMAs into the other register set.
  auto load = [&](int c, u32x4 (&xv)[TT][4], u32x4 (&wv)[ET][4]) {
    const bool ok = (c < H / 128) || (q < tail_q);
    const int k0 = c * 128 + q * 32;
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        xv[t][j] = ok ? *reinterpret_cast<const u32x4*>(xr[t] + k0 + 8 * j) : zero4;
#pragma unroll
    for (int e = 0; e < ET; ++e)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        wv[e][j] = ok ? *reinterpret_cast<const u32x4*>(wr[e] + k0 + 8 * j) : zero4;
  };
  auto mma = [&](const u32x4 (&xv)[TT][4], const u32x4 (&wv)[ET][4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < ET; ++e) {
        if constexpr (OP == kOpF16) {
          f16x8 a;
          if constexpr (WF16) a = __builtin_bit_cast(f16x8, wv[e][j]);
          else a = bf16x8_to_f16x8(wv[e][j]);
#pragma unroll
          for (int t = 0; t < TT; ++t) {
            f16x8 b;
            if constexpr (XF16) b = __builtin_bit_cast(f16x8, xv[t][j]);
            else b = bf16x8_to_f16x8(xv[t][j]);
            acc[e][t] = mfma16_f16(a, b, acc[e][t]);
          }
        } else if constexpr (OP == kOpExact) {
          static_assert(WF16 && !XF16, "exact mode splits fp16 weights against bf16 x");
          bf16x8 hi, lo;
          f16x8_split_bf16(wv[e][j], hi, lo);
#pragma unroll
          for (int t = 0; t < TT; ++t) {
            acc[e][t] = mfma16(hi, as_bf16x8(xv[t][j]), acc[e][t]);
            acc[e][t] = mfma16(lo, as_bf16x8(xv[t][j]), acc[e][t]);
          }
        } else {
          static_assert(!XF16, "bf16 MFMA takes bf16 x");
          bf16x8 a;
          if constexpr (WF16) a = f16x8_to_bf16x8(wv[e][j]);
          else a = as_bf16x8(wv[e][j]);
#pragma unroll
          for (int t = 0; t < TT; ++t) acc[e][t] = mfma16(a, as_bf16x8(xv[t][j]), acc[e][t]);
        }
      }
  };
  u32x4 xa[TT][4], wa[ET][4], xb[TT][4], wb[ET][4];
  int c = kw;
  if (c < nc) load(c, xa, wa);
  for (; c < nc; c += 2 * NW) {
    const int c1 = c + NW;
    if (c1 < nc) load(c1, xb, wb);
    mma(xa, wa);
    if (c1 >= nc) break;
    if (c1 + NW < nc) load(c1 + NW, xa, wa);
    mma(xb, wb);
  }
}

}  // namespace mxmoe
