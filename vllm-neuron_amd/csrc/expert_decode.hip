// Decode (token generation) expert MLP: weight-streaming grouped GEMMs over the
// experts the batch selected, fp32 arithmetic as in the reference decode flow.
//
//   route      one workgroup: per-expert slot lists (tokens ascending inside an
//              expert), the list of active experts, per-token slots sorted by expert
//   gate_up    grid (I/16 column pairs, active experts); a workgroup streams one
//              16-row gate group and the matching 16-row up group over all of K,
//              its 4 waves splitting K chunks; fused bias, clamps, activation;
//              the fp32 activation is stored as a bf16 hi/lo pair
//   down       grid (H/32, active experts); two MFMAs (hi, lo) per product
//   combine    out[t] = bf16(sum over the token's experts in ascending id of y * w)
#include <math.h>

#include "capi_util.h"
#include "common.h"

namespace mxmoe {

constexpr int kTkgMaxT = 1024;
constexpr int kTkgMaxE = 512;

__global__ void __launch_bounds__(1024) tkg_route_kernel(
    const int32_t* __restrict__ topk_idx, const float* __restrict__ topk_val, int T, int K, int E,
    int scale_mode, int32_t* __restrict__ expert_off, int32_t* __restrict__ active,
    int32_t* __restrict__ n_active, int32_t* __restrict__ slot_tok, int32_t* __restrict__ tok_slot,
    float* __restrict__ tok_w) {
  __shared__ unsigned long long masks[16][kTkgMaxE];
  __shared__ int off[kTkgMaxE];
  __shared__ int wsum[16], wact[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < 16 * kTkgMaxE; i += 1024) (&masks[0][0])[i] = 0ull;
  __syncthreads();
  int ids[8];
  float vals[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    ids[k] = -1;
    vals[k] = 0.f;
  }
  if (tid < T) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k >= K) break;
      int e = topk_idx[(size_t)tid * K + k];
      if (e < 0 || e >= E) e = -1;
      // A repeated expert id counts once (its last value, as a scatter would keep).
      for (int j = 0; j < k; ++j)
        if (ids[j] == e) ids[j] = -1;
      ids[k] = e;
      vals[k] = topk_val[(size_t)tid * K + k];
      if (e >= 0) atomicOr(&masks[wave][e], 1ull << lane);
    }
  }
  __syncthreads();
  // Counts -> exclusive offsets and the active-expert list (ascending id).
  int cnt = 0;
  if (tid < E)
    for (int w = 0; w < 16; ++w) cnt += __popcll(masks[w][tid]);
  int v = cnt, a = cnt > 0 ? 1 : 0;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int pv = __shfl_up(v, o), pa = __shfl_up(a, o);
    if (lane >= o) {
      v += pv;
      a += pa;
    }
  }
  if (lane == 63) {
    wsum[wave] = v;
    wact[wave] = a;
  }
  __syncthreads();
  int pv = 0, pa = 0;
  for (int w = 0; w < wave; ++w) {
    pv += wsum[w];
    pa += wact[w];
  }
  v += pv;
  a += pa;
  if (tid < E) {
    off[tid] = v - cnt;
    expert_off[tid] = v - cnt;
    if (cnt > 0) active[a - 1] = tid;
  }
  if (tid == E - 1) {
    expert_off[E] = v;
    *n_active = a;
  }
  __syncthreads();
  if (tid >= T) return;
  const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int es[8], ss[8];
  float ws[8];
  int n = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k >= K) break;
    const int e = ids[k];
    if (e < 0) continue;
    int r = off[e];
    for (int w = 0; w < wave; ++w) r += __popcll(masks[w][e]);
    r += __popcll(masks[wave][e] & below);
    slot_tok[r] = tid;
    // insertion into the expert-ascending list
    int p = n;
    while (p > 0 && es[p - 1] > e) {
      es[p] = es[p - 1];
      ss[p] = ss[p - 1];
      ws[p] = ws[p - 1];
      --p;
    }
    es[p] = e;
    ss[p] = r;
    ws[p] = (scale_mode == MXMOE_SCALE_NO) ? (vals[k] > 0.f ? 1.f : 0.f) : vals[k];
    ++n;
  }
  for (int k = 0; k < K; ++k) {
    tok_slot[(size_t)tid * K + k] = k < n ? ss[k] : -1;
    tok_w[(size_t)tid * K + k] = k < n ? ws[k] : 0.f;
  }
}

__device__ __forceinline__ float clampf_ref(float v, float lo, float hi) {
  // torch.clamp semantics: NaN stays NaN.
  v = (v > hi) ? hi : v;
  v = (v < lo) ? lo : v;
  return v;
}

__device__ __forceinline__ float act_f32(float g, int act) {
  if (act == kSwish) return g * sigmoid_f32(g * 1.702f);
  if (act == kSiLU) return g / (1.0f + expf(-g));
  return 0.5f * g * (1.0f + erff(g * 0.70710678118654752f));
}

// One wave's share of a streamed GEMM tile: R row groups (A = weights) times NT
// token tiles (B = activations) over chunks c = c0, c0 + cs, ...
// brow[t] points at this lane's activation row of token tile t (bf16, length K),
// or is null for a token past the expert's list.  With SPLIT the activations come
// as (hi, lo) pairs: brow2 points at the lo rows.
template <int R, int NT, bool SPLIT>
__device__ __forceinline__ void stream_wave(const uint8_t* __restrict__ wq,
                                            const uint8_t* __restrict__ ws, size_t rg_bytes,
                                            size_t rg_sbytes, const uint16_t* const* brow,
                                            const uint16_t* const* brow2, int ntv, int K, int c0,
                                            int cs, f32x4 (&acc)[R][NT]) {
  const int lane = threadIdx.x & 63, q = lane >> 4;
  const int nc = (K + 127) / 128, nfull = K / 128, tail_q = (K % 128) / 32;
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  for (int c = c0; c < nc; c += cs) {
    const bool ok = (c < nfull) || (q < tail_q);
    u32x4 wv[R];
    uint32_t sv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      wv[r] = ok ? *reinterpret_cast<const u32x4*>(wq + r * rg_bytes + (size_t)c * 1024 + lane * 16)
                 : zero4;
      sv[r] = ok ? (uint32_t)ws[r * rg_sbytes + (size_t)c * 64 + lane] : 0u;
    }
    const int k0 = c * 128 + q * 32;
    u32x4 bv[NT][4], bv2[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bool tv = ok && brow[t] != nullptr;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bv[t][j] = tv ? *reinterpret_cast<const u32x4*>(brow[t] + k0 + 8 * j) : zero4;
        if (SPLIT) bv2[t][j] = tv ? *reinterpret_cast<const u32x4*>(brow2[t] + k0 + 8 * j) : zero4;
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float sc = e8m0_to_f32(sv[r]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bf16x8 wf = dequant8(wv[r][j], sc);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          if (t < ntv) {  // wave-uniform
            acc[r][t] = mfma16(wf, as_bf16x8(bv[t][j]), acc[r][t]);
            if (SPLIT) acc[r][t] = mfma16(wf, as_bf16x8(bv2[t][j]), acc[r][t]);
          }
        }
      }
    }
  }
}

template <int NT>
__global__ void __launch_bounds__(256) tkg_gate_up_kernel(
    const uint16_t* __restrict__ x, int H, int I, const uint8_t* __restrict__ gu_q,
    const uint8_t* __restrict__ gu_s, const uint16_t* __restrict__ gu_bias,
    const int32_t* __restrict__ expert_off, const int32_t* __restrict__ active,
    const int32_t* __restrict__ n_active, const int32_t* __restrict__ slot_tok, ExpertParams p,
    uint16_t* __restrict__ h_hi, uint16_t* __restrict__ h_lo) {
  __shared__ f32x4 red[4][2][NT][64];
  if ((int)blockIdx.y >= *n_active) return;
  const int e = active[blockIdx.y];
  const int s0 = expert_off[e], ne = expert_off[e + 1] - s0;
  const int pair = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const size_t rg_bytes = (size_t)H * 8, rg_sbytes = (size_t)H / 2;
  const size_t n_rg = (size_t)(2 * I) / 16;
  const uint8_t* wq = gu_q + ((size_t)e * n_rg + 2 * pair) * rg_bytes;
  const uint8_t* ws = gu_s + ((size_t)e * n_rg + 2 * pair) * rg_sbytes;
  for (int tb = 0; tb < ne; tb += 16 * NT) {
    const int ntv = min(NT, (ne - tb + 15) / 16);
    const uint16_t* brow[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int li = tb + 16 * t + (lane & 15);
      brow[t] = (li < ne) ? x + (size_t)slot_tok[s0 + li] * H : nullptr;
    }
    f32x4 acc[2][NT];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    stream_wave<2, NT, false>(wq, ws, rg_bytes, rg_sbytes, brow, brow, ntv, H, wave, 4, acc);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int t = 0; t < NT; ++t) red[wave][r][t][lane] = acc[r][t];
    __syncthreads();
    for (int t = wave; t < ntv; t += 4) {
      f32x4 g = red[0][0][t][lane], u = red[0][1][t][lane];
#pragma unroll
      for (int v = 1; v < 4; ++v) {
        g += red[v][0][t][lane];
        u += red[v][1][t][lane];
      }
      const int li = tb + 16 * t + (lane & 15);
      if (li >= ne) continue;
      const int col0 = 16 * pair + 4 * (lane >> 4);
      const size_t slot = (size_t)(s0 + li);
      uint16_t hi[4], lo[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float gv = g[i], uv = u[i];
        if (gu_bias) {
          gv += bf16_bits_to_f32(gu_bias[(size_t)e * 2 * I + col0 + i]);
          uv += bf16_bits_to_f32(gu_bias[(size_t)e * 2 * I + I + col0 + i]);
        }
        gv = clampf_ref(gv, p.gate_lo, p.gate_hi);
        uv = clampf_ref(uv, p.up_lo, p.up_hi);
        const float h = uv * act_f32(gv, p.act);
        split_bf16(h, hi[i], lo[i]);
      }
      typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
      *reinterpret_cast<u16x4*>(h_hi + slot * I + col0) = u16x4{hi[0], hi[1], hi[2], hi[3]};
      *reinterpret_cast<u16x4*>(h_lo + slot * I + col0) = u16x4{lo[0], lo[1], lo[2], lo[3]};
    }
    __syncthreads();
  }
}

template <int NT>
__global__ void __launch_bounds__(256) tkg_down_kernel(
    const uint16_t* __restrict__ h_hi, const uint16_t* __restrict__ h_lo, int H, int I,
    const uint8_t* __restrict__ dn_q, const uint8_t* __restrict__ dn_s,
    const uint16_t* __restrict__ dn_bias, const int32_t* __restrict__ expert_off,
    const int32_t* __restrict__ active, const int32_t* __restrict__ n_active,
    float* __restrict__ y) {
  __shared__ f32x4 red[4][2][NT][64];
  if ((int)blockIdx.y >= *n_active) return;
  const int e = active[blockIdx.y];
  const int s0 = expert_off[e], ne = expert_off[e + 1] - s0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const size_t rg_bytes = (size_t)I * 8, rg_sbytes = (size_t)I / 2;
  const size_t n_rg = (size_t)H / 16;
  const int rg0 = 2 * blockIdx.x;
  const uint8_t* wq = dn_q + ((size_t)e * n_rg + rg0) * rg_bytes;
  const uint8_t* ws = dn_s + ((size_t)e * n_rg + rg0) * rg_sbytes;
  for (int tb = 0; tb < ne; tb += 16 * NT) {
    const int ntv = min(NT, (ne - tb + 15) / 16);
    const uint16_t* b1[NT];
    const uint16_t* b2[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int li = tb + 16 * t + (lane & 15);
      b1[t] = (li < ne) ? h_hi + (size_t)(s0 + li) * I : nullptr;
      b2[t] = (li < ne) ? h_lo + (size_t)(s0 + li) * I : nullptr;
    }
    f32x4 acc[2][NT];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    stream_wave<2, NT, true>(wq, ws, rg_bytes, rg_sbytes, b1, b2, ntv, I, wave, 4, acc);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int t = 0; t < NT; ++t) red[wave][r][t][lane] = acc[r][t];
    __syncthreads();
    for (int idx = wave; idx < 2 * ntv; idx += 4) {
      const int r = idx & 1, t = idx >> 1;
      f32x4 s = red[0][r][t][lane];
#pragma unroll
      for (int v = 1; v < 4; ++v) s += red[v][r][t][lane];
      const int li = tb + 16 * t + (lane & 15);
      if (li >= ne) continue;
      const int n0 = 16 * (rg0 + r) + 4 * (lane >> 4);
      if (dn_bias) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] += bf16_bits_to_f32(dn_bias[(size_t)e * H + n0 + i]);
      }
      *reinterpret_cast<f32x4*>(y + (size_t)(s0 + li) * H + n0) = s;
    }
    __syncthreads();
  }
}

// out[t, n] = bf16(sum_k y[slot(t, k), n] * w(t, k)), k in ascending expert order.
__global__ void __launch_bounds__(256) tkg_combine_kernel(const float* __restrict__ y,
                                                          const int32_t* __restrict__ tok_slot,
                                                          const float* __restrict__ tok_w, int H,
                                                          int K, uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int n = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (n >= H) return;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < K; ++k) {
    const int s = tok_slot[(size_t)t * K + k];
    if (s < 0) continue;
    const float w = tok_w[(size_t)t * K + k];
    const f32x4 v = *reinterpret_cast<const f32x4*>(y + (size_t)s * H + n);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = __fadd_rn(acc[i], __fmul_rn(v[i], w));
  }
  typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
  *reinterpret_cast<u16x4*>(out + (size_t)t * H + n) =
      u16x4{f32_to_bf16_bits(acc[0]), f32_to_bf16_bits(acc[1]), f32_to_bf16_bits(acc[2]),
            f32_to_bf16_bits(acc[3])};
}

struct TkgWs {
  int32_t *expert_off, *active, *n_active, *slot_tok, *tok_slot;
  float* tok_w;
  uint16_t *h_hi, *h_lo;
  float* y;
};

static size_t tkg_carve(void* base, size_t cap, int64_t T, int64_t H, int64_t I, int64_t E,
                        int K, TkgWs* w) {
  Carver cv(base, cap);
  const int64_t S = T * K;
  TkgWs t;
  t.expert_off = cv.take<int32_t>(E + 1);
  t.active = cv.take<int32_t>(E);
  t.n_active = cv.take<int32_t>(1);
  t.slot_tok = cv.take<int32_t>(S);
  t.tok_slot = cv.take<int32_t>(S);
  t.tok_w = cv.take<float>(S);
  t.h_hi = cv.take<uint16_t>(S * I);
  t.h_lo = cv.take<uint16_t>(S * I);
  t.y = cv.take<float>(S * H);
  if (w) *w = t;
  return cv.off + 256;
}

}  // namespace mxmoe

using namespace mxmoe;

extern "C" size_t mxmoe_moe_tkg_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                                                int top_k) {
  char* nil = nullptr;
  return tkg_carve(nil, ~(size_t)0, T, H, I, E, top_k, nullptr);
}

extern "C" int mxmoe_moe_tkg(const uint16_t* x, const int32_t* topk_idx, const float* topk_val,
                             const uint8_t* gu_q, const uint8_t* gu_s, const uint8_t* dn_q,
                             const uint8_t* dn_s, const uint16_t* gu_bias,
                             const uint16_t* dn_bias, int64_t T, int64_t H, int64_t I, int64_t E,
                             int top_k, int act, const float* clamps, int scale_mode,
                             uint16_t* out, void* workspace, size_t workspace_bytes,
                             void* const* stage_events, void* stream) {
  clear_error();
  MXMOE_REQUIRE(x && topk_idx && topk_val && gu_q && gu_s && dn_q && dn_s && out && workspace,
                "moe_tkg: null pointer");
  MXMOE_REQUIRE(T >= 1 && T <= kTkgMaxT, "moe_tkg: T=%lld out of range [1, %d]", (long long)T,
                kTkgMaxT);
  MXMOE_REQUIRE(E >= 1 && E <= kTkgMaxE, "moe_tkg: E=%lld out of range [1, %d]", (long long)E,
                kTkgMaxE);
  MXMOE_REQUIRE(H % 32 == 0 && I % 32 == 0 && H >= 32 && I >= 32,
                "moe_tkg: H=%lld and I=%lld must be multiples of 32", (long long)H, (long long)I);
  MXMOE_REQUIRE(top_k >= 1 && top_k <= 8, "moe_tkg: top_k=%d out of range [1, 8]", top_k);
  MXMOE_REQUIRE(act >= 0 && act <= 2, "moe_tkg: unknown activation %d", act);
  MXMOE_REQUIRE(scale_mode == MXMOE_SCALE_POST || scale_mode == MXMOE_SCALE_NO,
                "moe_tkg: unsupported scale mode %d", scale_mode);
  const size_t need = mxmoe_moe_tkg_workspace_bytes(T, H, I, E, top_k);
  if (workspace_bytes < need)
    return set_error(MXMOE_E_WORKSPACE, "moe_tkg: workspace %zu < %zu", workspace_bytes, need);
  TkgWs w;
  tkg_carve(workspace, workspace_bytes, T, H, I, E, top_k, &w);
  ExpertParams p;
  p.gate_lo = clamps ? clamps[0] : -INFINITY;
  p.gate_hi = clamps ? clamps[1] : INFINITY;
  p.up_lo = clamps ? clamps[2] : -INFINITY;
  p.up_hi = clamps ? clamps[3] : INFINITY;
  p.act = act;
  hipStream_t s = as_stream(stream);
  auto mark = [&](int i) {
    if (stage_events) hipEventRecord(reinterpret_cast<hipEvent_t>(stage_events[i]), s);
  };
  mark(0);
  hipLaunchKernelGGL(tkg_route_kernel, dim3(1), dim3(1024), 0, s, topk_idx, topk_val, (int)T,
                     top_k, (int)E, scale_mode, w.expert_off, w.active, w.n_active, w.slot_tok,
                     w.tok_slot, w.tok_w);
  mark(1);
  const int64_t maxne = T;  // an expert sees each token at most once
  const dim3 g1((unsigned)(I / 16), (unsigned)E), g2((unsigned)(H / 32), (unsigned)E);
#define MXMOE_TKG_LAUNCH(NT)                                                                 \
  do {                                                                                       \
    hipLaunchKernelGGL((tkg_gate_up_kernel<NT>), g1, dim3(256), 0, s, x, (int)H, (int)I, gu_q, \
                       gu_s, gu_bias, w.expert_off, w.active, w.n_active, w.slot_tok, p,     \
                       w.h_hi, w.h_lo);                                                      \
    mark(2);                                                                                 \
    hipLaunchKernelGGL((tkg_down_kernel<NT>), g2, dim3(256), 0, s, w.h_hi, w.h_lo, (int)H,     \
                       (int)I, dn_q, dn_s, dn_bias, w.expert_off, w.active, w.n_active, w.y); \
    mark(3);                                                                                 \
  } while (0)
  if (maxne <= 16) MXMOE_TKG_LAUNCH(1);
  else if (maxne <= 32) MXMOE_TKG_LAUNCH(2);
  else MXMOE_TKG_LAUNCH(4);
#undef MXMOE_TKG_LAUNCH
  hipLaunchKernelGGL(tkg_combine_kernel, dim3((unsigned)((H / 4 + 255) / 256), (unsigned)T),
                     dim3(256), 0, s, w.y, w.tok_slot, w.tok_w, (int)H, top_k, out);
  mark(4);
  return check_launch("moe_tkg");
}
