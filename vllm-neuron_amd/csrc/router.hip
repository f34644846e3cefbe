// Router: fp32 logits with bf16 MFMA (products of bf16 values are exact in fp32),
// top-k by wave-wide arg-max rounds, activation, scatter; and the decode RMSNorm.
#include <math.h>

#include "capi_util.h"
#include "common.h"
#include "router_dev.h"

namespace mxmoe {

// logits[t, e] = sum_h x[t, h] * w[e, h] (+ bias[e]).  One workgroup = TT token tiles x
// ET expert tiles of 16; its 4 waves split the 128-wide K chunks round-robin and
// reduce through LDS in a fixed order.  A = router rows (experts), B = tokens.
template <int TT, int ET>
__global__ void __launch_bounds__(256) router_logits_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ bias, float* __restrict__ logits, int T, int H, int E) {
  __shared__ f32x4 red[4][ET][TT][64];
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int q = lane >> 4, r16 = lane & 15;
  const int t0 = blockIdx.x * 16 * TT, e0 = blockIdx.y * 16 * ET;
  const int nc = (H + 127) / 128;
  const int tail_q = (H % 128) / 32;  // blocks of 32 in a partial last chunk

  const uint16_t* xr[TT];
  const uint16_t* wr[ET];
#pragma unroll
  for (int t = 0; t < TT; ++t) xr[t] = x + (size_t)min(t0 + 16 * t + r16, T - 1) * H;
#pragma unroll
  for (int e = 0; e < ET; ++e) wr[e] = w + (size_t)min(e0 + 16 * e + r16, E - 1) * H;

  f32x4 acc[ET][TT];
#pragma unroll
  for (int e = 0; e < ET; ++e)
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[e][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  for (int c = wave; c < nc; c += 4) {
    // Lanes past K in a partial last chunk feed zeros; every lane runs the MFMAs.
    const bool ok = (c < H / 128) || (q < tail_q);
    const int k0 = c * 128 + q * 32;
    u32x4 xv[TT][4], wv[ET][4];
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
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < ET; ++e)
#pragma unroll
        for (int t = 0; t < TT; ++t)
          acc[e][t] = mfma16(as_bf16x8(wv[e][j]), as_bf16x8(xv[t][j]), acc[e][t]);
  }
#pragma unroll
  for (int e = 0; e < ET; ++e)
#pragma unroll
    for (int t = 0; t < TT; ++t) red[wave][e][t][lane] = acc[e][t];
  __syncthreads();
  // Each wave finishes a share of the (e, t) tiles: fixed summation order 0..3.
  for (int idx = wave; idx < ET * TT; idx += 4) {
    const int e = idx / TT, t = idx % TT;
    f32x4 s = red[0][e][t][lane];
#pragma unroll
    for (int v = 1; v < 4; ++v) s += red[v][e][t][lane];
    const int tok = t0 + 16 * t + r16;
    if (tok >= T) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ex = e0 + 16 * e + 4 * q + i;
      if (ex >= E) continue;
      float v = s[i];
      if (bias) v += bf16_bits_to_f32(bias[ex]);
      logits[(size_t)tok * E + ex] = v;
    }
  }
}

// One wave per token: top-k over the row (desc., ties -> lower id), activation, scatter.
template <int PER>
__global__ void __launch_bounds__(256) router_topk_kernel(
    const float* __restrict__ logits, float* __restrict__ aff, int32_t* __restrict__ topk_idx,
    float* __restrict__ topk_val, int T, int E, int K, int act, int act_first, int renorm,
    float renorm_eps) {
  const int lane = threadIdx.x & 63;
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= T) return;
  int sel_idx[8];
  float out[8];
  float vals[PER];
  load_row_wave<PER>(logits + (size_t)tok * E, E, vals);
  topk_row_wave<PER>(vals, E, K, act, act_first, renorm, renorm_eps, sel_idx, out);
  if (aff) {
    float* arow = aff + (size_t)tok * E;
    for (int e = lane; e < E; e += 64) {
      float a = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k < K && sel_idx[k] == e) a = out[k];
      arow[e] = a;
    }
  }
  store_topk_wave(sel_idx, out, K, topk_idx + (size_t)tok * K, topk_val + (size_t)tok * K);
}

// One workgroup per token: x_norm = bf16(gamma * (x * rsqrt(mean(x[:ha]^2) + eps))).
__global__ void __launch_bounds__(256) rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const float* __restrict__ gamma, int H,
                                                      int ha, float eps,
                                                      uint16_t* __restrict__ out) {
  __shared__ float part[4];
  const uint16_t* xr = x + (size_t)blockIdx.x * H;
  uint16_t* orow = out + (size_t)blockIdx.x * H;
  float s = 0.f;
  for (int h = threadIdx.x; h < ha; h += 256) {
    const float v = bf16_bits_to_f32(xr[h]);
    s += v * v;
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  const float var = (part[0] + part[1] + part[2] + part[3]) / (float)ha;
  const float inv = 1.0f / sqrtf(var + eps);
  for (int h = threadIdx.x; h < H; h += 256) {
    float v = 0.f;
    if (h < ha) v = gamma[h] * (bf16_bits_to_f32(xr[h]) * inv);
    orow[h] = (h < ha) ? f32_to_bf16_bits(v) : (uint16_t)0;
  }
}

}  // namespace mxmoe

using namespace mxmoe;

extern "C" size_t mxmoe_router_workspace_bytes(int64_t, int64_t) { return 0; }

namespace mxmoe {

// Shared by mxmoe_router_topk and the fused decode layer; affinities may be null.
int router_run(const uint16_t* x, const uint16_t* w, const uint16_t* bias, int64_t T, int64_t H,
               int64_t E, int top_k, int act, int act_before_topk, int renorm, float renorm_eps,
               float* logits, float* affinities, int32_t* topk_idx, float* topk_val,
               hipStream_t s) {
  MXMOE_REQUIRE(x && w && logits && topk_idx && topk_val, "router: null pointer");
  MXMOE_REQUIRE(T >= 0 && H > 0 && H % 32 == 0, "router: H=%lld must be a positive multiple of 32",
                (long long)H);
  MXMOE_REQUIRE(E >= 1 && E <= 64 * kMaxEPerLane, "router: E=%lld out of range [1, 1024]",
                (long long)E);
  MXMOE_REQUIRE(top_k >= 1 && top_k <= 8 && top_k <= E, "router: top_k=%d out of range", top_k);
  MXMOE_REQUIRE(act == MXMOE_ROUTER_SOFTMAX || act == MXMOE_ROUTER_SIGMOID,
                "router: unknown activation %d", act);
  if (T == 0) return MXMOE_OK;
  if (T >= 1024 && E >= 64) {
    // 32 tokens x 64 experts per workgroup: 256 workgroups at 4096 tokens and 128 experts
    // (64 x 64 tiles left half of the CUs idle: 34 -> 27 us with the top-k).
    dim3 grid((unsigned)((T + 31) / 32), (unsigned)((E + 63) / 64));
    hipLaunchKernelGGL((router_logits_kernel<2, 4>), grid, dim3(256), 0, s, x, w, bias, logits,
                       (int)T, (int)H, (int)E);
  } else {
    dim3 grid((unsigned)((T + 15) / 16), (unsigned)((E + 15) / 16));
    hipLaunchKernelGGL((router_logits_kernel<1, 1>), grid, dim3(256), 0, s, x, w, bias, logits,
                       (int)T, (int)H, (int)E);
  }
  int rc = check_launch("router_logits");
  if (rc) return rc;
  const dim3 g((unsigned)((T + 3) / 4));
  const int af = act_before_topk ? 1 : 0, rn = renorm ? 1 : 0;
#define MXMOE_TOPK(P)                                                                          \
  hipLaunchKernelGGL(router_topk_kernel<P>, g, dim3(256), 0, s, logits, affinities, topk_idx, \
                     topk_val, (int)T, (int)E, top_k, act, af, rn, renorm_eps)
  switch (topk_per_lane((int)E)) {
    case 1: MXMOE_TOPK(1); break;
    case 2: MXMOE_TOPK(2); break;
    case 4: MXMOE_TOPK(4); break;
    case 8: MXMOE_TOPK(8); break;
    default: MXMOE_TOPK(16); break;
  }
#undef MXMOE_TOPK
  return check_launch("router_topk");
}

}  // namespace mxmoe

extern "C" int mxmoe_router_topk(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                 int64_t T, int64_t H, int64_t E, int top_k, int act,
                                 int act_before_topk, int renorm, float renorm_eps, float* logits,
                                 float* affinities, int32_t* topk_idx, float* topk_val,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  clear_error();
  MXMOE_REQUIRE(affinities, "router: null affinities");
  return router_run(x, w, bias, T, H, E, top_k, act, act_before_topk, renorm, renorm_eps, logits,
                    affinities, topk_idx, topk_val, as_stream(stream));
}

namespace mxmoe {

int rmsnorm_run(const uint16_t* x, const float* gamma, int64_t T, int64_t H, int64_t ha,
                float eps, uint16_t* out, hipStream_t s) {
  MXMOE_REQUIRE(x && gamma && out, "rmsnorm: null pointer");
  MXMOE_REQUIRE(T >= 0 && H > 0 && ha > 0 && ha <= H, "rmsnorm: bad shape");
  if (T == 0) return MXMOE_OK;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)T), dim3(256), 0, s, x, gamma, (int)H,
                     (int)ha, eps, out);
  return check_launch("rmsnorm");
}

}  // namespace mxmoe

extern "C" int mxmoe_rmsnorm(const uint16_t* x, const float* gamma, int64_t T, int64_t H,
                             int64_t h_actual, float eps, uint16_t* out, void* stream) {
  clear_error();
  return rmsnorm_run(x, gamma, T, H, h_actual, eps, out, as_stream(stream));
}
