// Router: fp32 logits with bf16 MFMA (products of bf16 values are exact in fp32),
// top-k by wave-wide arg-max rounds, activation, scatter; and the decode RMSNorm.
#include <math.h>

#include "capi_util.h"
#include "common.h"
#include "router_dev.h"

namespace mxmoe {

// logits[t, e] = sum_h x[t, h] * w[e, h] (+ bias[e]).  One workgroup = TT token tiles x
// ET expert tiles of 16; its NW waves split the 128-wide K chunks round-robin and
// reduce through LDS in a fixed order.  A = router rows (experts), B = tokens.
// Operands are 16-bit (XF16 / WF16: fp16, else bf16), multiplied as OP says:
//   kOpBF16   bf16 MFMA; fp16 weights are first rounded to bf16 (a cast to bf16)
//   kOpF16    fp16 MFMA; bf16 operands are first rounded to fp16 (a cast to fp16)
//   kOpExact  x bf16 times fp16 weights split exactly into bf16 hi + lo, two bf16
//             MFMAs: every product is exact, as in an fp32 matmul of the two
// (products of two bf16 or two fp16 values are exact in fp32 as well).  The bias is
// rounded to bias_rnd and the logit to logit_rnd (Dt; kF32 leaves them as they are).
template <int TT, int ET, int NW, bool XF16, bool WF16, int OP>
__global__ void __launch_bounds__(64 * NW) router_logits_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const void* __restrict__ bias,
    int bias_dt, int bias_rnd, int logit_rnd, float* __restrict__ logits, int T, int H, int E) {
  __shared__ f32x4 red[NW][ET][TT][64];
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int q = lane >> 4, r16 = lane & 15;
  const int t0 = blockIdx.x * 16 * TT, e0 = blockIdx.y * 16 * ET;
  f32x4 acc[ET][TT];
  router_partial_logits<TT, ET, NW, XF16, WF16, OP>(x, w, T, H, E, t0, e0, wave, acc);
#pragma unroll
  for (int e = 0; e < ET; ++e)
#pragma unroll
    for (int t = 0; t < TT; ++t) red[wave][e][t][lane] = acc[e][t];
  __syncthreads();
  // Each wave finishes a share of the (e, t) tiles: fixed summation order 0..NW-1.
  for (int idx = wave; idx < ET * TT; idx += NW) {
    const int e = idx / TT, t = idx % TT;
    f32x4 s = red[0][e][t][lane];
#pragma unroll
    for (int v = 1; v < NW; ++v) s += red[v][e][t][lane];
    const int tok = t0 + 16 * t + r16;
    if (tok >= T) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ex = e0 + 16 * e + 4 * q + i;
      if (ex >= E) continue;
      float v = s[i];
      if (bias) v += round_to(load_opt_f32(bias, ex, bias_dt, w), bias_rnd);
      logits[(size_t)tok * E + ex] = round_to(v, logit_rnd);
    }
  }
}

// One wave per token: top-k over the row (desc., ties -> lower id), activation, scatter.
// The activation outputs are rounded to rnd (Dt); aff (fp32) or aff16 (bf16 bits) may be
// null.
template <int PER>
__global__ void __launch_bounds__(256) router_topk_kernel(
    const float* __restrict__ logits, float* __restrict__ aff, uint16_t* __restrict__ aff16,
    int32_t* __restrict__ topk_idx, float* __restrict__ topk_val, int T, int E, int K, int act,
    int act_first, int renorm, float renorm_eps, int rnd) {
  const int lane = threadIdx.x & 63;
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= T) return;
  int sel_idx[8];
  float out[8];
  float vals[PER];
  load_row_wave<PER>(logits + (size_t)tok * E, E, vals);
  topk_row_wave<PER>(vals, E, K, act, act_first, renorm, renorm_eps, rnd, sel_idx, out);
  if (aff || aff16) {
    for (int e = lane; e < E; e += 64) {
      float a = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k < K && sel_idx[k] == e) a = out[k];
      if (aff) aff[(size_t)tok * E + e] = a;
      if (aff16) aff16[(size_t)tok * E + e] = f32_to_bf16_bits(a);
    }
  }
  store_topk_wave(sel_idx, out, K, topk_idx + (size_t)tok * K, topk_val + (size_t)tok * K);
}

// One workgroup per token: RMSNorm of a bf16 row, fp32 arithmetic, the result rounded to
// out_dt (bf16 or fp16 bits).  The mean square divides by ha; the squares are summed
// over the first ha columns (all_cols = 0, then columns >= ha are written as 0) or over
// all H columns (all_cols = 1, every column normalized).  out = gamma * (x * inv) with
// inv = 1 / sqrt(mean + eps), the operation order of the reference's flows.
__global__ void __launch_bounds__(256) rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const float* __restrict__ gamma, int H,
                                                      int ha, int all_cols, float eps, int out_dt,
                                                      uint16_t* __restrict__ out) {
  __shared__ float part[4];
  const uint16_t* xr = x + (size_t)blockIdx.x * H;
  uint16_t* orow = out + (size_t)blockIdx.x * H;
  const int ncols = all_cols ? H : ha;
  float s = 0.f;
  for (int h = threadIdx.x; h < ncols; h += 256) {
    const float v = bf16_bits_to_f32(xr[h]);
    s += v * v;
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  const float var = (part[0] + part[1] + part[2] + part[3]) / (float)ha;
  const float inv = 1.0f / sqrtf(var + eps);
  for (int h = threadIdx.x; h < H; h += 256) {
    const bool keep = all_cols || h < ha;
    const float v = keep ? gamma[h] * (bf16_bits_to_f32(xr[h]) * inv) : 0.f;
    orow[h] = out_dt == kF16 ? f32_to_f16_bits(v) : f32_to_bf16_bits(v);
  }
}

}  // namespace mxmoe

using namespace mxmoe;

extern "C" size_t mxmoe_router_workspace_bytes(int64_t, int64_t) { return 0; }

namespace mxmoe {

template <int TT, int ET, int NW>
static void launch_logits(const RouterSpec& r, dim3 grid, float* logits, int T, int H, int E,
                          hipStream_t s) {
#define MXMOE_LOGITS(XF, WF, OP)                                                              \
  hipLaunchKernelGGL((router_logits_kernel<TT, ET, NW, XF, WF, OP>), grid, dim3(64 * NW), 0, s, \
                     r.x, r.w, r.bias, r.bias_dt, r.bias_rnd, r.logit_rnd, logits, T, H, E)
  const bool xh = r.x_dt == kF16, wh = r.w_dt == kF16;
  if (r.op == kOpF16) {
    if (xh && wh) MXMOE_LOGITS(true, true, kOpF16);
    else if (xh) MXMOE_LOGITS(true, false, kOpF16);
    else if (wh) MXMOE_LOGITS(false, true, kOpF16);
    else MXMOE_LOGITS(false, false, kOpF16);
  } else if (r.op == kOpExact && wh) {
    MXMOE_LOGITS(false, true, kOpExact);
  } else if (wh) {
    MXMOE_LOGITS(false, true, kOpBF16);
  } else {
    MXMOE_LOGITS(false, false, kOpBF16);
  }
#undef MXMOE_LOGITS
}

int router_check(const RouterSpec& r) {
  MXMOE_REQUIRE(r.x && r.w, "router: null pointer");
  MXMOE_REQUIRE(r.x_dt == kBF16 || r.x_dt == kF16, "router: x dtype %d must be bf16 or fp16",
                r.x_dt);
  MXMOE_REQUIRE(r.w_dt == kBF16 || r.w_dt == kF16, "router: weight dtype %d must be bf16 or fp16",
                r.w_dt);
  MXMOE_REQUIRE(!r.bias || (r.bias_dt >= kF32 && r.bias_dt <= kBF16),
                "router: bias dtype %d unknown", r.bias_dt);
  MXMOE_REQUIRE(r.op == kOpBF16 || r.op == kOpF16 || r.op == kOpExact,
                "router: operand mode %d unknown", r.op);
  MXMOE_REQUIRE(r.op == kOpF16 || r.x_dt == kBF16,
                "router: fp16 activations are multiplied in fp16 only");
  return MXMOE_OK;
}

// Shared by the router entry points and the fused decode layer; affinities (fp32) and
// aff16 (bf16) may be null.
int router_run(const RouterSpec& r, int64_t T, int64_t H, int64_t E, int top_k, int act,
               int act_before_topk, int renorm, float renorm_eps, float* logits,
               float* affinities, uint16_t* aff16, int32_t* topk_idx, float* topk_val,
               hipStream_t s) {
  int rc = router_check(r);
  if (rc) return rc;
  MXMOE_REQUIRE(logits && topk_idx && topk_val, "router: null pointer");
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
    // (64 x 64 tiles left half of the CUs idle: 34 -> 27 us with the top-k; eight waves
    // per workgroup on 32 x 32 or 16 x 64 tiles measured 11 % and 26 % slower).
    dim3 grid((unsigned)((T + 31) / 32), (unsigned)((E + 63) / 64));
    launch_logits<2, 4, 4>(r, grid, logits, (int)T, (int)H, (int)E, s);
  } else {
    dim3 grid((unsigned)((T + 15) / 16), (unsigned)((E + 15) / 16));
    launch_logits<1, 1, 4>(r, grid, logits, (int)T, (int)H, (int)E, s);
  }
  rc = check_launch("router_logits");
  if (rc) return rc;
  const dim3 g((unsigned)((T + 3) / 4));
  const int af = act_before_topk ? 1 : 0, rn = renorm ? 1 : 0;
#define MXMOE_TOPK(P)                                                                          \
  hipLaunchKernelGGL(router_topk_kernel<P>, g, dim3(256), 0, s, logits, affinities, aff16,    \
                     topk_idx, topk_val, (int)T, (int)E, top_k, act, af, rn, renorm_eps,       \
                     r.act_rnd)
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

extern "C" int mxmoe_router_topk(const void* x, int x_dtype, const void* w, int w_dtype,
                                 const void* bias, int bias_dtype, int64_t T, int64_t H,
                                 int64_t E, int top_k, int act, int act_before_topk, int renorm,
                                 float renorm_eps, int compute_dtype, float* logits,
                                 float* affinities, int32_t* topk_idx, float* topk_val,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  clear_error();
  MXMOE_REQUIRE(affinities, "router: null affinities");
  MXMOE_REQUIRE(compute_dtype >= kF32 && compute_dtype <= kBF16,
                "router: compute dtype %d unknown", compute_dtype);
  RouterSpec r;
  r.x = static_cast<const uint16_t*>(x);
  r.x_dt = x_dtype;
  r.w = static_cast<const uint16_t*>(w);
  r.w_dt = w_dtype;
  r.bias = bias;
  r.bias_dt = bias_dtype;
  if (compute_dtype == kF32) {
    // Every operand is exact in fp32: fp16 weights go through the exact split.
    MXMOE_REQUIRE(x_dtype == kBF16, "router: fp32 computation takes bf16 activations");
    r.op = w_dtype == kF16 ? kOpExact : kOpBF16;
  } else {
    MXMOE_REQUIRE(compute_dtype == kF16 || x_dtype == kBF16,
                  "router: bf16 computation takes bf16 activations");
    r.op = compute_dtype == kF16 ? kOpF16 : kOpBF16;
  }
  r.bias_rnd = r.logit_rnd = r.act_rnd = compute_dtype;
  return router_run(r, T, H, E, top_k, act, act_before_topk, renorm, renorm_eps, logits,
                    affinities, nullptr, topk_idx, topk_val, as_stream(stream));
}

namespace mxmoe {

int rmsnorm_run(const uint16_t* x, const float* gamma, int64_t T, int64_t H, int64_t ha,
                int all_cols, float eps, int out_dt, uint16_t* out, hipStream_t s) {
  MXMOE_REQUIRE(x && gamma && out, "rmsnorm: null pointer");
  MXMOE_REQUIRE(T >= 0 && H > 0 && ha > 0 && ha <= H, "rmsnorm: bad shape");
  MXMOE_REQUIRE(out_dt == kBF16 || out_dt == kF16, "rmsnorm: output dtype %d must be bf16 or fp16",
                out_dt);
  if (T == 0) return MXMOE_OK;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)T), dim3(256), 0, s, x, gamma, (int)H,
                     (int)ha, all_cols ? 1 : 0, eps, out_dt, out);
  return check_launch("rmsnorm");
}

}  // namespace mxmoe

extern "C" int mxmoe_rmsnorm(const uint16_t* x, const float* gamma, int64_t T, int64_t H,
                             int64_t h_actual, int all_cols, float eps, int out_dtype,
                             uint16_t* out, void* stream) {
  clear_error();
  return rmsnorm_run(x, gamma, T, H, h_actual, all_cols, eps, out_dtype, out, as_stream(stream));
}

extern "C" size_t mxmoe_rmsnorm_router_topk_workspace_bytes(int64_t T, int64_t E, int top_k) {
  return align_up((size_t)T * (size_t)E * 4u, 256) + align_up((size_t)T * (size_t)top_k * 4u, 256);
}

extern "C" int mxmoe_rmsnorm_router_topk(const uint16_t* x, const float* gamma, int64_t h_actual,
                                         float eps, const void* router_w, int w_dtype,
                                         const void* router_b, int b_dtype, int64_t T, int64_t H,
                                         int64_t E, int top_k, int act, int mm_dtype,
                                         uint16_t* norm_out, int32_t* topk_idx,
                                         uint16_t* affinities, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  clear_error();
  MXMOE_REQUIRE(workspace && topk_idx && affinities && norm_out,
                "rmsnorm_router_topk: null pointer");
  MXMOE_REQUIRE(mm_dtype == kF16 || mm_dtype == kBF16,
                "rmsnorm_router_topk: router matmul dtype %d must be fp16 or bf16", mm_dtype);
  const size_t need = mxmoe_rmsnorm_router_topk_workspace_bytes(T, E, top_k);
  if (workspace_bytes < need)
    return set_error(MXMOE_E_WORKSPACE, "rmsnorm_router_topk: workspace %zu < %zu",
                     workspace_bytes, need);
  hipStream_t s = as_stream(stream);
  int rc = rmsnorm_run(x, gamma, T, H, h_actual, /*all_cols=*/1, eps, mm_dtype, norm_out, s);
  if (rc) return rc;
  float* logits = static_cast<float*>(workspace);
  float* vals = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                         align_up((size_t)T * (size_t)E * 4u, 256));
  RouterSpec r;
  r.x = norm_out;
  r.x_dt = mm_dtype;
  r.w = static_cast<const uint16_t*>(router_w);
  r.w_dt = w_dtype;
  r.bias = router_b;
  r.bias_dt = b_dtype;
  r.op = mm_dtype == kF16 ? kOpF16 : kOpBF16;
  r.bias_rnd = mm_dtype;
  r.logit_rnd = kF32;
  r.act_rnd = kF32;
  return router_run(r, T, H, E, top_k, act, /*act_before_topk=*/0, /*renorm=*/0, 0.f, logits,
                    nullptr, affinities, topk_idx, vals, s);
}
