// Prefill (context encoding) expert MLP over the blockwise mapping.
//
// Both projections run the same LDS-tiled grouped GEMM:
//   workgroup tile = 128 slots (M) x 512 weight rows (N, 32 row groups) x 128-wide
//   K chunks; 8 waves as 2 (M) x 4 (N), each wave 64 slots x 128 rows = 8 x 4
//   MFMA 16x16x32 tiles.  Per chunk the workgroup moves 32 KiB of activations (bf16,
//   16-byte blocks XOR-swizzled by row against bank conflicts), 32 KiB of packed
//   weights and 2 KiB of scales from global memory straight into LDS (no register
//   staging), two stages deep: chunk c + 1 streams in while chunk c computes.
//   Weights are dequantized from LDS to bf16 in registers by the CDNA4 scaled
//   conversion, right before the MFMAs.
//   M-tiles never straddle blocks (block_size % 128 == 0) so one tile has one
//   expert; tiles whose 128 slots are all padding exit at once, and inside a tile
//   each wave runs only the 16-slot MFMA tiles that hold real slots.  Tiles are
//   ordered N-fastest and dealt out XCD by XCD, so the workgroups sharing an
//   M-tile's activations (and an expert's weights) sit on the same L2.
// gate_up: A = x rows gathered through token_position_to_id; epilogue = bias,
//          clamps, activation and up * act with the reference's bf16 roundings;
//          writes h [slots, I] bf16.
// down:    A = h rows of the same slots; epilogue = bias with bf16 roundings;
//          writes y [slots, H] bf16.
// combine: out[t] = bf16(sum over experts in ascending id of y * affinity) in fp32.
#include <math.h>

#include <type_traits>

#include "capi_util.h"
#include "common.h"

namespace mxmoe {

constexpr int kPM = 128;    // slots per M-tile
constexpr int kPRG = 32;    // row groups per N-tile (512 rows), 8 per wave
constexpr int kPThreads = 512;

struct PrefillArgs {
  const uint16_t* a;      // x [T, H] (gate_up) or h [slots, I] (down)
  const uint8_t* wq;      // packed weights, all experts
  const uint8_t* ws;      // packed scales
  const uint16_t* bias;   // gate_up: [E, 2, I]; down: [E, H]; may be null
  const int32_t* tp2id;   // token_position_to_id [slots]
  const int32_t* b2e;     // block_to_expert [n_blocks]
  uint16_t* out;          // h [slots, I] or y [slots, H]
  int T, K, N_rows, I, H, B;
  int n_mtiles, n_ntiles;
  ExpertParams p;
};

__device__ __forceinline__ float rb(float v) { return round_bf16(v); }

__device__ __forceinline__ float clamp_ref(float v, float lo, float hi) {
  v = (v > hi) ? hi : v;
  v = (v < lo) ? lo : v;
  return v;
}

// Activation on a bf16 value with the reference's bf16 intermediate roundings.
__device__ __forceinline__ float act_bf16(float g, int act) {
  if (act == kSwish) {
    const float t1 = rb(g * 1.702f);
    const float t2 = rb(1.0f / (1.0f + expf(-t1)));
    return rb(g * t2);
  }
  if (act == kSiLU) return rb(g / (1.0f + expf(-g)));
  return rb(0.5f * g * (1.0f + erff(g * 0.70710678118654752f)));
}

template <bool GATE_UP>
__global__ void __launch_bounds__(kPThreads) prefill_gemm_kernel(PrefillArgs args) {
  constexpr int WR = kPRG / 4;  // row groups per wave (4 waves across N)
  constexpr int NQ = kPRG / 4;  // scale quads per tile
  static_assert(NQ == kPThreads / 64, "one scale quad per wave");
  // The two pipeline stages are separate arrays indexed at compile time: the
  // compiler then tells the stage being read from the one a direct load is filling
  // and waits only for the former.
  __shared__ __attribute__((aligned(1024))) uint8_t sa0[kPM * 256], sa1[kPM * 256];
  __shared__ __attribute__((aligned(1024))) uint8_t sb0[kPRG * 1024], sb1[kPRG * 1024];
  __shared__ __attribute__((aligned(1024))) uint8_t ss0[NQ * 256], ss1[NQ * 256];
  __shared__ int32_t stok[kPM];
  __shared__ int s_any;

  // XCD-aware tile order (workgroups are dealt round-robin over the 8 XCDs).
  const int G = args.n_mtiles * args.n_ntiles;
  const int wg = blockIdx.x;
  const int xcd = wg & 7, i8 = wg >> 3;
  const int per = G >> 3, rem = G & 7;
  const int lin = xcd * per + min(xcd, rem) + i8;
  const int mt = lin / args.n_ntiles, nt = lin % args.n_ntiles;
  const int m0 = mt * kPM;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int q = lane >> 4;

  if (tid == 0) s_any = 0;
  __syncthreads();
  if (tid < kPM) {
    // Without a mapping (plain linear) slot m0 + tid is row m0 + tid of A.
    int tk = args.tp2id ? args.tp2id[m0 + tid] : m0 + tid;
    if (tk < 0 || tk >= args.T) tk = -1;
    stok[tid] = tk;
    if (tk >= 0) s_any = 1;
  }
  __syncthreads();
  if (!s_any) return;

  const int e = args.b2e ? args.b2e[m0 / args.B] : 0;
  const int K = args.K;
  const size_t rg_bytes = (size_t)K * 8, q_sbytes = (size_t)K * 2;
  const int n_rg_total = args.N_rows / 16;
  const int rg0 = nt * kPRG;  // a multiple of 4: the tile holds NQ scale quads
  const int rg_valid = min(kPRG, n_rg_total - rg0);
  const uint8_t* wq = args.wq + ((size_t)e * n_rg_total + rg0) * rg_bytes;
  const uint8_t* ws = args.ws + ((size_t)e * ((n_rg_total + 3) / 4) + rg0 / 4) * q_sbytes;
  const int nc = (K + 127) / 128, nfull = K / 128, tail_q = (K % 128) / 32;
  auto lane_in_k = [&](int c, int l) { return c < nfull || (l >> 4) < tail_q; };

  // ---- global -> LDS, no registers: each wave issues 4 x 1 KiB of activations (rows
  // 16w + 4i + lane/16), 4 x 1 KiB of weights (row groups 4w + i) and 256 B of
  // scales (quad w) per chunk.  A chunk row of activations (128 bf16) is 16 blocks of
  // 16 B; block cb of row r sits at slot cb ^ (r % 16), so the 16 rows an MFMA reads
  // hit 16 different slots (no bank conflicts) without padding.  Addresses are
  // clamped to real data (padding slots read token 0, columns past K read column 0,
  // row groups past the tile read the first): an MFMA output column depends on its
  // own slot only and discarded rows are never stored, and compute() gives lanes past
  // K a zero scale so their weights add nothing.
  const uint16_t* a_row[4];
  int a_swz[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 16 * wave + 4 * i + (lane >> 4);
    const int tk = stok[row];
    a_row[i] = GATE_UP ? args.a + (size_t)(tk >= 0 ? tk : 0) * K
                       : args.a + (size_t)(m0 + row) * K;
    a_swz[i] = (lane & 15) ^ (row & 15);  // the column block this lane's slot holds
  }
  auto issue_chunk = [&](auto st_c, int c) {
    constexpr int ST = decltype(st_c)::value;
    uint8_t* sa = ST ? sa1 : sa0;
    uint8_t* sb = ST ? sb1 : sb0;
    uint8_t* ss = ST ? ss1 : ss0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kcol = c * 128 + a_swz[i] * 8;
      const uint16_t* src = a_row[i] + (kcol < K ? kcol : 0);  // column 0: in the row
      __builtin_amdgcn_global_load_lds(src, &sa[(16 * wave + 4 * i) * 256], 16, 0, 0);
    }
    const int bl = lane_in_k(c, lane) ? lane : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rg = 4 * wave + i;
      const int rgc = rg < rg_valid ? rg : 0;
      __builtin_amdgcn_global_load_lds(wq + rgc * rg_bytes + (size_t)c * 1024 + bl * 16,
                                       &sb[rg * 1024], 16, 0, 0);
    }
    const int qc = 4 * wave < rg_valid ? wave : 0;
    __builtin_amdgcn_global_load_lds(ws + qc * q_sbytes + (size_t)c * 256 + bl * 4,
                                     &ss[wave * 256], 4, 0, 0);
  };

  const int wm = wave & 1, wn = wave >> 1;
  // Wave-uniform activity: its row groups exist; ntv = its 16-slot MFMA tiles that
  // hold a real slot (real slots of a block come first, so they are a prefix).
  const bool wave_rows = (WR * wn) < rg_valid;
  int ntv = 0;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    bool any = false;
    for (int i = 0; i < 16; ++i) any |= stok[64 * wm + 16 * t + i] >= 0;
    ntv = any ? t + 1 : ntv;
  }
  const bool active = wave_rows && ntv > 0;

  f32x4 acc[WR][4];
#pragma unroll
  for (int r = 0; r < WR; ++r)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // A wave computes 64 slots (NTV tiles of 16 hold real ones) x WR row groups.
  auto compute = [&](auto ntv_c, auto st_c, int c) {
    constexpr int NTV = decltype(ntv_c)::value;
    constexpr int ST = decltype(st_c)::value;
    const uint8_t* sa = ST ? sa1 : sa0;
    const uint8_t* sb = ST ? sb1 : sb0;
    const uint8_t* ss = ST ? ss1 : ss0;
    const bool kok = lane_in_k(c, lane);
    float sc[WR];
#pragma unroll
    for (int h = 0; h < WR / 4; ++h) {
      const uint32_t s4 =
          *reinterpret_cast<const uint32_t*>(&ss[(WR / 4 * wn + h) * 256 + lane * 4]);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sc[4 * h + r] = kok ? e8m0_to_f32((s4 >> (8 * r)) & 0xffu) : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int slot = (4 * q + j) ^ (lane & 15);
      u32x4 xv[NTV];
#pragma unroll
      for (int t = 0; t < NTV; ++t)
        xv[t] = *reinterpret_cast<const u32x4*>(
            &sa[(64 * wm + 16 * t + (lane & 15)) * 256 + slot * 16]);
      // dword j of each row group's 16 bytes: 8 weights of this MFMA step
      uint32_t wj[WR];
#pragma unroll
      for (int r = 0; r < WR; ++r)
        wj[r] = *reinterpret_cast<const uint32_t*>(&sb[(WR * wn + r) * 1024 + lane * 16 + 4 * j]);
#pragma unroll
      for (int r = 0; r < WR; ++r) {
        const bf16x8 wf = dequant8(wj[r], sc[r]);
#pragma unroll
        for (int t = 0; t < NTV; ++t) acc[r][t] = mfma16(wf, as_bf16x8(xv[t]), acc[r][t]);
      }
    }
  };
  // The whole K loop per tile count, so no branch sits between the MFMAs.  Chunk
  // c + 1 streams into the other LDS stage while chunk c computes; the barrier at
  // the top of each half waits (its release fence) for the chunk about to be read
  // and for every wave to be done with the stage about to be refilled.
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  auto main_loop = [&](auto ntv_c) {
    issue_chunk(S0(), 0);
    for (int c = 0; c < nc; c += 2) {
      __syncthreads();
      if (c + 1 < nc) issue_chunk(S1(), c + 1);
      if (active) compute(ntv_c, S0(), c);
      if (c + 1 >= nc) break;
      __syncthreads();
      if (c + 2 < nc) issue_chunk(S0(), c + 2);
      if (active) compute(ntv_c, S1(), c + 1);
    }
  };
  switch (ntv) {
    case 1: main_loop(std::integral_constant<int, 1>()); break;
    case 2: main_loop(std::integral_constant<int, 2>()); break;
    case 3: main_loop(std::integral_constant<int, 3>()); break;
    default: main_loop(std::integral_constant<int, 4>()); break;
  }
  if (!active) return;

  typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
  if (GATE_UP) {
    const int I = args.I;
#pragma unroll
    for (int pp = 0; pp < WR / 2; ++pp) {
      if (WR * wn + 2 * pp >= rg_valid) continue;
      const int P = (rg0 + WR * wn) / 2 + pp;  // pair index = 16 intermediate columns
      const int col0 = 16 * P + 4 * q;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int row = 64 * wm + 16 * t + (lane & 15);
        if (stok[row] < 0) continue;
        const f32x4 g4 = acc[2 * pp][t], u4 = acc[2 * pp + 1][t];
        uint16_t h[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float g = rb(g4[i]), u = rb(u4[i]);
          if (args.bias) {
            g = rb(g + bf16_bits_to_f32(args.bias[(size_t)e * 2 * I + col0 + i]));
            u = rb(u + bf16_bits_to_f32(args.bias[(size_t)e * 2 * I + I + col0 + i]));
          }
          g = clamp_ref(g, args.p.gate_lo, args.p.gate_hi);
          u = clamp_ref(u, args.p.up_lo, args.p.up_hi);
          h[i] = f32_to_bf16_bits(u * act_bf16(g, args.p.act));
        }
        *reinterpret_cast<u16x4*>(args.out + (size_t)(m0 + row) * I + col0) =
            u16x4{h[0], h[1], h[2], h[3]};
      }
    }
  } else {
    const int H = args.H;
#pragma unroll
    for (int r = 0; r < WR; ++r) {
      if (WR * wn + r >= rg_valid) continue;
      const int n0 = 16 * (rg0 + WR * wn + r) + 4 * q;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int row = 64 * wm + 16 * t + (lane & 15);
        if (stok[row] < 0) continue;
        uint16_t y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = rb(acc[r][t][i]);
          if (args.bias) v = rb(v + bf16_bits_to_f32(args.bias[(size_t)e * H + n0 + i]));
          y[i] = f32_to_bf16_bits(v);
        }
        *reinterpret_cast<u16x4*>(args.out + (size_t)(m0 + row) * H + n0) =
            u16x4{y[0], y[1], y[2], y[3]};
      }
    }
  }
}

// inv[t, e] = slot of (t, e) or -1.
__global__ void cte_inverse_kernel(const int32_t* __restrict__ tp2id,
                                   const int32_t* __restrict__ b2e, int64_t n_slots, int B, int T,
                                   int E, int32_t* __restrict__ inv) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n_slots) return;
  const int tk = tp2id[p];
  if (tk < 0 || tk >= T) return;
  const int e = b2e[p / B];
  if (e < 0 || e >= E) return;
  inv[(size_t)tk * E + e] = (int32_t)p;
}

// out[t, n] = bf16(sum_e float(y[inv[t,e], n]) * aff[t*E + e]) for e ascending.
__global__ void __launch_bounds__(256) cte_combine_kernel(const uint16_t* __restrict__ y,
                                                          const int32_t* __restrict__ inv,
                                                          const float* __restrict__ aff, int H,
                                                          int E, int scale_mode, int out_f32,
                                                          void* __restrict__ out) {
  const int t = blockIdx.y;
  const int n = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (n >= H) return;
  typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int e = 0; e < E; ++e) {
    const int p = inv[(size_t)t * E + e];
    if (p < 0) continue;
    float a = aff[(size_t)t * E + e];
    if (scale_mode == MXMOE_SCALE_NO) a = 1.0f;
    const u16x4 v = *reinterpret_cast<const u16x4*>(y + (size_t)p * H + n);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = __fadd_rn(acc[i], __fmul_rn(bf16_bits_to_f32(v[i]), a));
  }
  if (out_f32) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(out) + (size_t)t * H + n) = acc;
  } else {
    *reinterpret_cast<u16x4*>(static_cast<uint16_t*>(out) + (size_t)t * H + n) =
        u16x4{f32_to_bf16_bits(acc[0]), f32_to_bf16_bits(acc[1]), f32_to_bf16_bits(acc[2]),
              f32_to_bf16_bits(acc[3])};
  }
}

__global__ void fill_i32_k(int32_t* __restrict__ p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

struct CteWs {
  uint16_t* h;
  uint16_t* y;
  int32_t* inv;
};

static size_t cte_carve(void* base, size_t cap, int64_t T, int64_t H, int64_t I, int64_t E,
                        int64_t n_slots, CteWs* w) {
  Carver cv(base, cap);
  CteWs c;
  c.h = cv.take<uint16_t>(n_slots * I);
  c.y = cv.take<uint16_t>(n_slots * H);
  c.inv = cv.take<int32_t>(T * E);
  if (w) *w = c;
  return cv.off + 256;
}

}  // namespace mxmoe

using namespace mxmoe;

extern "C" size_t mxmoe_moe_cte_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                                                int64_t block_size, int64_t n_blocks) {
  return cte_carve(nullptr, ~(size_t)0, T, H, I, E, block_size * n_blocks, nullptr);
}

extern "C" int mxmoe_moe_cte(const uint16_t* x, const float* affinities_masked,
                             const uint8_t* gu_q, const uint8_t* gu_s, const uint8_t* dn_q,
                             const uint8_t* dn_s, const uint16_t* gu_bias,
                             const uint16_t* dn_bias, const int32_t* token_position_to_id,
                             const int32_t* block_to_expert, int64_t n_blocks, int64_t block_size,
                             int64_t T, int64_t H, int64_t I, int64_t E, int act,
                             const float* clamps, int scale_mode, int out_f32, void* out,
                             void* workspace, size_t workspace_bytes, void* const* stage_events,
                             void* stream) {
  clear_error();
  MXMOE_REQUIRE(x && affinities_masked && gu_q && gu_s && dn_q && dn_s && token_position_to_id &&
                    block_to_expert && out && workspace,
                "moe_cte: null pointer");
  MXMOE_REQUIRE(T >= 1 && E >= 1 && n_blocks >= 1, "moe_cte: bad T/E/n_blocks");
  MXMOE_REQUIRE(block_size >= 128 && block_size % 128 == 0,
                "moe_cte: block_size=%lld must be a multiple of 128", (long long)block_size);
  MXMOE_REQUIRE(H % 32 == 0 && I % 32 == 0 && H >= 32 && I >= 32,
                "moe_cte: H=%lld and I=%lld must be multiples of 32", (long long)H, (long long)I);
  MXMOE_REQUIRE(act >= 0 && act <= 2, "moe_cte: unknown activation %d", act);
  MXMOE_REQUIRE(scale_mode == MXMOE_SCALE_POST || scale_mode == MXMOE_SCALE_NO,
                "moe_cte: unsupported scale mode %d", scale_mode);
  const int64_t n_slots = n_blocks * block_size;
  const size_t need = cte_carve(nullptr, ~(size_t)0, T, H, I, E, n_slots, nullptr);
  if (workspace_bytes < need)
    return set_error(MXMOE_E_WORKSPACE, "moe_cte: workspace %zu < %zu", workspace_bytes, need);
  CteWs w;
  cte_carve(workspace, workspace_bytes, T, H, I, E, n_slots, &w);
  hipStream_t s = as_stream(stream);
  auto mark = [&](int i) {
    mark_event(stage_events, i, s);
  };

  PrefillArgs a;
  a.tp2id = token_position_to_id;
  a.b2e = block_to_expert;
  a.T = (int)T;
  a.I = (int)I;
  a.H = (int)H;
  a.B = (int)block_size;
  a.n_mtiles = (int)(n_slots / kPM);
  a.p.gate_lo = clamps ? clamps[0] : -INFINITY;
  a.p.gate_hi = clamps ? clamps[1] : INFINITY;
  a.p.up_lo = clamps ? clamps[2] : -INFINITY;
  a.p.up_hi = clamps ? clamps[3] : INFINITY;
  a.p.act = act;

  // gate_up: A = x (K = H), rows = 2I
  a.a = x;
  a.wq = gu_q;
  a.ws = gu_s;
  a.bias = gu_bias;
  a.out = w.h;
  a.K = (int)H;
  a.N_rows = (int)(2 * I);
  a.n_ntiles = (int)((2 * I / 16 + kPRG - 1) / kPRG);
  mark(0);
  hipLaunchKernelGGL(prefill_gemm_kernel<true>, dim3((unsigned)(a.n_mtiles * a.n_ntiles)),
                     dim3(kPThreads), 0, s, a);
  mark(1);
  // down: A = h (K = I), rows = H
  a.a = w.h;
  a.wq = dn_q;
  a.ws = dn_s;
  a.bias = dn_bias;
  a.out = w.y;
  a.K = (int)I;
  a.N_rows = (int)H;
  a.n_ntiles = (int)((H / 16 + kPRG - 1) / kPRG);
  hipLaunchKernelGGL(prefill_gemm_kernel<false>, dim3((unsigned)(a.n_mtiles * a.n_ntiles)),
                     dim3(kPThreads), 0, s, a);
  mark(2);
  hipLaunchKernelGGL(fill_i32_k, dim3((unsigned)((T * E + 255) / 256)), dim3(256), 0, s, w.inv,
                     T * E, -1);
  hipLaunchKernelGGL(cte_inverse_kernel, dim3((unsigned)((n_slots + 255) / 256)), dim3(256), 0, s,
                     token_position_to_id, block_to_expert, n_slots, (int)block_size, (int)T,
                     (int)E, w.inv);
  hipLaunchKernelGGL(cte_combine_kernel, dim3((unsigned)((H / 4 + 255) / 256), (unsigned)T),
                     dim3(256), 0, s, w.y, w.inv, affinities_masked, (int)H, (int)E, scale_mode,
                     out_f32, out);
  mark(3);
  return check_launch("moe_cte");
}

extern "C" int mxmoe_linear(const uint16_t* x, int64_t M, const uint8_t* wq, const uint8_t* ws,
                            int64_t N, int64_t K, uint16_t* y, void* stream) {
  clear_error();
  MXMOE_REQUIRE(x && wq && ws && y, "linear: null pointer");
  MXMOE_REQUIRE(M >= 0 && N >= 16 && N % 16 == 0 && K >= 32 && K % 32 == 0,
                "linear: N=%lld must be a multiple of 16 and K=%lld of 32", (long long)N,
                (long long)K);
  if (M == 0) return MXMOE_OK;
  PrefillArgs a = {};
  a.a = x;
  a.wq = wq;
  a.ws = ws;
  a.out = y;
  a.T = (int)M;
  a.K = (int)K;
  a.N_rows = (int)N;
  a.H = (int)N;
  a.I = 0;
  a.B = kPM;
  a.n_mtiles = (int)((M + kPM - 1) / kPM);
  a.n_ntiles = (int)((N / 16 + kPRG - 1) / kPRG);
  a.p.gate_lo = -INFINITY;
  a.p.gate_hi = INFINITY;
  a.p.up_lo = -INFINITY;
  a.p.up_hi = INFINITY;
  hipLaunchKernelGGL(prefill_gemm_kernel<false>, dim3((unsigned)(a.n_mtiles * a.n_ntiles)),
                     dim3(kPThreads), 0, as_stream(stream), a);
  return check_launch("linear");
}
