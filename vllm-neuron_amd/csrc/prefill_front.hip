// The prefill MoE layer in one call: router, blockwise mapping, the M-tile schedule and
// the moe_cte flow (expert_prefill.hip) behind them.
//
// The separate operator calls take seven dependent launches before the first GEMM
// (router logits, top-k, mapping count / scan / scatter, tile order) and the router
// logits read their operands in 32-token x 64-expert tiles.  Here three launches do it:
//   pf_logits_kernel   workgroup = 64 tokens x 64 ETW experts x one quarter of K (the
//                      128-wide chunks q, q + 4, ...), operands staged through LDS once
//                      per workgroup; writes fp32 partial sums part[q][T][E] and clears the
//                      64-token chunk masks;
//   pf_topk_kernel     a wave per token: partial sums added in the order 0..3, bias,
//                      top-k and activation, the masked affinities, the token's bits in
//                      its chunk's per-expert masks (global atomic OR); fills
//                      token_position_to_id with -1;
//   pf_place_kernel    a workgroup per 64-token chunk: each derives the per-expert totals
//                      and its chunk's prefix from all masks and places its chunk's pairs;
//                      workgroup 0 also writes block_to_expert and the schedule of the GEMMs'
//                      M-tile groups, whose weights follow from the totals (a block's real
//                      slots come first).
// The logits are the router kernel's (router.hip) bit for bit: the same K quarters, the
// same MFMA sequence per accumulator, the quarters summed in the same order.  The mapping
// and schedule equal mxmoe_blockwise_mapping's and cte_tile_order_kernel's.
#include <math.h>

#include <type_traits>

#include "capi_util.h"
#include "common.h"
#include "permute_dev.h"
#include "prefill_common.h"
#include "router_dev.h"

namespace mxmoe {

constexpr int kPfParts = 4;    // K quarters (the router kernel's four waves)
constexpr int kPfTok = 64;     // tokens per logits workgroup and per mapping chunk
// M-tiles one call schedules: the placement kernel's LDS (5 B per tile next to 25.3 KB of
// tables) stays under 64 KiB.
constexpr int kPfMaxTiles = 7168;
template <int N>
using IntC = std::integral_constant<int, N>;
static_assert(kPfTok == kChunkTok, "a logits tile is one mapping chunk");

// Partial logits part[kp][t][e] = sum over chunks c = kp, kp + 4, ... (ascending) and MFMA
// steps j = 0..3 of expert row e (A operand) times token row t (B operand), lane (q, r)
// of step j holding columns 128 c + 32 q + 8 j .. + 7 of row r: the accumulation of
// router_partial_logits' wave kp.  Workgroup: 64 tokens (4 tiles of 16) x 64 ETW experts;
// wave w takes expert tiles ETW w .. ETW w + ETW - 1 against all 64 tokens.  A chunk's
// rows (16-byte blocks XOR-swizzled by row) go global -> registers -> LDS, one chunk
// ahead, through two stages; one barrier per chunk.  The workgroups of expert tile 0 and
// part 0 also clear their token tile's chunk masks (64 bits per expert).
template <int ETW, bool XF16, bool WF16, int OP>
__global__ void __launch_bounds__(256) pf_logits_kernel(const uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ w, int T,
                                                        int H, int E, float* __restrict__ part,
                                                        unsigned long long* __restrict__ masks) {
  constexpr int TT = kPfTok / 16;
  constexpr int WR = 64 * ETW;                   // router rows per workgroup
  constexpr int XB = kPfTok * 16 / 256, WB = WR * 16 / 256;  // 16-B blocks per thread
  __shared__ __attribute__((aligned(16))) uint8_t sx[2][kPfTok * 256];
  __shared__ __attribute__((aligned(16))) uint8_t sw[2][WR * 256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, r16 = lane & 15;
  const int t0 = blockIdx.x * kPfTok, e0 = blockIdx.y * WR, kp = blockIdx.z;
  const int nc = (H + 127) / 128;
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  // The top-k kernel ORs token bits into the chunk masks: clear this token tile's.
  if (blockIdx.y == 0 && kp == 0)
    for (int i = tid; i < E; i += 256) masks[(size_t)blockIdx.x * E + i] = 0ull;

  // The part's chunks kp, kp + 4, ... go global -> registers through a ring of D slots,
  // D chunks ahead (chunk indices past the part re-read its last chunk, never computed),
  // then registers -> LDS stage one chunk ahead of the MFMAs.
  constexpr int D = 3;
  const int np = nc > kp ? (nc - kp + kPfParts - 1) / kPfParts : 0;
  auto chunk = [&](int i) { return min(kp + kPfParts * i, nc - 1); };
  u32x4 rx[D][XB], rw[D][WB];
  // Chunk c into slot d: block id = tid + 256 i -> (row id / 16, 16-B block id % 16); rows
  // past T or E re-read the last one.  Every load is issued (a block past H re-reads
  // column 0 of its row; lstore writes zeros for it), so that no branch separates them and
  // the compiler counts the ring's outstanding loads instead of draining them.
  auto gload = [&](auto d_c, int c) {
    constexpr int d = decltype(d_c)::value;
#pragma unroll
    for (int i = 0; i < XB; ++i) {
      const int id = tid + 256 * i, row = id >> 4, col = c * 128 + 8 * (id & 15);
      const int t = min(t0 + row, T - 1);
      rx[d][i] = *reinterpret_cast<const u32x4*>(x + (size_t)t * H + (col < H ? col : 0));
    }
#pragma unroll
    for (int i = 0; i < WB; ++i) {
      const int id = tid + 256 * i, row = id >> 4, col = c * 128 + 8 * (id & 15);
      const int e = min(e0 + row, E - 1);
      rw[d][i] = *reinterpret_cast<const u32x4*>(w + (size_t)e * H + (col < H ? col : 0));
    }
  };
  auto lstore = [&](auto d_c, int s, int c, bool live) {
    constexpr int d = decltype(d_c)::value;
#pragma unroll
    for (int i = 0; i < XB; ++i) {
      const int id = tid + 256 * i, row = id >> 4, b = id & 15;
      const bool ok = live && c * 128 + 8 * b < H;
      *reinterpret_cast<u32x4*>(&sx[s][row * 256 + ((b ^ (row & 15)) << 4)]) =
          ok ? rx[d][i] : zero4;
    }
#pragma unroll
    for (int i = 0; i < WB; ++i) {
      const int id = tid + 256 * i, row = id >> 4, b = id & 15;
      const bool ok = live && c * 128 + 8 * b < H;
      *reinterpret_cast<u32x4*>(&sw[s][row * 256 + ((b ^ (row & 15)) << 4)]) =
          ok ? rw[d][i] : zero4;
    }
  };

  f32x4 acc[ETW][TT];
#pragma unroll
  for (int e = 0; e < ETW; ++e)
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[e][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int s) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int boff = (((4 * q + j) ^ r16) << 4) + r16 * 256;
      u32x4 xv[TT];
#pragma unroll
      for (int t = 0; t < TT; ++t)
        xv[t] = *reinterpret_cast<const u32x4*>(&sx[s][16 * t * 256 + boff]);
#pragma unroll
      for (int e = 0; e < ETW; ++e) {
        const u32x4 wv =
            *reinterpret_cast<const u32x4*>(&sw[s][16 * (ETW * wave + e) * 256 + boff]);
        if constexpr (OP == kOpF16) {
          f16x8 a;
          if constexpr (WF16) a = __builtin_bit_cast(f16x8, wv);
          else a = bf16x8_to_f16x8(wv);
#pragma unroll
          for (int t = 0; t < TT; ++t) {
            f16x8 b;
            if constexpr (XF16) b = __builtin_bit_cast(f16x8, xv[t]);
            else b = bf16x8_to_f16x8(xv[t]);
            acc[e][t] = mfma16_f16(a, b, acc[e][t]);
          }
        } else if constexpr (OP == kOpExact) {
          static_assert(WF16 && !XF16, "exact mode splits fp16 weights against bf16 x");
          bf16x8 hi, lo;
          f16x8_split_bf16(wv, hi, lo);
#pragma unroll
          for (int t = 0; t < TT; ++t) {
            acc[e][t] = mfma16(hi, as_bf16x8(xv[t]), acc[e][t]);
            acc[e][t] = mfma16(lo, as_bf16x8(xv[t]), acc[e][t]);
          }
        } else {
          static_assert(!XF16, "bf16 MFMA takes bf16 x");
          bf16x8 a;
          if constexpr (WF16) a = f16x8_to_bf16x8(wv);
          else a = as_bf16x8(wv);
#pragma unroll
          for (int t = 0; t < TT; ++t) acc[e][t] = mfma16(a, as_bf16x8(xv[t]), acc[e][t]);
        }
      }
    }
  };

  gload(IntC<0>(), chunk(0));
  gload(IntC<1>(), chunk(1));
  gload(IntC<2>(), chunk(2));
  lstore(IntC<0>(), 0, chunk(0), np > 0);
  __syncthreads();
  int s = 0;
  // Step i (slot k = i % D holds chunk i, already in stage s): refill slot k with chunk
  // i + D, the MFMAs of chunk i, chunk i + 1 from slot k + 1 into the other stage.  The
  // steps run in whole rounds of D with no exit between them (a load whose value an early
  // exit leaves unused is moved past the exit by the compiler, which would empty the
  // ring): steps past the part's last chunk stage zeros, whose MFMAs leave the sums as
  // they are (an accumulator that starts at +0 never becomes -0, and x + 0 = x).
  auto step = [&](auto k_c, int i) {
    constexpr int k = decltype(k_c)::value;
    gload(k_c, chunk(i + D));
    __builtin_amdgcn_sched_barrier(0);  // the refill issues before the MFMAs
    compute(s);
    __builtin_amdgcn_sched_barrier(0);
    lstore(IntC<(k + 1) % D>(), s ^ 1, chunk(i + 1), i + 1 < np);
    __syncthreads();
    s ^= 1;
  };
  for (int i = 0; i < np; i += D) {
    step(IntC<0>(), i);
    step(IntC<1>(), i + 1);
    step(IntC<2>(), i + 2);
  }
  // The ring's last loads are operands here, so the compiler keeps them where issued.
#pragma unroll
  for (int d = 0; d < D; ++d) {
#pragma unroll
    for (int i = 0; i < XB; ++i) asm volatile("" ::"v"(rx[d][i]));
#pragma unroll
    for (int i = 0; i < WB; ++i) asm volatile("" ::"v"(rw[d][i]));
  }
  // Lane (q, r) of tile (e, t) holds experts 4q .. 4q + 3 of token r.
  float* pk = part + (size_t)kp * T * E;
#pragma unroll
  for (int e = 0; e < ETW; ++e)
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const int tok = t0 + 16 * t + r16;
      const int ex = e0 + 16 * (ETW * wave + e) + 4 * q;
      if (tok >= T) continue;
      float* dst = pk + (size_t)tok * E + ex;
      if ((E & 3) == 0 && ex + 3 < E) {
        *reinterpret_cast<f32x4*>(dst) = acc[e][t];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (ex + i < E) dst[i] = acc[e][t][i];
      }
    }
}

// Top-k of 4 tokens per workgroup, one token per wave (lane l holds experts l, l + 64, ...;
// topk_row_wave, as the router kernel's top-k): the selection is VALU latency-bound, and
// four waves per SIMD hide it (16-lane rows with four tokens per wave and one wave per SIMD
// measured 11.3 against 9.4 us at 4,096 tokens and 128 experts).  Per token: the logits as
// the router kernel forms them (partial sums 0..3 in order, plus the bias rounded to
// bias_rnd, the sum rounded to logit_rnd), top-k and activation, sel[t][k] = the k-th
// selected expert if its affinity a is nonzero, else -1, and val[t][k] its masked affinity
// a * padding_mask (the combine's weight; the value the masked affinity row that
// bw_count_kernel reads holds for it, a row the fused flow never needs, since its scaling is
// after the down GEMM and its combine reads these pairs); each nonzero affinity sets bit t % 64 of the
// token's 64-token chunk mask of its expert, chunk_masks[t / 64][e] (zeroed by the logits
// kernel; an OR commutes, so the masks are those bw_count_kernel writes).  The workgroups
// also fill token_position_to_id with -1.  P: values per lane.
constexpr int kPfTopkTok = 4;
template <int P>
__global__ void __launch_bounds__(256) pf_topk_kernel(
    const float* __restrict__ part, const void* __restrict__ bias, int bias_dt, int bias_rnd,
    int logit_rnd, int T, int E, int K, int act, int act_first, int renorm, float renorm_eps,
    int rnd, const uint8_t* __restrict__ pmask, int32_t* __restrict__ sel, float* __restrict__ val,
    unsigned long long* __restrict__ chunk_masks, int32_t* __restrict__ tp2id,
    int64_t n_slots) {
  const int tid = threadIdx.x, lane = tid & 63, b = blockIdx.x;
  for (int64_t i = (int64_t)b * 256 + tid; i < n_slots; i += (int64_t)gridDim.x * 256)
    tp2id[i] = -1;
  const int t = b * kPfTopkTok + wave_id();
  if (t >= T) return;
  const size_t TE = (size_t)T * E;
  float v[P];
  // every load issued first (lanes past E read expert E - 1 and are dropped), then the sums
  float pv[P][kPfParts], bv[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int ec = min(lane + 64 * i, E - 1);
    const size_t o = (size_t)t * E + ec;
#pragma unroll
    for (int q = 0; q < kPfParts; ++q) pv[i][q] = part[q * TE + o];
    bv[i] = load_opt_f32(bias, ec, bias_dt, part);
  }
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int e = lane + 64 * i;
    float r = -INFINITY;
    if (e < E) {
      float sum = pv[i][0];
#pragma unroll
      for (int q = 1; q < kPfParts; ++q) sum += pv[i][q];
      if (bias) sum += round_to(bv[i], bias_rnd);
      r = round_to(sum, logit_rnd);
    }
    v[i] = r;
  }
  int sel_idx[8];
  float out[8];
  topk_row_wave<P>(v, E, K, act, act_first, renorm, renorm_eps, rnd, sel_idx, out);
  const float pm = pmask ? (pmask[t] ? 1.0f : 0.0f) : 1.0f;
  unsigned long long* mk = chunk_masks + (size_t)(t / kPfTok) * E;
  const unsigned long long bit = 1ull << (t % kPfTok);
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int e = lane + 64 * i;
    if (e >= E) break;
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < K && sel_idx[k] == e) a = out[k];
    if (a != 0.0f) atomicOr(mk + e, bit);
  }
  if (lane < K) {
    int si = -1;
    float sv = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k == lane) {
        si = (sel_idx[k] >= 0 && sel_idx[k] < E && out[k] != 0.0f) ? sel_idx[k] : -1;
        sv = out[k];
      }
    sel[(size_t)t * K + lane] = si;
    val[(size_t)t * K + lane] = pmask ? sv * pm : sv;
  }
}

// The mapping's placement, one workgroup of 1024 threads per 64-token chunk c, and one
// more (c = n_chunks) for the schedule.  Every workgroup reads all chunk masks: tot[e] =
// the expert's tokens (integer sums, so the order of the LDS atomics is free), then scans
// the experts' block counts into the first slot of each run, expert_pos[e] (as
// bw_scan_body).  A chunk's workgroup also sums pre[e] = the expert's tokens in chunks
// before c, keeps its own chunk's masks in LDS and writes its chunk's pairs: slot =
// expert_pos[e] + pre[e] + (the expert's tokens below t in the chunk), the slot
// bw_scatter_kernel gives them, and tslot[t][k] = that slot (-1: none), the pair list the
// combine reads; the chunk's selections are loaded with the masks, so no global load
// waits behind the scan.  The schedule's workgroup writes block_to_expert[n] = #{e < E - 1
// : n >= cum[e]} and the schedule of the GEMMs' M-tile groups: M-tile mt lies in block
// n = 128 mt / B of expert e = block_to_expert[n], whose real slots come first,
// clamp(tot[e] - (n - first block of e) B, 0, B) of them; the tile holds r = clamp(that -
// 128 i, 0, 128) (i = its place in the block) and its weight (16-slot subtiles whose first
// slot is real) is ceil(r / 16): the weight cte_tile_order_kernel reads off
// token_position_to_id.  Dynamic LDS: max(5 B per M-tile, 8 B per expert).
__global__ void __launch_bounds__(kOrderThreads) pf_place_kernel(
    const int32_t* __restrict__ sel, const unsigned long long* __restrict__ chunk_masks, int T,
    int E, int K, int n_chunks, int B, int N, int G, int32_t* __restrict__ tp2id,
    int64_t n_slots, int32_t* __restrict__ tslot, int32_t* __restrict__ block_to_expert,
    int2* __restrict__ order) {
  static_assert(kOrderThreads == 1024, "one expert per thread in the block scan");
  static_assert(kPfTok * 8 <= kOrderThreads, "one pair of the chunk per thread");
  extern __shared__ __attribute__((aligned(16))) uint8_t order_dyn[];
  __shared__ int tot[kMaxE], pre[kMaxE], cum[kMaxE], pos0[kMaxE], wsum[16];
  __shared__ OrderLds L;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = blockIdx.x;
  const bool place = c < n_chunks;
  unsigned long long* own = reinterpret_cast<unsigned long long*>(order_dyn);
  // this thread's pair of the chunk (token c * 64 + tid / K, selection tid % K)
  const int tl = tid / K, tp = c * kPfTok + tl;
  const bool has_pair = place && tid < kPfTok * K && tp < T;
  const int xs = place ? sel[has_pair ? (size_t)tp * K + tid % K : 0] : -1;
  for (int e = tid; e < E; e += 1024) tot[e] = pre[e] = 0;
  __syncthreads();
  // All masks, eight per thread in flight at a time.
  const int nm = n_chunks * E;
  for (int i0 = 0; i0 < nm; i0 += 8 * 1024) {
    unsigned long long m[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * 1024 + tid;
      m[u] = i < nm ? chunk_masks[i] : 0ull;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * 1024 + tid;
      const int n = __popcll(m[u]);
      if (place && i / E == c) own[i % E] = m[u];
      if (n) {
        const int e = i % E;
        atomicAdd(&tot[e], n);
        if (i / E < c) atomicAdd(&pre[e], n);
      }
    }
  }
  __syncthreads();
  // Inclusive scan of the block counts over experts: wave scan, then across waves.
  const int e = tid;
  const int nb = e < E ? (tot[e] + B - 1) / B : 0;
  int v = nb;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(v, off);
    if (lane >= off) v += o;
  }
  if (lane == 63) wsum[wave] = v;
  __syncthreads();
  for (int w = 0; w < wave; ++w) v += wsum[w];
  if (e < E) {
    cum[e] = v;
    pos0[e] = (v - nb) * B;
  }
  __syncthreads();
  if (place) {
    if (has_pair) {
      int32_t sl = -1;
      if (xs >= 0) {
        const unsigned long long below = (tl == 0) ? 0ull : (~0ull >> (64 - tl));
        const int64_t pos = (int64_t)pos0[xs] + pre[xs] + __popcll(own[xs] & below);
        if (pos < n_slots) {
          tp2id[pos] = tp;
          sl = (int32_t)pos;
        }
      }
      tslot[(size_t)tp * K + tid % K] = sl;
    }
    return;
  }
  // The schedule's workgroup: block_to_expert and the schedule.
  auto expert_of_block = [&](int n) {  // #{e < E - 1 : n >= cum[e]} (cum non-decreasing)
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (cum[mid] <= n) lo = mid + 1;
      else hi = mid;
    }
    return lo;
  };
  for (int n = tid; n < N; n += 1024) block_to_expert[n] = expert_of_block(n);
  const int n_mtiles = N * (B / kPM), per = B / kPM;
  int32_t* s_e = reinterpret_cast<int32_t*>(order_dyn);
  uint8_t* s_w = order_dyn + 4 * (size_t)n_mtiles;
  for (int mt = tid; mt < n_mtiles; mt += 1024) {
    const int n = mt / per, i = mt - n * per;
    const int x = expert_of_block(n);
    const int nbx = (tot[x] + B - 1) / B;
    const int first = cum[x] - nbx;
    const int in_block = min(max(tot[x] - (n - first) * B, 0), B);
    const int r = min(max(in_block - i * kPM, 0), kPM);
    s_w[mt] = (uint8_t)((r + 15) / 16);
    s_e[mt] = x;
  }
  __syncthreads();
  order_pass(s_w, s_e, n_mtiles / G, G, order, L);
}

struct PfWs {
  float *part, *val;
  int32_t *sel, *tslot, *tp2id, *b2e;
  unsigned long long* masks;
  int2* order;
  char* cte;
  size_t cte_bytes;
};

static size_t pf_carve(void* base, size_t cap, int64_t T, int64_t H, int64_t I, int64_t E, int K,
                       int64_t B, PfWs* w) {
  Carver cv(base, cap);
  PfWs c;
  const int64_t nch = (T + kPfTok - 1) / kPfTok;
  const int64_t nb = blockwise_n_blocks(T, E, K, B);
  c.part = cv.take<float>(kPfParts * T * E);
  c.sel = cv.take<int32_t>(T * K);
  c.val = cv.take<float>(T * K);
  c.tslot = cv.take<int32_t>(T * K);
  c.masks = cv.take<unsigned long long>(nch * E);
  c.tp2id = cv.take<int32_t>(nb * B);
  c.b2e = cv.take<int32_t>(nb);
  c.order = cv.take<int2>(nb * B / kPM);
  c.cte_bytes = mxmoe_moe_cte_workspace_bytes(T, H, I, E, B, nb, MXMOE_SCALE_POST);
  c.cte = cv.take<char>(c.cte_bytes);
  if (w) *w = c;
  return cv.off + 256;
}

template <int ETW>
static void launch_pf_logits(const RouterSpec& r, dim3 g, int T, int H, int E, float* part,
                             unsigned long long* masks, hipStream_t s) {
#define MXMOE_PFL(XF, WF, OP)                                                           \
  hipLaunchKernelGGL((pf_logits_kernel<ETW, XF, WF, OP>), g, dim3(256), 0, s, r.x, r.w, T, H, \
                     E, part, masks)
  const bool xh = r.x_dt == kF16, wh = r.w_dt == kF16;
  if (r.op == kOpF16) {
    if (xh && wh) MXMOE_PFL(true, true, kOpF16);
    else if (xh) MXMOE_PFL(true, false, kOpF16);
    else if (wh) MXMOE_PFL(false, true, kOpF16);
    else MXMOE_PFL(false, false, kOpF16);
  } else if (r.op == kOpExact && wh) {
    MXMOE_PFL(false, true, kOpExact);
  } else if (wh) {
    MXMOE_PFL(false, true, kOpBF16);
  } else {
    MXMOE_PFL(false, false, kOpBF16);
  }
#undef MXMOE_PFL
}

}  // namespace mxmoe

using namespace mxmoe;

extern "C" size_t mxmoe_moe_prefill_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                                                    int top_k, int64_t block_size) {
  if (T < 1 || E < 1 || top_k < 1 || block_size < kPM) return 256;
  return pf_carve(nullptr, ~(size_t)0, T, H, I, E, top_k, block_size, nullptr);
}

extern "C" int mxmoe_moe_prefill(const uint16_t* x, const void* router_w, int router_w_dtype,
                                 const void* router_b, int router_b_dtype, int router_act,
                                 int act_before_topk, int renorm, float renorm_eps,
                                 int router_compute_dtype, const uint8_t* padding_mask,
                                 const uint8_t* gu_q, const uint8_t* gu_s, const uint8_t* dn_q,
                                 const uint8_t* dn_s, int weight_fmt, const uint16_t* gu_bias,
                                 const uint16_t* dn_bias, int64_t T, int64_t H, int64_t I,
                                 int64_t E, int top_k, int64_t block_size, int act,
                                 const float* clamps, int out_f32, void* out, void* workspace,
                                 size_t workspace_bytes, void* const* stage_events,
                                 void* stream) {
  clear_error();
  MXMOE_REQUIRE(x && router_w && gu_q && gu_s && dn_q && dn_s && out && workspace,
                "moe_prefill: null pointer");
  MXMOE_REQUIRE(weight_fmt == MXMOE_WFMT_MXFP4 || weight_fmt == MXMOE_WFMT_MXFP8,
                "moe_prefill: weight format %d must be MXFP4 or MXFP8", weight_fmt);
  MXMOE_REQUIRE(T >= 1 && E >= 1 && E <= kMaxE && top_k >= 1 && top_k <= 8 && top_k <= E,
                "moe_prefill: T=%lld E=%lld top_k=%d out of range (E <= %d, top_k <= 8)",
                (long long)T, (long long)E, top_k, kMaxE);
  MXMOE_REQUIRE(H >= 32 && H % 32 == 0, "moe_prefill: H=%lld must be a positive multiple of 32",
                (long long)H);
  MXMOE_REQUIRE(block_size >= kPM && block_size % kPM == 0,
                "moe_prefill: block_size=%lld must be a multiple of 128", (long long)block_size);
  MXMOE_REQUIRE(router_act == MXMOE_ROUTER_SOFTMAX || router_act == MXMOE_ROUTER_SIGMOID,
                "moe_prefill: unknown router activation %d", router_act);
  MXMOE_REQUIRE(router_compute_dtype >= kF32 && router_compute_dtype <= kBF16,
                "moe_prefill: router compute dtype %d unknown", router_compute_dtype);
  RouterSpec r;
  r.x = x;
  r.x_dt = kBF16;
  r.w = static_cast<const uint16_t*>(router_w);
  r.w_dt = router_w_dtype;
  r.bias = router_b;
  r.bias_dt = router_b_dtype;
  if (router_compute_dtype == kF32)
    r.op = router_w_dtype == kF16 ? kOpExact : kOpBF16;  // every product exact, as in fp32
  else
    r.op = router_compute_dtype == kF16 ? kOpF16 : kOpBF16;
  r.bias_rnd = r.logit_rnd = r.act_rnd = router_compute_dtype;
  int rc = router_check(r);
  if (rc) return rc;
  const int64_t n_blocks = blockwise_n_blocks(T, E, top_k, block_size);
  const int64_t n_slots = n_blocks * block_size, n_mtiles = n_slots / kPM;
  MXMOE_REQUIRE(n_mtiles <= kPfMaxTiles,
                "moe_prefill: %lld slots exceed the %d M-tiles of 128 slots one call schedules",
                (long long)n_slots, kPfMaxTiles);
  MXMOE_REQUIRE((int64_t)kPfParts * T * E < ((int64_t)1 << 31),
                "moe_prefill: %lld tokens x %lld experts exceed one call", (long long)T,
                (long long)E);
  const size_t need = pf_carve(nullptr, ~(size_t)0, T, H, I, E, top_k, block_size, nullptr);
  if (workspace_bytes < need)
    return set_error(MXMOE_E_WORKSPACE, "moe_prefill: workspace %zu < %zu", workspace_bytes,
                     need);
  PfWs w;
  pf_carve(workspace, workspace_bytes, T, H, I, E, top_k, block_size, &w);
  hipStream_t s = as_stream(stream);
  const int nch = (int)((T + kPfTok - 1) / kPfTok);
  mark_event(stage_events, 0, s);
  if (E <= 64)
    launch_pf_logits<1>(r, dim3((unsigned)nch, (unsigned)((E + 63) / 64), kPfParts), (int)T,
                        (int)H, (int)E, w.part, w.masks, s);
  else
    launch_pf_logits<2>(r, dim3((unsigned)nch, (unsigned)((E + 127) / 128), kPfParts), (int)T,
                        (int)H, (int)E, w.part, w.masks, s);
  const int af = act_before_topk ? 1 : 0, rn = renorm ? 1 : 0;
  const dim3 tg((unsigned)((T + kPfTopkTok - 1) / kPfTopkTok));
#define MXMOE_PFT(P)                                                                          \
  hipLaunchKernelGGL(pf_topk_kernel<P>, tg, dim3(256), 0, s, w.part, r.bias, r.bias_dt,       \
                     r.bias_rnd, r.logit_rnd, (int)T, (int)E, top_k, router_act, af, rn,       \
                     renorm_eps, r.act_rnd, padding_mask, w.sel, w.val, w.masks,      \
                     w.tp2id, n_slots)
  switch (topk_per_lane((int)E)) {
    case 1: MXMOE_PFT(1); break;
    case 2: MXMOE_PFT(2); break;
    case 4: MXMOE_PFT(4); break;
    case 8: MXMOE_PFT(8); break;
    default: MXMOE_PFT(16); break;
  }
#undef MXMOE_PFT
  const int G = prefill_group_tiles(block_size);
  const size_t place_lds = std::max((size_t)n_mtiles * 5, (size_t)E * 8);
  hipLaunchKernelGGL(pf_place_kernel, dim3((unsigned)nch + 1), dim3(kOrderThreads), place_lds, s, w.sel, w.masks, (int)T, (int)E, top_k, nch,
                     (int)block_size, (int)n_blocks, G, w.tp2id, n_slots, w.tslot, w.b2e,
                     w.order);
  rc = check_launch("moe_prefill front end");
  if (rc) return rc;
  void* cte_ev[4];
  void* const* cev = nullptr;
  if (stage_events) {
    for (int i = 0; i < 4; ++i) cte_ev[i] = stage_events[i + 1];
    cev = cte_ev;
  }
  const CteTokPairs pairs = {w.tslot, w.sel, w.val, top_k};
  return cte_run(x, nullptr, gu_q, gu_s, dn_q, dn_s, weight_fmt, gu_bias, dn_bias, nullptr,
                 w.tp2id, w.b2e, n_blocks, block_size, T, H, I, E, act, clamps,
                 MXMOE_SCALE_POST, out_f32, out, w.cte, w.cte_bytes, cev, w.order, s, &pairs);
}
