// Decode (token generation) expert MLP: weight-streaming grouped GEMMs over the
// experts the batch selected, fp32 arithmetic as in the reference decode flow.
//
//   front end  (mxmoe_moe_decode, T <= 128) router logits split over many workgroups,
//              then the top-k of every token (one workgroup per 16 tokens) and the
//              routing below; up to 16 tokens, one workgroup takes both
//   route      one workgroup: per-expert slot lists (tokens ascending inside an
//              expert), the list of active experts, per-token slots sorted by expert
//   gate_up    streaming kernel, one wave per item (active expert, 4 row groups =
//              2 gate/up pairs; one pair in the smallest batches): the item's packed
//              weights stream over all of K
//              through a register ring of D chunks; fused bias, clamps and
//              activation; the fp32 activation is stored as a bf16 (hi, lo) pair
//   down       the same streaming kernel over (active expert, 4 row groups of H, or 8
//              when enough experts are active to fill the chip with half as many
//              waves); the fp32 activation as hi + lo: a tile of at most 8 tokens puts
//              the tokens' hi and lo rows side by side in one MFMA, a larger one takes
//              two MFMAs (hi, lo) per product; fp32 bias
//   combine    out[t] = bf16(sum over the token's experts in ascending id of y * w)
// Items are independent and each writes its own outputs.
#include <math.h>

#include <mutex>

#include "capi_util.h"
#include "common.h"
#include "router_dev.h"

namespace mxmoe {

constexpr int kTkgMaxT = 1024;
constexpr int kTkgMaxE = 512;

// Routing of a decode batch by one workgroup of 1024 threads (thread t = token t):
// per-expert slot lists with tokens ascending inside an expert (ranks from wave-wide
// 64-bit masks and popcounts), the ascending list of active experts, and per token its
// slots and weights sorted by expert id.
__device__ __forceinline__ void tkg_route_block(
    const int32_t* __restrict__ topk_idx, const float* __restrict__ topk_val, int T, int K, int E,
    int scale_mode, int32_t* __restrict__ expert_off, int32_t* __restrict__ active,
    int32_t* __restrict__ n_active, int32_t* __restrict__ slot_tok, int32_t* __restrict__ tok_slot,
    float* __restrict__ tok_w, int32_t* __restrict__ tiles, int32_t* __restrict__ n_tiles) {
  __shared__ unsigned long long masks[16][kTkgMaxE];
  __shared__ int off[kTkgMaxE];
  __shared__ int wsum[16], wact[16], wtile[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = lane; e < E; e += 64) masks[wave][e] = 0ull;  // the rows' first E entries
  __syncthreads();
  int ids[8];
  float vals[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    ids[k] = -1;
    vals[k] = 0.f;
  }
  if (tid < T) {
    // every entry loaded first (entries past K re-read entry 0), so that the loads issue
    // together instead of one round trip per entry
    int ei[8];
    float vi[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const size_t i = (size_t)tid * K + (k < K ? k : 0);
      ei[k] = topk_idx[i];
      vi[k] = topk_val[i];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k >= K) break;
      int e = ei[k];
      if (e < 0 || e >= E) e = -1;
      // A repeated expert id counts once (its last value, as a scatter would keep).
      for (int j = 0; j < k; ++j)
        if (ids[j] == e) ids[j] = -1;
      ids[k] = e;
      vals[k] = vi[k];
      if (e >= 0) atomicOr(&masks[wave][e], 1ull << lane);
    }
  }
  __syncthreads();
  // Counts -> exclusive offsets and the active-expert list (ascending id).
  int cnt = 0;
  if (tid < E)
    for (int w = 0; w < 16; ++w) cnt += __popcll(masks[w][tid]);
  // Token tiles: 16 of an expert's tokens each (the work unit of the one-tile decode
  // kernels, so that an expert with many tokens is spread over several waves).
  const int ntl = (cnt + 15) >> 4;
  int v = cnt, a = cnt > 0 ? 1 : 0, tl = ntl;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int pv = __shfl_up(v, o), pa = __shfl_up(a, o), pt = __shfl_up(tl, o);
    if (lane >= o) {
      v += pv;
      a += pa;
      tl += pt;
    }
  }
  if (lane == 63) {
    wsum[wave] = v;
    wact[wave] = a;
    wtile[wave] = tl;
  }
  __syncthreads();
  int pv = 0, pa = 0, pt = 0;
  for (int w = 0; w < wave; ++w) {
    pv += wsum[w];
    pa += wact[w];
    pt += wtile[w];
  }
  v += pv;
  a += pa;
  tl += pt;
  if (tid < E) {
    off[tid] = v - cnt;
    expert_off[tid] = v - cnt;
    if (cnt > 0) active[a - 1] = tid;
    // (expert, first slot, tokens) per 16-token tile: one load gives an item all it needs
    for (int j = 0; j < ntl; ++j)
      reinterpret_cast<int4*>(tiles)[tl - ntl + j] =
          make_int4(tid, v - cnt + 16 * j, min(16, cnt - 16 * j), 0);
  }
  if (tid == E - 1) {
    expert_off[E] = v;
    *n_active = a;
    *n_tiles = tl;
  }
  __syncthreads();
  if (tid >= T) return;
  const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  // The token's selections in ascending expert id: selection k goes to position
  // #{valid j : ids[j] < ids[k]} (ids are distinct); unused positions get -1.
  int n = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) n += (k < K && ids[k] >= 0) ? 1 : 0;
  for (int k = n; k < K; ++k) {
    tok_slot[(size_t)tid * K + k] = -1;
    tok_w[(size_t)tid * K + k] = 0.f;
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k >= K) break;
    const int e = ids[k];
    if (e < 0) continue;
    int r = off[e];
    for (int w = 0; w < wave; ++w) r += __popcll(masks[w][e]);
    r += __popcll(masks[wave][e] & below);
    slot_tok[r] = tid;
    int pos = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) pos += (j < K && ids[j] >= 0 && ids[j] < e) ? 1 : 0;
    tok_slot[(size_t)tid * K + pos] = r;
    tok_w[(size_t)tid * K + pos] =
        (scale_mode == MXMOE_SCALE_NO) ? (vals[k] > 0.f ? 1.f : 0.f) : vals[k];
  }
}

__global__ void __launch_bounds__(1024) tkg_route_kernel(
    const int32_t* __restrict__ topk_idx, const float* __restrict__ topk_val, int T, int K, int E,
    int scale_mode, int32_t* __restrict__ expert_off, int32_t* __restrict__ active,
    int32_t* __restrict__ n_active, int32_t* __restrict__ slot_tok, int32_t* __restrict__ tok_slot,
    float* __restrict__ tok_w, int32_t* __restrict__ tiles, int32_t* __restrict__ n_tiles) {
  tkg_route_block(topk_idx, topk_val, T, K, E, scale_mode, expert_off, active, n_active, slot_tok,
                  tok_slot, tok_w, tiles, n_tiles);
}

// Decode front end for small batches: router logits as 16-token x 16-expert MFMA tiles
// whose K reduction is split over kFrontSlices workgroups (so the router weights stream
// through many CUs), then the partial sums added, the top-k of every token and the
// routing: one workgroup for all three up to 16 tokens, else a top-k workgroup per 16
// tokens and the routing kernel.
constexpr int kFrontMaxT = 128;  // larger batches take the standalone router kernels
constexpr int kFrontSlices = 4;
constexpr int kFrontWaves = 16 / kFrontSlices;  // waves per workgroup

// Wave w of slice s (blockIdx.z) takes the 128-wide K chunks gw, gw + 16, ... with
// gw = s * kFrontWaves + w; the workgroup adds its waves' sums in wave order and
// stores partial s [kFrontSlices, T, E].  A = router rows (experts), B = tokens.
// WSPLIT: the router weights are fp16, each split exactly into bf16 hi + lo (two MFMAs),
// so the products are those of the fp32 matmul of the reference flow.
template <bool WSPLIT>
__global__ void __launch_bounds__(64 * kFrontWaves) front_logits_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, float* __restrict__ part,
    int T, int H, int E) {
  __shared__ f32x4 red[kFrontWaves][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int gw = blockIdx.z * kFrontWaves + wave;
  const int q = lane >> 4, r16 = lane & 15;
  const int t0 = blockIdx.x * 16, e0 = blockIdx.y * 16;
  const int nc = (H + 127) / 128, tail_q = (H % 128) / 32;
  const uint16_t* xr = x + (size_t)min(t0 + r16, T - 1) * H;
  const uint16_t* wr = w + (size_t)min(e0 + r16, E - 1) * H;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  for (int c = gw; c < nc; c += 16) {
    const bool ok = (c < H / 128) || (q < tail_q);
    const int k0 = ok ? c * 128 + q * 32 : 0;
    u32x4 xv[4], wv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xv[j] = *reinterpret_cast<const u32x4*>(xr + k0 + 8 * j);
      wv[j] = *reinterpret_cast<const u32x4*>(wr + k0 + 8 * j);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xv[j] = ok ? xv[j] : zero4;
      if constexpr (WSPLIT) {
        bf16x8 hi, lo;
        f16x8_split_bf16(wv[j], hi, lo);
        acc = mfma16(hi, as_bf16x8(xv[j]), acc);
        acc = mfma16(lo, as_bf16x8(xv[j]), acc);
      } else {
        acc = mfma16(as_bf16x8(wv[j]), as_bf16x8(xv[j]), acc);
      }
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  for (int o = tid; o < 256; o += 64 * kFrontWaves) {
    const int l = o & 63, i = o >> 6;  // D lane l, element i: expert 4(l/16)+i, token l%16
    float v = 0.f;
#pragma unroll
    for (int wv = 0; wv < kFrontWaves; ++wv) v += red[wv][l][i];
    const int tok = t0 + (l & 15), ex = e0 + 4 * (l >> 4) + i;
    if (tok < T && ex < E) part[((size_t)blockIdx.z * T + tok) * E + ex] = v;
  }
}

// One workgroup of 1024 threads: logits = partials added in slice order + bias (stored
// to logits), the top-k of token t by the 16-lane row t % 64 (lane j holds experts
// j, j+16, ...), then the routing of the batch from the selections kept in LDS.
template <int PER>
__global__ void __launch_bounds__(1024) front_route_kernel(
    const float* __restrict__ part, const void* __restrict__ bias, int bias_dt,
    float* __restrict__ logits, int T, int E, int K, int act, int act_first, int renorm,
    float renorm_eps, int scale_mode, int32_t* __restrict__ topk_idx_out,
    int32_t* __restrict__ expert_off, int32_t* __restrict__ active, int32_t* __restrict__ n_active,
    int32_t* __restrict__ slot_tok, int32_t* __restrict__ tok_slot, float* __restrict__ tok_w,
    int32_t* __restrict__ tiles, int32_t* __restrict__ n_tiles) {
  __shared__ int32_t s_idx[kFrontMaxT * 8];
  __shared__ float s_val[kFrontMaxT * 8];
  const int tid = threadIdx.x, row = tid >> 4, j = tid & 15;
  // Every load of a token is issued before any is used (addresses clamped into the row),
  // so the partial sums and the bias arrive in one round trip.
  float bval[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) bval[i] = load_opt_f32(bias, min(j + 16 * i, E - 1), bias_dt, part);
  for (int t = row; t < T; t += 64) {
    float pv[kFrontSlices][PER];
#pragma unroll
    for (int sl = 0; sl < kFrontSlices; ++sl)
#pragma unroll
      for (int i = 0; i < PER; ++i)
        pv[sl][i] = part[((size_t)sl * T + t) * E + min(j + 16 * i, E - 1)];
    float v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      float a = pv[0][i];
#pragma unroll
      for (int sl = 1; sl < kFrontSlices; ++sl) a += pv[sl][i];
      a += bval[i];
      const int e = j + 16 * i;
      if (e < E) logits[(size_t)t * E + e] = a;
      v[i] = e < E ? a : -INFINITY;
    }
    int sel_idx[8];
    float out[8];
    topk_row_group<16, PER>(v, E, K, act, act_first, renorm, renorm_eps, kF32, sel_idx, out);
    if (j < K) {
      int si = 0;
      float so = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k == j) {
          si = sel_idx[k];
          so = out[k];
        }
      s_idx[t * K + j] = si;
      s_val[t * K + j] = so;
      if (topk_idx_out) topk_idx_out[t * K + j] = si;
    }
  }
  __syncthreads();
  tkg_route_block(s_idx, s_val, T, K, E, scale_mode, expert_off, active, n_active, slot_tok,
                  tok_slot, tok_w, tiles, n_tiles);
}

// The top-k of 16 tokens per workgroup of 256 threads (token t by the 16-lane row t % 16,
// as in front_route_kernel), the selections stored for the routing kernel: the top-k
// work, the front end's VALU-bound part, then spreads over T / 16 CUs.
template <int PER>
__global__ void __launch_bounds__(256) front_topk_kernel(
    const float* __restrict__ part, const void* __restrict__ bias, int bias_dt,
    float* __restrict__ logits, int T, int E, int K, int act, int act_first, int renorm,
    float renorm_eps, int32_t* __restrict__ topk_idx, float* __restrict__ topk_val) {
  const int tid = threadIdx.x, j = tid & 15;
  const int t = blockIdx.x * 16 + (tid >> 4);
  if (t >= T) return;  // whole 16-lane rows
  float bval[PER];
  float pv[kFrontSlices][PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) bval[i] = load_opt_f32(bias, min(j + 16 * i, E - 1), bias_dt, part);
#pragma unroll
  for (int sl = 0; sl < kFrontSlices; ++sl)
#pragma unroll
    for (int i = 0; i < PER; ++i)
      pv[sl][i] = part[((size_t)sl * T + t) * E + min(j + 16 * i, E - 1)];
  float v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    float a = pv[0][i];
#pragma unroll
    for (int sl = 1; sl < kFrontSlices; ++sl) a += pv[sl][i];
    a += bval[i];
    const int e = j + 16 * i;
    if (e < E) logits[(size_t)t * E + e] = a;
    v[i] = e < E ? a : -INFINITY;
  }
  int sel_idx[8];
  float out[8];
  topk_row_group<16, PER>(v, E, K, act, act_first, renorm, renorm_eps, kF32, sel_idx, out);
  if (j < K) {
    int si = 0;
    float so = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k == j) {
        si = sel_idx[k];
        so = out[k];
      }
    topk_idx[(size_t)t * K + j] = si;
    topk_val[(size_t)t * K + j] = so;
  }
}

// Experts per lane of a 16-lane row: the template argument of front_route_kernel.
inline int front_per_lane(int E) {
  const int per = (E + 15) / 16;
  return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : per <= 16 ? 16 : 32;
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

// Registers of one K chunk of a streamed tile: R weight row groups (16 B per lane
// each), their scale bytes (one 32-bit word per lane and quad of row groups: the
// packed scales keep quads together) and NT token tiles of activations (4 x 16 B per
// lane; with SPLIT a second (lo) copy).
template <int R, int NT, bool SPLIT>
struct ChunkFrag {
  static_assert(R % 4 == 0 || R == 2, "a streamed tile is whole quads of row groups or a pair");
  u32x4 w[R];
  uint32_t s[(R + 3) / 4];
  u32x4 b[NT][4];
  u32x4 b2[SPLIT ? NT : 1][4];
};

struct StreamGeom {
  const uint8_t* wq;  // first row group of the tile
  const uint8_t* ws;  // the tile's first quad of scales
  uint32_t rg_bytes, q_bytes;
  int rv;             // valid row groups in the tile (<= R)
  int nfull, tail_q;  // full 128-wide chunks, 32-blocks in the partial last chunk
  int cb, ce;         // the K chunks [cb, ce) this tile streams
  int sb;             // byte of the tile's first row group in its quad's scale word
};

// Plain loads only, so nothing waits on them before their use: lanes past K in a
// partial last chunk re-read lane 0's bytes of the same chunk, row groups past the
// tile re-read its last valid one, and lanes of absent tokens read a valid row of
// the expert (the same address as their neighbours, so the requests coalesce).
// mma_chunk gives the lanes past K a zero scale, so their weights dequantize to
// exact zeros; row groups past the tile and columns of absent tokens are computed
// and never stored.
template <int R, int NT, bool SPLIT>
__device__ __forceinline__ void load_chunk(ChunkFrag<R, NT, SPLIT>& f, int c, const StreamGeom& g,
                                           const char* b1, const char* b2,
                                           const uint32_t* row_off) {
  const int lane = threadIdx.x & 63, q = lane >> 4;
  const bool ok = (c < g.nfull) || (q < g.tail_q);
  const uint32_t lo = ok ? (uint32_t)lane : 0u;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t rr = r < g.rv ? r : g.rv - 1;
    // One wave-uniform base and a 32-bit offset per lane.  Weights are read once per
    // step: non-temporal, so they do not evict the activations and scales that
    // neighbouring waves re-read from the caches.
    const uint32_t off = rr * g.rg_bytes + (uint32_t)c * 1024u + lo * 16u;
    f.w[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(g.wq + off));
  }
#pragma unroll
  for (int h = 0; h < (R + 3) / 4; ++h) {
    const uint32_t qq = 4 * h < g.rv ? h : 0;  // a partial last tile stays in its expert
    // Scales are read once per step too (non-temporal, about 2 % faster than cached).
    f.s[h] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(
        g.ws + qq * g.q_bytes + (uint32_t)c * 256u + lo * 4u));
  }
  const uint32_t k0b = ok ? (uint32_t)(c * 128 + q * 32) * 2u : 0u;  // byte offset in a row
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t off = row_off[t] + k0b + 16u * j;
      f.b[t][j] = *reinterpret_cast<const u32x4*>(b1 + off);
      if (SPLIT) f.b2[t][j] = *reinterpret_cast<const u32x4*>(b2 + off);
    }
  }
}

// No branches around the MFMAs: a branch join would make the compiler copy the
// accumulators between register files.
template <int R, int NT, bool SPLIT>
__device__ __forceinline__ void mma_chunk(const ChunkFrag<R, NT, SPLIT>& f, int c,
                                          const StreamGeom& g, f32x4 (&acc)[R][NT]) {
  // chunks at or past ce (the loop rounds up to whole rings) contribute exact zeros
  const bool ok =
      c < g.ce && ((c < g.nfull) || (c == g.nfull && ((threadIdx.x & 63) >> 4) < g.tail_q));
#pragma unroll
  for (int r = 0; r < R; ++r) {
    // a pair (R = 2) sits in one quad, from byte g.sb (0 or 2) of its scale word;
    // constant word indices keep the chunk in registers
    const uint32_t sw = f.s[R % 4 == 0 ? r / 4 : 0];
    const int sh = 8 * (R % 4 == 0 ? r % 4 : g.sb + r);
    const float sc = ok ? e8m0_to_f32((sw >> sh) & 0xffu) : 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x8 wf = dequant8(f.w[r][j], sc);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        acc[r][t] = mfma16(wf, as_bf16x8(f.b[t][j]), acc[r][t]);
        if (SPLIT) acc[r][t] = mfma16(wf, as_bf16x8(f.b2[t][j]), acc[r][t]);
      }
    }
    // One row group's conversions at a time: registers go to chunks in flight.
    __builtin_amdgcn_sched_barrier(0);
  }
}

// One wave streams an R-row-group tile over the K chunks [g.cb, g.ce), D chunks in
// flight.  Activation rows are b1 (and, with SPLIT, b2 for the lo parts) plus this
// lane's byte offset row_off[t] for token tile t (a valid row also for lanes without a
// token).
template <int R, int NT, bool SPLIT, int D>
__device__ __forceinline__ void stream_tile(const StreamGeom& g, const char* b1, const char* b2,
                                            const uint32_t* row_off, f32x4 (&acc)[R][NT]) {
  // Every ring slot is refilled right after its MFMAs, unconditionally (past the
  // end with the last chunk again, a cache hit), and the loop body has no branch:
  // a load whose issue depends on a branch would make the wait before a chunk's
  // MFMAs assume the shorter queue and drain the loads of the chunks behind it, and
  // a branch join around the MFMAs would copy the accumulators.  The loop covers
  // whole rings; chunks past ce add exact zeros.
  const int cl = g.ce > g.cb ? g.ce - 1 : g.cb;  // last chunk to (re)load
  ChunkFrag<R, NT, SPLIT> f[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load_chunk(f[d], g.cb + d < cl ? g.cb + d : cl, g, b1, b2, row_off);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int c = g.cb; c < g.ce; c += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      mma_chunk(f[d], c + d, g, acc);
      const int cn = c + d + D;
      load_chunk(f[d], cn < cl ? cn : cl, g, b1, b2, row_off);
      // Keep program order: the scheduler would otherwise hoist the refills above
      // the MFMAs and consume them in the same iteration, leaving nothing in flight.
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

struct TkgArgs {
  const uint16_t* x;       // gate_up: tokens [T, H]
  int T, S;                // tokens, routed slots (bounds of x and of h)
  const uint16_t* h_hi;    // down: activations [slots, I] (hi, lo)
  const uint16_t* h_lo;
  const uint8_t* wq;
  const uint8_t* ws;
  const uint16_t* bias;    // gate_up [E, 2, I]; down [E, H]; may be null
  const int32_t* expert_off;
  const int32_t* active;
  const int32_t* n_active;
  const int32_t* slot_tok;
  const int32_t* tiles;    // (expert, first slot, tokens, 0) per 16-token tile of the routed
                           // batch, and their count
  const int32_t* n_tiles;
  uint32_t lo_shift;       // down: bytes from h_hi to h_lo
  uint16_t* out_hi;        // gate_up: h (hi, lo)
  uint16_t* out_lo;
  float* y;                // down: [nq, slots, H] (K part q of every slot's output)
  float* part;             // gate_up with nq > 1: [nq, slots, 2I] raw K-part sums
  size_t part_stride;      // elements of one K part of y / part
  int nq, cpq;             // K parts of a row-group chunk, 128-wide chunks per part
  int H, I;
  ExpertParams p;
};

// One work item = (active expert, R row groups) of the projection GATE_UP selects:
// stream the item's packed weights against the expert's tokens, then the epilogue.
// gate_up items hold whole gate/up pairs (R even).
// PACK (down items of a tile of at most 8 tokens): the MFMA's 16 columns hold the
// tokens' hi activation rows (columns 0-7) and their lo rows (columns 8-15), so a
// product takes one MFMA and one activation load per lane instead of two; the epilogue
// adds column j + 8 to column j.  Without PACK a down item issues the hi and the lo MFMA.
template <int R, int NT, bool GATE_UP, int D, bool PACK = false>
__device__ __forceinline__ void tkg_item(const TkgArgs& a, int item, int ipe, int q = 0) {
  static_assert(!GATE_UP || R % 2 == 0, "gate_up items hold gate/up pairs");
  static_assert(!PACK || (!GATE_UP && NT == 1), "packed items are down items of one tile");
  constexpr bool SPLIT = !GATE_UP && !PACK;
  constexpr int TT = PACK ? 8 : 16;  // tokens per pass
  const int lane = threadIdx.x & 63;
  const int H = a.H, I = a.I;
  const int K = GATE_UP ? H : I;
  const int n_rg = GATE_UP ? (2 * I) / 16 : H / 16;
  const int nc = (K + 127) / 128;
  StreamGeom g;
  g.rg_bytes = (uint32_t)K * 8u;
  g.q_bytes = (uint32_t)K * 2u;
  g.nfull = K / 128;
  g.tail_q = (K % 128) / 32;
  const int ai = item / ipe, ri = item - ai * ipe;
  // K part q of the chunk: chunks [q * cpq, (q + 1) * cpq) (all of K when nq = 1)
  g.cb = q * a.cpq;
  g.ce = min(nc, g.cb + a.cpq);
  // Item metadata is wave-uniform: keep it in scalar registers.  With one token tile per
  // pass (NT = 1) an item is (token tile, row groups): an expert's 16-token tiles are
  // separate items; else (active expert, row groups), looping over the expert's tokens.
  int e, s0, ne;
  if constexpr (NT == 1) {
    const int4 tm = reinterpret_cast<const int4*>(a.tiles)[ai];
    e = __builtin_amdgcn_readfirstlane(tm.x);
    s0 = __builtin_amdgcn_readfirstlane(tm.y);
    ne = __builtin_amdgcn_readfirstlane(tm.z);
  } else {
    e = __builtin_amdgcn_readfirstlane(a.active[ai]);
    s0 = __builtin_amdgcn_readfirstlane(a.expert_off[e]);
    ne = __builtin_amdgcn_readfirstlane(a.expert_off[e + 1]) - s0;
  }
  const int rg0 = ri * R;
  g.wq = a.wq + ((size_t)e * n_rg + rg0) * (size_t)g.rg_bytes;
  g.ws = a.ws + ((size_t)e * ((n_rg + 3) / 4) + rg0 / 4) * (size_t)(2 * K);
  g.rv = min(R, n_rg - rg0);
  g.sb = rg0 % 4;
  const char* b1 = GATE_UP ? reinterpret_cast<const char*>(a.x)
                           : reinterpret_cast<const char*>(a.h_hi);
  const char* b2 = GATE_UP ? b1 : reinterpret_cast<const char*>(a.h_lo);
  // The item's biases, loaded before its weights stream (8-byte loads of 4 columns; their
  // latency then hides behind the stream instead of following it): gate_up [pair][gate,
  // up], down [row group].  A bias that is not 8-byte aligned is read in the epilogue.
  typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
  constexpr int NB = GATE_UP ? R : R;
  u16x4 bpre[NB];
  const bool use_bias = a.bias && (GATE_UP ? a.nq == 1 : q == 0);
  const bool bvec = use_bias && ((uintptr_t)a.bias & 7u) == 0;
#pragma unroll
  for (int j = 0; j < NB; ++j) bpre[j] = u16x4{0, 0, 0, 0};
  if (bvec) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      size_t idx;
      if constexpr (GATE_UP) {
        const int pp = (j / 2) * 2 < g.rv ? j / 2 : 0;  // pairs past the item: pair 0
        idx = (size_t)e * 2 * I + (j & 1 ? I : 0) + 8 * (rg0 + 2 * pp) + 4 * (lane >> 4);
      } else {
        const int r = j < g.rv ? j : 0;
        idx = (size_t)e * H + 16 * (rg0 + r) + 4 * (lane >> 4);
      }
      bpre[j] = *reinterpret_cast<const u16x4*>(a.bias + idx);
    }
  }
  auto bias_of = [&](int j, int i, size_t idx) -> float {
    return bvec ? bf16_bits_to_f32(bpre[j][i]) : bf16_bits_to_f32(a.bias[idx]);
  };
  for (int tb = 0; tb < ne; tb += TT * NT) {
    uint32_t row_off[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int li = tb + TT * t + (lane & (TT - 1));
      const int lr = li < ne ? li : tb;
      row_off[t] = GATE_UP ? (uint32_t)a.slot_tok[s0 + lr] * (uint32_t)(2 * H)
                           : (uint32_t)(s0 + lr) * (uint32_t)(2 * I);
      if (PACK && (lane & 8)) row_off[t] += a.lo_shift;  // columns 8-15: the lo rows
    }
    f32x4 acc[R][NT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    stream_tile<R, NT, SPLIT, D>(g, b1, b2, row_off, acc);
    if constexpr (PACK) {
      // y of token j = (hi sums, column j) + (lo sums, column j + 8), then the bias
      const int li = tb + (lane & 7);
      const size_t slot = (size_t)(s0 + (li < ne ? li : 0));
#pragma unroll
      for (int r = 0; r < R; ++r) {
        f32x4 v = acc[r][0];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] += __shfl_xor(v[i], 8);
        if (r >= g.rv || (lane & 8) || li >= ne) continue;
        const int n0 = 16 * (rg0 + r) + 4 * (lane >> 4);
        if (use_bias) {  // the first K part carries the bias
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] += bias_of(r, i, (size_t)e * H + n0 + i);
        }
        *reinterpret_cast<f32x4*>(a.y + q * a.part_stride + slot * H + n0) = v;
      }
      continue;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int li = tb + 16 * t + (lane & 15);
      if (li >= ne) continue;
      const size_t slot = (size_t)(s0 + li);
      if (GATE_UP && a.nq > 1) {
        // raw K-part sums; the activation kernel adds the parts in order, then the bias
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r >= g.rv) continue;
          const int rg = rg0 + r;  // even: gate rows, odd: up rows of columns 8 (rg & ~1)..
          const int col = (rg & 1 ? I : 0) + 8 * (rg & ~1) + 4 * (lane >> 4);
          *reinterpret_cast<f32x4*>(a.part + q * a.part_stride + slot * 2 * I + col) =
              acc[r][t];
        }
      } else if (GATE_UP) {
#pragma unroll
        for (int pp = 0; pp < R / 2; ++pp) {
          if (2 * pp >= g.rv) continue;
          const int col0 = 8 * (rg0 + 2 * pp) + 4 * (lane >> 4);  // 16 * pair index
          uint16_t hi[4], lo[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float gv = acc[2 * pp][t][i], uv = acc[2 * pp + 1][t][i];
            if (use_bias) {
              gv += bias_of(2 * pp, i, (size_t)e * 2 * I + col0 + i);
              uv += bias_of(2 * pp + 1, i, (size_t)e * 2 * I + I + col0 + i);
            }
            gv = clampf_ref(gv, a.p.gate_lo, a.p.gate_hi);
            uv = clampf_ref(uv, a.p.up_lo, a.p.up_hi);
            split_bf16(uv * act_f32(gv, a.p.act), hi[i], lo[i]);
          }
          *reinterpret_cast<u16x4*>(a.out_hi + slot * I + col0) = u16x4{hi[0], hi[1], hi[2], hi[3]};
          *reinterpret_cast<u16x4*>(a.out_lo + slot * I + col0) = u16x4{lo[0], lo[1], lo[2], lo[3]};
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r >= g.rv) continue;
          const int n0 = 16 * (rg0 + r) + 4 * (lane >> 4);
          f32x4 v = acc[r][t];
          if (use_bias) {  // the first K part carries the bias
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] += bias_of(r, i, (size_t)e * H + n0 + i);
          }
          *reinterpret_cast<f32x4*>(a.y + q * a.part_stride + slot * H + n0) = v;
        }
      }
    }
  }
}

__host__ __device__ inline int tkg_items_per_expert(int H, int I, bool gate_up, int R) {
  const int n_rg = gate_up ? (2 * I) / 16 : H / 16;
  return (n_rg + R - 1) / R;
}

// Grid dispatch: wave w of workgroup b takes work unit WPB * b + w, unit u = item * nq + q
// (the item's K part q; nq = 1: the whole item); the grid covers the most units a batch
// can have (every expert, or every possible token tile), waves past the batch's units
// return at once.  The hardware dispatcher hands a freed wave slot the next workgroup, so
// batches with more units than slots balance over the SIMDs as they stream.  One token
// tile per item keeps three waves per SIMD (168 registers).  Down items of one tile
// choose per item: packed hi/lo columns when the tile holds at most 8 tokens.
template <int R, int NT, bool GATE_UP, int D, int WPB>
__global__ void __launch_bounds__(64 * WPB)
    __attribute__((amdgpu_waves_per_eu(NT == 1 ? 3 : 1))) tkg_stream_kernel(TkgArgs a) {
  const int ipe = tkg_items_per_expert(a.H, a.I, GATE_UP, R);
  const int u = blockIdx.x * WPB + (WPB == 1 ? 0 : wave_id());
  if (u >= (NT == 1 ? *a.n_tiles : *a.n_active) * ipe * a.nq) return;
  const int item = u / a.nq;
  if constexpr (!GATE_UP && NT == 1) {
    const int ne =
        __builtin_amdgcn_readfirstlane(reinterpret_cast<const int4*>(a.tiles)[item / ipe].z);
    if (ne <= 8) {
      tkg_item<R, NT, GATE_UP, D, true>(a, item, ipe, u - item * a.nq);
      return;
    }
  }
  tkg_item<R, NT, GATE_UP, D>(a, item, ipe, u - item * a.nq);
}

// The gate_up epilogue of split-K batches: h = up' * act(gate') with gate' / up' the
// clamped sums of the nq K parts (added in order) plus the bias, stored as bf16 (hi, lo).
// Grid (column groups of 1024, slots of the largest batch); slots past the batch return.
__global__ void __launch_bounds__(256) tkg_act_kernel(TkgArgs a, int E) {
  const int slot = blockIdx.y;
  const int n_slots = a.expert_off[E];
  if (slot >= n_slots) return;
  const int I = a.I;
  const int c = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= I) return;
  // the slot's expert: experts' slots are contiguous and ascending
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.expert_off[mid] <= slot) lo = mid;
    else hi = mid - 1;
  }
  const int e = lo;
  f32x4 gv = {0.f, 0.f, 0.f, 0.f}, uv = {0.f, 0.f, 0.f, 0.f};
  for (int q = 0; q < a.nq; ++q) {
    const float* row = a.part + q * a.part_stride + (size_t)slot * 2 * I;
    gv += *reinterpret_cast<const f32x4*>(row + c);
    uv += *reinterpret_cast<const f32x4*>(row + I + c);
  }
  typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
  uint16_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float g = gv[i], u = uv[i];
    if (a.bias) {
      g += bf16_bits_to_f32(a.bias[(size_t)e * 2 * I + c + i]);
      u += bf16_bits_to_f32(a.bias[(size_t)e * 2 * I + I + c + i]);
    }
    g = clampf_ref(g, a.p.gate_lo, a.p.gate_hi);
    u = clampf_ref(u, a.p.up_lo, a.p.up_hi);
    split_bf16(u * act_f32(g, a.p.act), h[i], l[i]);
  }
  *reinterpret_cast<u16x4*>(a.out_hi + (size_t)slot * I + c) = u16x4{h[0], h[1], h[2], h[3]};
  *reinterpret_cast<u16x4*>(a.out_lo + (size_t)slot * I + c) = u16x4{l[0], l[1], l[2], l[3]};
}

// out[t, n] = bf16(sum_k y[slot(t, k), n] * w(t, k)), k in ascending expert order, each
// y the sum of its nq K parts in order.  KM (4 or 8) >= top-k: the token's slots and
// weights are loaded first (entries past K re-read entry 0), then the rows of K part 0 of
// every entry (an absent slot reads row 0), all in flight before the first is used; with
// a condition per entry the compiler waited for each load on its own.  KM = 0: any top-k,
// one entry at a time.
template <int KM>
__global__ void __launch_bounds__(256) tkg_combine_kernel(const float* __restrict__ y,
                                                          const int32_t* __restrict__ tok_slot,
                                                          const float* __restrict__ tok_w, int H,
                                                          int K, int nq, size_t part_stride,
                                                          uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int n = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (n >= H) return;
  typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
  if constexpr (KM == 0) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < K; ++k) {
      const int s = tok_slot[(size_t)t * K + k];
      if (s < 0) continue;
      const float w = tok_w[(size_t)t * K + k];
      f32x4 v = *reinterpret_cast<const f32x4*>(y + (size_t)s * H + n);
      for (int q = 1; q < nq; ++q) {
        const f32x4 vq = *reinterpret_cast<const f32x4*>(y + q * part_stride + (size_t)s * H + n);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = __fadd_rn(v[i], vq[i]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = __fadd_rn(acc[i], __fmul_rn(v[i], w));
    }
    *reinterpret_cast<u16x4*>(out + (size_t)t * H + n) =
        u16x4{f32_to_bf16_bits(acc[0]), f32_to_bf16_bits(acc[1]), f32_to_bf16_bits(acc[2]),
              f32_to_bf16_bits(acc[3])};
    return;
  }
  constexpr int KA = KM > 0 ? KM : 1;
  int sl[KA];
  float wt[KA];
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    const size_t i = (size_t)t * K + (k < K ? k : 0);
    sl[k] = tok_slot[i];
    wt[k] = tok_w[i];
  }
  f32x4 v[KA];
#pragma unroll
  for (int k = 0; k < KM; ++k)
    v[k] = *reinterpret_cast<const f32x4*>(y + (size_t)(sl[k] >= 0 ? sl[k] : 0) * H + n);
  if constexpr (KM == 4)
    asm volatile("" ::"v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]));
  else
    asm volatile("" ::"v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]),
                 "v"(v[6]), "v"(v[7]));
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    if (k >= K || sl[k] < 0) continue;
    f32x4 vk = v[k];
    for (int q = 1; q < nq; ++q) {
      const f32x4 vq =
          *reinterpret_cast<const f32x4*>(y + q * part_stride + (size_t)sl[k] * H + n);
#pragma unroll
      for (int i = 0; i < 4; ++i) vk[i] = __fadd_rn(vk[i], vq[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = __fadd_rn(acc[i], __fmul_rn(vk[i], wt[k]));
  }
  *reinterpret_cast<u16x4*>(out + (size_t)t * H + n) =
      u16x4{f32_to_bf16_bits(acc[0]), f32_to_bf16_bits(acc[1]), f32_to_bf16_bits(acc[2]),
            f32_to_bf16_bits(acc[3])};
}

// The combine for top-k entries per token.
static void launch_tkg_combine(const float* y, const int32_t* tok_slot, const float* tok_w,
                               int64_t T, int64_t H, int K, int nq, size_t part_stride,
                               uint16_t* out, hipStream_t s) {
  const dim3 g((unsigned)((H / 4 + 255) / 256), (unsigned)T);
  if (K <= 4)
    hipLaunchKernelGGL(tkg_combine_kernel<4>, g, dim3(256), 0, s, y, tok_slot, tok_w, (int)H, K,
                       nq, part_stride, out);
  else if (K <= 8)
    hipLaunchKernelGGL(tkg_combine_kernel<8>, g, dim3(256), 0, s, y, tok_slot, tok_w, (int)H, K,
                       nq, part_stride, out);
  else
    hipLaunchKernelGGL(tkg_combine_kernel<0>, g, dim3(256), 0, s, y, tok_slot, tok_w, (int)H, K,
                       nq, part_stride, out);
}

// Token tiles of the routed batch: sum over touched experts of ceil(n_e / 16) with
// sum n_e = T K, at most when every expert is touched: min(E, T K) + (T K - min(E, T K)) / 16.
inline int64_t tkg_max_tiles(int64_t T, int64_t E, int K) {
  const int64_t S = T * K, a = E < S ? E : S;
  return a + (S - a) / 16;
}

// Work split of a decode batch of the one-tile kernels.  A batch touching few experts has
// fewer row-group items than wave slots and is latency-bound (each wave streams one item
// with one or two chunks in flight).  Such batches split each item's K into parts, each
// part its own work unit: gate_up in 2 parts when it has under 2,000 items (the raw part
// sums go through the activation kernel).  Measured on the 20B-shaped layer, us per step:
// 1 token 47.4 unsplit -> 37.5.  More parts lose: each costs a unit start-up and a
// combine read, and so does a gate_up split at 2,700 items and more (16 tokens: +0.5 us;
// 64 tokens: +16 us).
// Down, with the packed hi/lo items (one MFMA per product for tiles of at most 8
// tokens), from a sweep of item shape x K parts at 4-64 tokens on the 20B- and
// 120B-shaped layers (same box, two alternating runs each):
//   * batches whose tiles hold 2.5 tokens or more on average, with under 1,400 wide
//     items (8 row groups, one-wave workgroups, 12 per CU: 3,072 wave slots on 256 CUs):
//     wide items in 2 K parts, both parts in one round of slots (20B shape, 24 / 32 / 48
//     / 64 tokens: 95.6 / 97.5 / 101.7 / 108.5 us; 4-row-group items unsplit 96.2 /
//     98.8 / 107 / 117.3);
//   * else 4-row-group items (two chunks in flight, one-wave workgroups) while they
//     stay under 1.7 rounds of wave slots and do not start a nearly empty round (a last
//     round under 15 % full): 120B shape 16 / 32 / 48 tokens 135.4 / 199.4 / 239.1 us
//     against 139.8 / 203.7 / 242.0 with wide items; at 24 tokens (~3,090 items, a
//     second round of a few items) wide items 171.4 against 173.8; at 64 tokens (~5,400
//     items, 1.76 rounds) wide 263.5 against 264.2.  Under 800 items they take 2 K parts
//     (20B shape, 4 tokens: 55.6 us against 57.0 unsplit and 57.7 in 3 parts; 120B
//     shape, 4 tokens: 62.5 with 1 or 2 parts, 63.8 in 3);
//   * else wide items, whole K.
// The smallest batches (under 1,300 gate_up items: 1-3 tokens here, and 4 on the 20B
// shape) take gate_up items of one gate/up pair over all of K, four chunks in flight, in
// one-wave workgroups, instead of the 2 K parts: as many units and bytes per unit, no
// part sums and no activation launch, and the waves spread over every CU (a 1-token
// batch's 720 pair items fill only 180 workgroups of four).  Same box, alternating runs,
// us per step against the 2 K parts: 20B-shaped layer 1 token 38.0 -> 35.0, 2 tokens
// 50.4 -> 46.8, 3 tokens 54.8 -> 54.3, 4 tokens (~1,210 items) 60.0 -> 59.2; 120B-shaped
// 1 token 40.1 -> 36.7, 2 tokens 53.3 -> 50.0, 3 tokens 59.7 -> 58.3.  Pair items at 4
// tokens on the 120B shape (~1,380 items) measured 67.0 -> 69.0: hence the threshold.
constexpr double kTkgGateUpPairItems = 1300.0;
constexpr double kTkgGateUpSplitItems = 2000.0;
constexpr double kTkgWaveSlots = 3072.0;        // one-wave workgroups in one round
constexpr double kTkgWideSplitItems = 1400.0;
constexpr double kTkgWideTileTokens = 2.5;      // tokens per tile that favour wide items
constexpr double kTkgNarrowMaxRounds = 1.7;
constexpr double kTkgNarrowMinLastRound = 0.15;
constexpr double kTkgNarrowSplitItems = 800.0;
constexpr double kTkgGuWideMinRounds = 1.2, kTkgGuWideMaxRounds = 1.7;
struct TkgSplit {
  int nq_gu = 1, nq_dn = 1;    // K parts
  int cpq_gu = 1 << 20, cpq_dn = 1 << 20;  // 128-wide chunks per part
  bool one_tile = true;
  bool gu_pairs = false;       // gate_up items of one gate/up pair, all of K
  bool dn_wide = false;        // down items of 8 row groups, one chunk in flight
  bool gu_wide = false;        // gate_up items of 8 row groups (4 pairs), one chunk in flight
};

// q K parts of nc chunks: cpq = ceil(nc / q) chunks each, and the part count recomputed
// from it, so that every part [p * cpq, min(nc, (p + 1) * cpq)) holds at least one chunk.
static void tkg_parts(int nc, int q, int& nq, int& cpq) {
  q = q < 1 ? 1 : (q > nc ? nc : q);
  cpq = (nc + q - 1) / q;
  nq = (nc + cpq - 1) / cpq;
}

static TkgSplit tkg_split(int64_t T, int64_t H, int64_t I, int64_t E, int K) {
  TkgSplit sp;
  sp.one_tile = T <= 16 || T * K <= 8 * E;
  if (!sp.one_tile) return sp;
  const double active = (double)E * (1.0 - pow(1.0 - (double)K / (double)E, (double)T));
  const double tiles = active + ((double)(T * K) - active) / 16.0;  // 16-token tiles
  const double gu_items = tiles * (double)((2 * I / 16 + 3) / 4);
  sp.gu_pairs = gu_items < kTkgGateUpPairItems;
  // gate_up items of 4 pairs, one chunk in flight, one-wave workgroups, when items of 2
  // pairs would make between 1.2 and 1.7 rounds of wave slots and the tiles hold 2.5
  // tokens or more on average: the wide items then run in one round and read each
  // activation row once per 8 row groups instead of 4.  Same box, alternating runs, us per
  // step: 20B-shaped layer 48 / 56 / 64 tokens (4.6-5.6 tokens per tile) 100.4 / 103.6 /
  // 107.1 -> 100.1 / 102.1 / 104.2; with about one token per tile they lose (120B shape 12
  // and 16 tokens +2.4 and +7.9, 256-expert layer 8 tokens +1.7), as they do outside that
  // range of rounds (20B shape 24 and 32 tokens, just over one round, +1.1 to +1.5; 120B
  // shape 24 to 64 tokens, 2 to 3.3 rounds, +2.5 to +11).
  const double gu_rounds = gu_items / kTkgWaveSlots;
  sp.gu_wide = !sp.gu_pairs && gu_rounds >= kTkgGuWideMinRounds &&
               gu_rounds < kTkgGuWideMaxRounds && (double)(T * K) >= kTkgWideTileTokens * tiles;
  if (!sp.gu_pairs && !sp.gu_wide && gu_items < kTkgGateUpSplitItems)
    tkg_parts((int)((H + 127) / 128), 2, sp.nq_gu, sp.cpq_gu);
  const int nc_dn = (int)((I + 127) / 128);
  const double wide_items = tiles * (double)((H / 16 + 7) / 8);
  if ((double)(T * K) >= kTkgWideTileTokens * tiles && wide_items < kTkgWideSplitItems) {
    sp.dn_wide = true;
    tkg_parts(nc_dn, 2, sp.nq_dn, sp.cpq_dn);
    return sp;
  }
  const double dn_items = tiles * (double)((H / 16 + 3) / 4);
  const double rounds = dn_items / kTkgWaveSlots;
  const bool narrow = rounds < kTkgNarrowMaxRounds &&
                      (rounds < 1.0 || rounds - floor(rounds) >= kTkgNarrowMinLastRound);
  sp.dn_wide = !narrow;
  if (narrow && dn_items < kTkgNarrowSplitItems) tkg_parts(nc_dn, 2, sp.nq_dn, sp.cpq_dn);
  return sp;
}

struct TkgWs {
  int32_t *expert_off, *active, *n_active, *slot_tok, *tok_slot, *tiles, *n_tiles;
  float* tok_w;
  uint16_t *h_hi, *h_lo;
  float* y;     // [nq_dn, S, H]
  float* part;  // [nq_gu, S, 2I] when nq_gu > 1
};

static size_t tkg_carve(void* base, size_t cap, int64_t T, int64_t H, int64_t I, int64_t E,
                        int K, TkgWs* w) {
  Carver cv(base, cap);
  const int64_t S = T * K;
  const TkgSplit sp = tkg_split(T, H, I, E, K);
  TkgWs t;
  t.expert_off = cv.take<int32_t>(E + 1);
  t.active = cv.take<int32_t>(E);
  t.n_active = cv.take<int32_t>(1);
  t.slot_tok = cv.take<int32_t>(S);
  t.tok_slot = cv.take<int32_t>(S);
  t.tok_w = cv.take<float>(S);
  t.tiles = cv.take<int32_t>(4 * tkg_max_tiles(T, E, K));
  t.n_tiles = cv.take<int32_t>(1);
  t.h_hi = cv.take<uint16_t>(S * I);
  t.h_lo = cv.take<uint16_t>(S * I);
  t.y = cv.take<float>(sp.nq_dn * S * H);
  t.part = cv.take<float>(sp.nq_gu > 1 ? sp.nq_gu * S * 2 * I : 0);
  if (w) *w = t;
  return cv.off + 256;
}

}  // namespace mxmoe

using namespace mxmoe;

extern "C" size_t mxmoe_moe_tkg_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                                                int top_k) {
  return tkg_carve(nullptr, ~(size_t)0, T, H, I, E, top_k, nullptr);
}

namespace mxmoe {

static int tkg_check(int64_t T, int64_t H, int64_t I, int64_t E, int top_k, int act,
                     int scale_mode) {
  MXMOE_REQUIRE(T >= 1 && T <= kTkgMaxT, "moe_tkg: T=%lld out of range [1, %d]", (long long)T,
                kTkgMaxT);
  MXMOE_REQUIRE(E >= 1 && E <= kTkgMaxE, "moe_tkg: E=%lld out of range [1, %d]", (long long)E,
                kTkgMaxE);
  MXMOE_REQUIRE(H % 32 == 0 && I % 32 == 0 && H >= 32 && I >= 32,
                "moe_tkg: H=%lld and I=%lld must be multiples of 32", (long long)H, (long long)I);
  MXMOE_REQUIRE(top_k >= 1 && top_k <= 8, "moe_tkg: top_k=%d out of range [1, 8]", top_k);
  MXMOE_REQUIRE(act >= 0 && act <= 2, "moe_tkg: unknown activation %d", act);
  // the streaming items address activations by 32-bit byte offsets from h_hi, the lo
  // rows included (h_hi and h_lo are each [T k, I] bf16, one after the other)
  MXMOE_REQUIRE((double)T * top_k * (double)I * 4.0 + (double)(H + I) * 4.0 + 4096.0 <
                    4294967296.0,
                "moe_tkg: T=%lld x top_k=%d x I=%lld activations exceed 32-bit offsets",
                (long long)T, top_k, (long long)I);
  MXMOE_REQUIRE(scale_mode == MXMOE_SCALE_POST || scale_mode == MXMOE_SCALE_NO,
                "moe_tkg: unsupported scale mode %d", scale_mode);
  return MXMOE_OK;
}

// route -> gate_up -> down -> combine; ev (may be null) gets 5 marks: before the
// routing kernel and after each of the four kernels.
static int tkg_pipeline(const uint16_t* x, const int32_t* topk_idx, const float* topk_val,
                        const uint8_t* gu_q, const uint8_t* gu_s, const uint8_t* dn_q,
                        const uint8_t* dn_s, const uint16_t* gu_bias, const uint16_t* dn_bias,
                        int64_t T, int64_t H, int64_t I, int64_t E, int top_k, int act,
                        const float* clamps, int scale_mode, uint16_t* out, const TkgWs& w,
                        void* const* ev, hipStream_t s, bool routed = false) {
  TkgArgs a = {};
  a.p.gate_lo = clamps ? clamps[0] : -INFINITY;
  a.p.gate_hi = clamps ? clamps[1] : INFINITY;
  a.p.up_lo = clamps ? clamps[2] : -INFINITY;
  a.p.up_hi = clamps ? clamps[3] : INFINITY;
  a.p.act = act;
  a.H = (int)H;
  a.I = (int)I;
  a.expert_off = w.expert_off;
  a.active = w.active;
  a.n_active = w.n_active;
  a.slot_tok = w.slot_tok;
  a.tiles = w.tiles;
  a.n_tiles = w.n_tiles;
  a.nq = 1;
  a.cpq = 1 << 20;  // one K part: all chunks
  mark_event(ev, 0, s);
  if (!routed)  // else the decode front end has routed the batch into w
    hipLaunchKernelGGL(tkg_route_kernel, dim3(1), dim3(1024), 0, s, topk_idx, topk_val, (int)T,
                       top_k, (int)E, scale_mode, w.expert_off, w.active, w.n_active, w.slot_tok,
                       w.tok_slot, w.tok_w, w.tiles, w.n_tiles);
  mark_event(ev, 1, s);
  TkgArgs gu = a, dn = a;
  gu.x = x;
  gu.wq = gu_q;
  gu.ws = gu_s;
  gu.bias = gu_bias;
  gu.out_hi = w.h_hi;
  gu.out_lo = w.h_lo;
  dn.h_hi = w.h_hi;
  dn.h_lo = w.h_lo;
  dn.lo_shift = (uint32_t)((const char*)w.h_lo - (const char*)w.h_hi);
  dn.wq = dn_q;
  dn.ws = dn_s;
  dn.bias = dn_bias;
  dn.y = w.y;
  // One wave per item; the grid covers the most items the batch can have (the active
  // experts and token tiles are known on the device only); surplus waves return at once.
  auto grid = [&](bool gate_up, int R, int wpb, int64_t units) {
    return dim3((unsigned)((units * tkg_items_per_expert((int)H, (int)I, gate_up, R) + wpb - 1) /
                           wpb));
  };
  const int64_t n_tile_max = tkg_max_tiles(T, E, top_k);
  const TkgSplit sp = tkg_split(T, H, I, E, top_k);
  // The one-tile kernels need fewer registers than three waves per SIMD allow; unused
  // dynamic LDS holds them at three (3 workgroups of 4 waves per CU), the occupancy
  // their item sizes and the dispatcher's spreading are set for.
  constexpr unsigned kLds3x4 = 50 * 1024, kLds12x1 = 13 * 1024;
  if (sp.one_tile) {
    const int S = (int)(T * top_k);
    gu.nq = sp.nq_gu;
    gu.cpq = sp.cpq_gu;
    gu.part = w.part;
    gu.part_stride = (size_t)S * 2 * (size_t)I;
    // One 16-token tile per item of 2 gate/up pairs; with nq_gu > 1 each item's K in
    // nq_gu parts, whose raw sums the activation kernel adds in order before the bias,
    // clamps and activation.  The smallest batches: items of one pair, four chunks in
    // flight, one-wave workgroups.
    // Unsplit batches of up to 16 tokens: one-wave workgroups too (same box, alternating
    // runs, us per step: 120B-shaped layer 8 / 12 / 16 tokens -1.9 / -1.1 / -1.8, 20B-shaped
    // 12 / 16 tokens -4.6 / -2.8; at 24-64 tokens on the 20B shape +0.4 to +2.5, at 48
    // and 64 tokens on the 120B shape +1.6 and +1.0, at 4 split tokens +0.7).
    if (sp.gu_pairs)
      hipLaunchKernelGGL((tkg_stream_kernel<2, 1, true, 4, 1>),
                         dim3(grid(true, 2, 1, n_tile_max).x), dim3(64), kLds12x1, s, gu);
    else if (sp.gu_wide)
      hipLaunchKernelGGL((tkg_stream_kernel<8, 1, true, 1, 1>),
                         dim3(grid(true, 8, 1, n_tile_max).x), dim3(64), kLds12x1, s, gu);
    else if (sp.nq_gu == 1 && T <= 16)
      hipLaunchKernelGGL((tkg_stream_kernel<4, 1, true, 2, 1>),
                         dim3(grid(true, 4, 1, n_tile_max).x), dim3(64), kLds12x1, s, gu);
    else
      hipLaunchKernelGGL((tkg_stream_kernel<4, 1, true, 2, 4>),
                         dim3(grid(true, 4, 4, n_tile_max).x * sp.nq_gu), dim3(256), kLds3x4,
                         s, gu);
    if (sp.nq_gu > 1)
      hipLaunchKernelGGL(tkg_act_kernel, dim3((unsigned)((I + 1023) / 1024), (unsigned)S),
                         dim3(256), 0, s, gu, (int)E);
    mark_event(ev, 2, s);
    // down (the item shape and K parts from tkg_split, on the expected active experts
    // E (1 - (1 - k/E)^T)): wide items of 8 row groups with one chunk in flight, three
    // waves per SIMD, one wave per workgroup, so that a 64-token batch's items run in one
    // round spread over the CUs one wave at a time and every CU streams about the same
    // share of the weights; or items of 4 row groups with two chunks in flight.  Each
    // item's K in nq_dn parts: the first part adds the bias, the combine adds the parts
    // in order.
    dn.part_stride = (size_t)S * (size_t)H;
    dn.nq = sp.nq_dn;
    dn.cpq = sp.cpq_dn;
    if (sp.dn_wide) {
      hipLaunchKernelGGL((tkg_stream_kernel<8, 1, false, 1, 1>),
                         dim3(grid(false, 8, 1, n_tile_max).x * sp.nq_dn), dim3(64), kLds12x1, s,
                         dn);
    } else {
      // one-wave workgroups (us per step against four-wave ones, same box: 20B-shaped
      // layer 12 / 16 / 24 / 32 tokens -3.4 / -2.6 / -6.2 / -6.8, 120B-shaped 4 / 8 tokens
      // -1.5 / -1.4, elsewhere within +-0.7 except 8 tokens on the 20B shape: +1.1, -0.7
      // and +1.9 in three comparisons)
      hipLaunchKernelGGL((tkg_stream_kernel<4, 1, false, 2, 1>),
                         dim3(grid(false, 4, 1, n_tile_max).x * sp.nq_dn), dim3(64), kLds12x1, s,
                         dn);
    }
  } else {
    // Two token tiles per pass (an expert with more tokens loops over passes).
    hipLaunchKernelGGL((tkg_stream_kernel<4, 2, true, 2, 4>), grid(true, 4, 4, E), dim3(256), 0, s,
                       gu);
    mark_event(ev, 2, s);
    hipLaunchKernelGGL((tkg_stream_kernel<4, 2, false, 2, 4>), grid(false, 4, 4, E), dim3(256), 0,
                       s, dn);
  }
  mark_event(ev, 3, s);
  launch_tkg_combine(w.y, w.tok_slot, w.tok_w, T, H, top_k, dn.nq, dn.part_stride, out, s);
  mark_event(ev, 4, s);
  return check_launch("moe_tkg");
}

struct DecodeWs {
  float* part;  // front end: [kFrontSlices, T, E] partial logits (T <= kFrontMaxT)
  float* logits;
  int32_t* idx;
  float* val;
  void* tkg;
  size_t tkg_bytes;
};

static size_t decode_carve(void* base, size_t cap, int64_t T, int64_t H, int64_t I, int64_t E,
                           int K, DecodeWs* d) {
  Carver cv(base, cap);
  DecodeWs r;
  r.part = cv.take<float>((T <= kFrontMaxT ? T : 0) * kFrontSlices * E);
  r.logits = cv.take<float>(T * E);
  r.idx = cv.take<int32_t>(T * K);
  r.val = cv.take<float>(T * K);
  r.tkg_bytes = tkg_carve(nullptr, ~(size_t)0, T, H, I, E, K, nullptr);
  r.tkg = cv.take<char>(r.tkg_bytes);
  if (d) *d = r;
  return cv.off + 256;
}

// ---------------------------------------------------------------------------------------
// Decode with bf16 expert weights (the bf16 model's moe_block_tkg operands: gate_up
// [E][H][2I], each row gate columns then up columns; down [E][I][H]).  The routing, the
// 16-token tiles, the split-K activation kernel and the combine are the MXFP4 decode's; the
// streaming items differ: one wave per (tile, 64 output columns, K part), weights K-major.
// Per 32-row chunk a lane loads 4 x 16 B of the weight block (8 lanes per 128-byte row
// segment) and 16 B of its token's activations, bounds-checked buffer loads three chunks
// ahead; the wave writes the block to its own 4 KiB of LDS and reads it back with the
// transposing read (ds_read_b64_tr_b16) as MFMA A operands (rows = output columns, 8
// K-values of one column per lane), the activations being the B operand (columns =
// tokens).  No barrier: each wave only reads what it wrote, and its LDS operations run in
// order.  gate_up writes raw K-part sums [nq, S, 2I] (tkg_act_kernel adds the parts, bias,
// clamps and activation); down reads h as hi + lo (two MFMAs, exact bf16 products) and
// writes its K parts [nq, S, H], the first carrying the bias (tkg_combine_kernel adds them).
constexpr int kBdCols = 64;    // output columns per item
constexpr int kBdK = 32;       // K rows per chunk
constexpr int kBdWaves = 4;    // waves per workgroup, each with its own LDS block
constexpr int kBdBlock = kBdK * kBdCols * 2;  // 4 KiB
constexpr uint32_t kBdOff = 0xFFFFFFF0u;      // past every buffer resource's range

__device__ __forceinline__ __amdgpu_buffer_rsrc_t bd_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bd_load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
// LDS byte offset of (row r, column c) in a wave's [32][64] bf16 block: 32-byte column groups
// XOR-swizzled by row so that the 16 rows one transposing read touches spread over the banks.
__device__ __forceinline__ uint32_t bd_off(int r, int c) {
  const uint32_t sw = (uint32_t)((((r >> 1) ^ (r >> 3)) & 3) << 1);
  return (uint32_t)r * (kBdCols * 2) + ((((uint32_t)c >> 3) ^ sw) << 4) + (uint32_t)((c & 7) << 1);
}
typedef short bd_s16x4 __attribute__((ext_vector_type(4)));
typedef short bd_s16x8 __attribute__((ext_vector_type(8)));

struct BdChunk {
  u32x4 w[4];
  u32x4 x, x2;  // the lane's token's 8 K-values (down: hi, lo)
};

template <bool GATE_UP>
__global__ void __launch_bounds__(64 * kBdWaves) __attribute__((amdgpu_waves_per_eu(3)))
    tkgb_stream_kernel(TkgArgs a, float* __restrict__ out, size_t out_stride) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kBdWaves][kBdBlock];
  const int N = GATE_UP ? 2 * a.I : a.H;  // output columns = weight row length
  const int K = GATE_UP ? a.H : a.I;
  const int nb = (N + kBdCols - 1) / kBdCols;
  const int wave = wave_id();
  const int u = blockIdx.x * kBdWaves + wave;
  if (u >= *a.n_tiles * nb * a.nq) return;
  const int item = u / a.nq, q = u - item * a.nq;
  const int ti = item / nb, cb = (item - ti * nb) * kBdCols;
  const int4 tm = reinterpret_cast<const int4*>(a.tiles)[ti];
  const int e = __builtin_amdgcn_readfirstlane(tm.x);
  const int s0 = __builtin_amdgcn_readfirstlane(tm.y);
  const int ne = __builtin_amdgcn_readfirstlane(tm.z);
  const int lane = threadIdx.x & 63, li = lane & 15, lq = lane >> 4;
  const int nc = K / kBdK;
  const int c0 = q * a.cpq, c1 = min(nc, c0 + a.cpq);
  // weights of expert e, K rows of N; this lane's 16-byte block: row lane / 8 + 8 j, columns
  // cb + 8 (lane % 8) ..
  const __amdgpu_buffer_rsrc_t rw = bd_rsrc(
      reinterpret_cast<const uint16_t*>(a.wq) + (size_t)e * K * N, (uint32_t)((size_t)K * N * 2));
  const int wc = cb + 8 * (lane & 7), wr = lane >> 3;
  const bool wc_ok = wc < N;
  // activations: gate_up x[token] of [T, H]; down h rows [slots, I] (hi, lo)
  const bool t_ok = li < ne;
  uint32_t xrow = 0;
  if (t_ok) xrow = GATE_UP ? (uint32_t)a.slot_tok[s0 + li] : (uint32_t)(s0 + li);
  const uint32_t x_rows = GATE_UP ? (uint32_t)a.T : (uint32_t)a.S;
  const __amdgpu_buffer_rsrc_t rx =
      bd_rsrc(GATE_UP ? (const void*)a.x : (const void*)a.h_hi, x_rows * (uint32_t)K * 2u);
  const __amdgpu_buffer_rsrc_t rx2 =
      bd_rsrc(GATE_UP ? (const void*)a.x : (const void*)a.h_lo, x_rows * (uint32_t)K * 2u);
  auto load = [&](BdChunk& f, int c) {
    c = min(c, c1 - 1);  // past the part's last chunk: a re-read that is never used
    const int kc = c * kBdK;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      f.w[j] = bd_load(rw, wc_ok ? ((uint32_t)(kc + wr + 8 * j) * (uint32_t)N + (uint32_t)wc) * 2u
                                 : kBdOff);
    const uint32_t xo = t_ok ? (xrow * (uint32_t)K + (uint32_t)(kc + 8 * lq)) * 2u : kBdOff;
    f.x = bd_load(rx, xo);
    if (!GATE_UP) f.x2 = bd_load(rx2, xo);
  };
  uint8_t* blk = lds[wave];
  f32x4 acc[4];
#pragma unroll
  for (int f = 0; f < 4; ++f) acc[f] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto step = [&](const BdChunk& f) {
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4*>(blk + bd_off(wr + 8 * j, 8 * (lane & 7))) = f.w[j];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int n = 16 * t + 4 * (li & 3);
      const int r = 8 * lq + (li >> 2);
      const bd_s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) bd_s16x4*)(
              (__attribute__((address_space(3))) uint8_t*)(blk + bd_off(r, n))));
      const bd_s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) bd_s16x4*)(
              (__attribute__((address_space(3))) uint8_t*)(blk + bd_off(r + 4, n))));
      const bd_s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      const bf16x8 wa = __builtin_bit_cast(bf16x8, v);
      acc[t] = mfma16(wa, as_bf16x8(f.x), acc[t]);
      if (!GATE_UP) acc[t] = mfma16(wa, as_bf16x8(f.x2), acc[t]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // three chunks in flight; every load issued in a fixed order (counted waits)
  BdChunk r0, r1, r2;
  load(r0, c0);
  load(r1, c0 + 1);
  load(r2, c0 + 2);
  // No exit inside the loop: the steps past the part's last chunk are skipped, their loads
  // still issued, so every path issues the same loads and the waits stay counted.
  for (int c = c0; c < c1; c += 3) {
    step(r0);
    load(r0, c + 3);
    if (c + 1 < c1) step(r1);
    load(r1, c + 4);
    if (c + 2 < c1) step(r2);
    load(r2, c + 5);
  }
  if (!t_ok) return;
  const size_t slot = (size_t)(s0 + li);
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int n = cb + 16 * t + 4 * lq;
    if (n >= N) continue;
    f32x4 v = acc[t];
    if (!GATE_UP && a.bias && q == 0) {  // the first K part carries the down bias
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] += bf16_bits_to_f32(a.bias[(size_t)e * N + n + i]);
    }
    *reinterpret_cast<f32x4*>(out + q * out_stride + slot * N + n) = v;
  }
}

// K parts of the bf16 items: enough units for the wave slots (about 3,000), at most 8 parts.
static void tkgb_parts(double units, int nc, int& nq, int& cpq) {
  int q = (int)ceil(3000.0 / (units > 1.0 ? units : 1.0));
  tkg_parts(nc, q > 8 ? 8 : q, nq, cpq);
}

struct TkgbPlan {
  int nq_gu, cpq_gu, nq_dn, cpq_dn;
};
static TkgbPlan tkgb_plan(int64_t T, int64_t H, int64_t I, int64_t E, int K) {
  const double active = (double)E * (1.0 - pow(1.0 - (double)K / (double)E, (double)T));
  const double tiles = active + ((double)(T * K) - active) / 16.0;
  TkgbPlan p;
  tkgb_parts(tiles * (double)((2 * I + kBdCols - 1) / kBdCols), (int)(H / kBdK), p.nq_gu,
             p.cpq_gu);
  tkgb_parts(tiles * (double)((H + kBdCols - 1) / kBdCols), (int)(I / kBdK), p.nq_dn, p.cpq_dn);
  return p;
}

static size_t tkgb_carve(void* base, size_t cap, int64_t T, int64_t H, int64_t I, int64_t E,
                         int K, TkgWs* w) {
  Carver cv(base, cap);
  const int64_t S = T * K;
  const TkgbPlan p = tkgb_plan(T, H, I, E, K);
  TkgWs t;
  t.expert_off = cv.take<int32_t>(E + 1);
  t.active = cv.take<int32_t>(E);
  t.n_active = cv.take<int32_t>(1);
  t.slot_tok = cv.take<int32_t>(S);
  t.tok_slot = cv.take<int32_t>(S);
  t.tok_w = cv.take<float>(S);
  t.tiles = cv.take<int32_t>(4 * tkg_max_tiles(T, E, K));
  t.n_tiles = cv.take<int32_t>(1);
  t.h_hi = cv.take<uint16_t>(S * I);
  t.h_lo = cv.take<uint16_t>(S * I);
  t.y = cv.take<float>(p.nq_dn * S * H);
  t.part = cv.take<float>(p.nq_gu * S * 2 * I);
  if (w) *w = t;
  return cv.off + 256;
}

size_t tkg_bf16_stream_workspace(int64_t T, int64_t H, int64_t I, int64_t E, int K) {
  return tkgb_carve(nullptr, ~(size_t)0, T, H, I, E, K, nullptr);
}

// route -> gate_up items -> activation -> down items -> combine (bf16 expert weights).
int tkg_bf16_stream(const uint16_t* x, const int32_t* topk_idx, const float* topk_val,
                    const uint16_t* gu_w, const uint16_t* dn_w, const uint16_t* gu_bias,
                    const uint16_t* dn_bias, int64_t T, int64_t H, int64_t I, int64_t E,
                    int top_k, int act, const float* clamps, int scale_mode, uint16_t* out,
                    void* workspace, size_t workspace_bytes, hipStream_t s) {
  MXMOE_REQUIRE(T <= kTkgMaxT && E <= kTkgMaxE && top_k <= 8,
                "moe_tkg_bf16: T=%lld, E=%lld or top_k=%d beyond the decode routing",
                (long long)T, (long long)E, top_k);
  const size_t need = tkgb_carve(nullptr, ~(size_t)0, T, H, I, E, top_k, nullptr);
  if (workspace_bytes < need)
    return set_error(MXMOE_E_WORKSPACE, "moe_tkg_bf16: workspace %zu < %zu", workspace_bytes,
                     need);
  TkgWs w;
  tkgb_carve(workspace, workspace_bytes, T, H, I, E, top_k, &w);
  const TkgbPlan pl = tkgb_plan(T, H, I, E, top_k);
  const int S = (int)(T * top_k);
  TkgArgs a = {};
  a.p.gate_lo = clamps ? clamps[0] : -INFINITY;
  a.p.gate_hi = clamps ? clamps[1] : INFINITY;
  a.p.up_lo = clamps ? clamps[2] : -INFINITY;
  a.p.up_hi = clamps ? clamps[3] : INFINITY;
  a.p.act = act;
  a.H = (int)H;
  a.I = (int)I;
  a.T = (int)T;
  a.S = S;
  a.expert_off = w.expert_off;
  a.active = w.active;
  a.n_active = w.n_active;
  a.slot_tok = w.slot_tok;
  a.tiles = w.tiles;
  a.n_tiles = w.n_tiles;
  hipLaunchKernelGGL(tkg_route_kernel, dim3(1), dim3(1024), 0, s, topk_idx, topk_val, (int)T,
                     top_k, (int)E, scale_mode, w.expert_off, w.active, w.n_active, w.slot_tok,
                     w.tok_slot, w.tok_w, w.tiles, w.n_tiles);
  const int64_t n_tile_max = tkg_max_tiles(T, E, top_k);
  auto blocks = [&](int64_t cols, int nq) {
    const int64_t units = n_tile_max * ((cols + kBdCols - 1) / kBdCols) * nq;
    return dim3((unsigned)((units + kBdWaves - 1) / kBdWaves));
  };
  TkgArgs gu = a;
  gu.x = x;
  gu.wq = reinterpret_cast<const uint8_t*>(gu_w);
  gu.bias = gu_bias;
  gu.nq = pl.nq_gu;
  gu.cpq = pl.cpq_gu;
  gu.part = w.part;
  gu.part_stride = (size_t)S * 2 * (size_t)I;
  gu.out_hi = w.h_hi;
  gu.out_lo = w.h_lo;
  hipLaunchKernelGGL(tkgb_stream_kernel<true>, blocks(2 * I, pl.nq_gu), dim3(64 * kBdWaves), 0,
                     s, gu, w.part, gu.part_stride);
  hipLaunchKernelGGL(tkg_act_kernel, dim3((unsigned)((I + 1023) / 1024), (unsigned)S),
                     dim3(256), 0, s, gu, (int)E);
  TkgArgs dn = a;
  dn.h_hi = w.h_hi;
  dn.h_lo = w.h_lo;
  dn.wq = reinterpret_cast<const uint8_t*>(dn_w);
  dn.bias = dn_bias;
  dn.nq = pl.nq_dn;
  dn.cpq = pl.cpq_dn;
  dn.part_stride = (size_t)S * (size_t)H;
  hipLaunchKernelGGL(tkgb_stream_kernel<false>, blocks(H, pl.nq_dn), dim3(64 * kBdWaves), 0, s,
                     dn, w.y, dn.part_stride);
  launch_tkg_combine(w.y, w.tok_slot, w.tok_w, T, H, top_k, pl.nq_dn, dn.part_stride, out, s);
  return check_launch("moe_tkg_bf16");
}

}  // namespace mxmoe

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
  int rc = tkg_check(T, H, I, E, top_k, act, scale_mode);
  if (rc) return rc;
  const size_t need = mxmoe_moe_tkg_workspace_bytes(T, H, I, E, top_k);
  if (workspace_bytes < need)
    return set_error(MXMOE_E_WORKSPACE, "moe_tkg: workspace %zu < %zu", workspace_bytes, need);
  TkgWs w;
  tkg_carve(workspace, workspace_bytes, T, H, I, E, top_k, &w);
  return tkg_pipeline(x, topk_idx, topk_val, gu_q, gu_s, dn_q, dn_s, gu_bias, dn_bias, T, H, I, E,
                      top_k, act, clamps, scale_mode, out, w, stage_events, as_stream(stream));
}

extern "C" size_t mxmoe_moe_decode_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                                                   int top_k) {
  return decode_carve(nullptr, ~(size_t)0, T, H, I, E, top_k, nullptr);
}

extern "C" int mxmoe_moe_decode(const uint16_t* x, const void* router_w, int router_w_dtype,
                                const void* router_b, int router_b_dtype, int router_act,
                                int act_before_topk, int renorm, float renorm_eps,
                                const uint8_t* gu_q, const uint8_t* gu_s, const uint8_t* dn_q,
                                const uint8_t* dn_s, const uint16_t* gu_bias,
                                const uint16_t* dn_bias, int64_t T, int64_t H, int64_t I,
                                int64_t E, int top_k, int act, const float* clamps,
                                int scale_mode, uint16_t* out, float* logits_out,
                                int32_t* topk_idx_out, void* workspace, size_t workspace_bytes,
                                void* const* stage_events, void* stream) {
  clear_error();
  MXMOE_REQUIRE(x && router_w && gu_q && gu_s && dn_q && dn_s && out && workspace,
                "moe_decode: null pointer");
  int rc = tkg_check(T, H, I, E, top_k, act, scale_mode);
  if (rc) return rc;
  const size_t need = mxmoe_moe_decode_workspace_bytes(T, H, I, E, top_k);
  if (workspace_bytes < need)
    return set_error(MXMOE_E_WORKSPACE, "moe_decode: workspace %zu < %zu", workspace_bytes,
                     need);
  DecodeWs d;
  decode_carve(workspace, workspace_bytes, T, H, I, E, top_k, &d);
  TkgWs w;
  tkg_carve(d.tkg, d.tkg_bytes, T, H, I, E, top_k, &w);
  MXMOE_REQUIRE(router_act == MXMOE_ROUTER_SOFTMAX || router_act == MXMOE_ROUTER_SIGMOID,
                "moe_decode: unknown router activation %d", router_act);
  MXMOE_REQUIRE(H % 32 == 0, "moe_decode: H=%lld must be a multiple of 32", (long long)H);
  // The reference decode flow computes the router in fp32 (moe_block_tkg.py:152-162): fp16
  // router weights are split exactly into two bf16 operands, bf16 ones are exact as they are.
  RouterSpec r;
  r.x = x;
  r.x_dt = kBF16;
  r.w = static_cast<const uint16_t*>(router_w);
  r.w_dt = router_w_dtype;
  r.bias = router_b;
  r.bias_dt = router_b_dtype;
  r.op = router_w_dtype == kF16 ? kOpExact : kOpBF16;
  rc = router_check(r);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
  float* logits = logits_out ? logits_out : d.logits;
  int32_t* idx = topk_idx_out ? topk_idx_out : d.idx;
  mark_event(stage_events, 0, s);
  if (T <= kFrontMaxT) {
    const dim3 fg((unsigned)((T + 15) / 16), (unsigned)((E + 15) / 16), kFrontSlices);
    if (router_w_dtype == kF16)
      hipLaunchKernelGGL(front_logits_kernel<true>, fg, dim3(64 * kFrontWaves), 0, s, x, r.w,
                         d.part, (int)T, (int)H, (int)E);
    else
      hipLaunchKernelGGL(front_logits_kernel<false>, fg, dim3(64 * kFrontWaves), 0, s, x, r.w,
                         d.part, (int)T, (int)H, (int)E);
    const int af = act_before_topk ? 1 : 0, rn = renorm ? 1 : 0;
    // One token tile, or up to 64 tokens over at most 64 experts: one workgroup takes the
    // top-k and routes (one launch less).  Else the top-k spreads over a workgroup per
    // tile, then the routing kernel.  Same box, alternating runs, us per step: 20B-shaped
    // layer (32 experts) 24 / 32 / 48 / 64 tokens 98.7 / 96.2 / 100.3 / 107.8 -> 93.8 / 95.6 /
    // 100.3 / 104.9; the 120B-shaped layer (128 experts) at 64 tokens 262.2 -> 263.6, so it
    // keeps two launches there.
    const bool fused = T <= 16 || (T <= 64 && E <= 64);
#define MXMOE_FRONT(P)                                                                       \
  if (fused)                                                                                 \
    hipLaunchKernelGGL(front_route_kernel<P>, dim3(1), dim3(1024), 0, s, d.part, router_b,    \
                       router_b_dtype, logits, (int)T, (int)E, top_k, router_act, af, rn,     \
                       renorm_eps, scale_mode, topk_idx_out, w.expert_off, w.active,          \
                       w.n_active, w.slot_tok, w.tok_slot, w.tok_w, w.tiles, w.n_tiles);      \
  else                                                                                       \
    hipLaunchKernelGGL(front_topk_kernel<P>, dim3((unsigned)((T + 15) / 16)), dim3(256), 0, s, \
                       d.part, router_b, router_b_dtype, logits, (int)T, (int)E, top_k,       \
                       router_act, af, rn, renorm_eps, idx, d.val)
    switch (front_per_lane((int)E)) {
      case 1: MXMOE_FRONT(1); break;
      case 2: MXMOE_FRONT(2); break;
      case 4: MXMOE_FRONT(4); break;
      case 8: MXMOE_FRONT(8); break;
      case 16: MXMOE_FRONT(16); break;
      default: MXMOE_FRONT(32); break;  // E <= 512
    }
#undef MXMOE_FRONT
    rc = check_launch("moe_decode front end");
    if (rc) return rc;
    return tkg_pipeline(x, idx, d.val, gu_q, gu_s, dn_q, dn_s, gu_bias, dn_bias, T, H, I, E,
                        top_k, act, clamps, scale_mode, out, w,
                        stage_events ? stage_events + 1 : nullptr, s, /*routed=*/fused);
  }
  rc = router_run(r, T, H, E, top_k, router_act, act_before_topk, renorm, renorm_eps, logits,
                  nullptr, nullptr, idx, d.val, s);
  if (rc) return rc;
  return tkg_pipeline(x, idx, d.val, gu_q, gu_s, dn_q, dn_s, gu_bias, dn_bias, T, H, I, E,
                      top_k, act, clamps, scale_mode, out, w,
                      stage_events ? stage_events + 1 : nullptr, s);
}

extern "C" size_t mxmoe_moe_block_decode_workspace_bytes(int64_t T, int64_t H, int64_t I,
                                                         int64_t E, int top_k) {
  return align_up(mxmoe_moe_decode_workspace_bytes(T, H, I, E, top_k), 256) +
         align_up((size_t)T * (size_t)H * 2u, 256);
}

extern "C" int mxmoe_moe_block_decode(
    const uint16_t* x, const float* gamma, int64_t h_actual, float eps, const void* router_w,
    int router_w_dtype, const void* router_b, int router_b_dtype, int router_act,
    int act_before_topk, int renorm, float renorm_eps, const uint8_t* gu_q, const uint8_t* gu_s,
    const uint8_t* dn_q, const uint8_t* dn_s, const uint16_t* gu_bias, const uint16_t* dn_bias,
    int64_t T, int64_t H, int64_t I, int64_t E, int top_k, int act, const float* clamps,
    int scale_mode, uint16_t* out, float* logits_out, int32_t* topk_idx_out, void* workspace,
    size_t workspace_bytes, void* const* stage_events, void* stream) {
  clear_error();
  MXMOE_REQUIRE(x && gamma && workspace, "moe_block_decode: null pointer");
  const size_t need = mxmoe_moe_block_decode_workspace_bytes(T, H, I, E, top_k);
  if (workspace_bytes < need)
    return set_error(MXMOE_E_WORKSPACE, "moe_block_decode: workspace %zu < %zu", workspace_bytes,
                     need);
  const size_t dec = align_up(mxmoe_moe_decode_workspace_bytes(T, H, I, E, top_k), 256);
  uint16_t* xn = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + dec);
  hipStream_t s = as_stream(stream);
  mark_event(stage_events, 0, s);
  int rc = rmsnorm_run(x, gamma, T, H, h_actual, /*all_cols=*/0, eps, kBF16, xn, s);
  if (rc) return rc;
  return mxmoe_moe_decode(xn, router_w, router_w_dtype, router_b, router_b_dtype, router_act,
                          act_before_topk, renorm, renorm_eps, gu_q, gu_s, dn_q, dn_s, gu_bias,
                          dn_bias, T, H, I, E, top_k, act, clamps, scale_mode, out, logits_out,
                          topk_idx_out, workspace, dec, stage_events ? stage_events + 1 : nullptr,
                          stream);
}

// ---- The decode block without allocation: the workspace is a file-scope device array.
//
// Callers that cannot allocate (code under graph capture, tight serving loops) get the
// same pipeline as mxmoe_moe_block_decode over a scratch array of fixed size in device
// memory, which each GPU the library runs on holds until the process ends.  Every
// buffer the pipeline reads in a call is written earlier in that call, so nothing needs
// clearing between calls; calls that overlap on one GPU share the array and race.

namespace mxmoe {

static __device__ __align__(256) unsigned char scratch[MXMOE_NOALLOC_SCRATCH_BYTES];

constexpr int kScratchMaxDevices = 64;
static std::once_flag g_scratch_once[kScratchMaxDevices];
static hipError_t g_scratch_rc[kScratchMaxDevices];
static void* g_scratch_ptr[kScratchMaxDevices];

// The current device's copy of the scratch array, looked up once per device with that
// device current: in host code the array's name is not a device address.
static int scratch_of_current_device(void** ptr) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(MXMOE_E_HIP, "moe_block_decode_noalloc: hipGetDevice: %s",
                     hipGetErrorString(e));
  MXMOE_REQUIRE(dev >= 0 && dev < kScratchMaxDevices,
                "moe_block_decode_noalloc: device %d beyond the %d supported", dev,
                kScratchMaxDevices);
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_rc[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_rc[dev] == hipSuccess ? p : nullptr;
  });
  if (g_scratch_rc[dev] != hipSuccess)
    return set_error(MXMOE_E_HIP, "moe_block_decode_noalloc: hipGetSymbolAddress: %s",
                     hipGetErrorString(g_scratch_rc[dev]));
  *ptr = g_scratch_ptr[dev];
  return MXMOE_OK;
}

}  // namespace mxmoe

extern "C" int mxmoe_moe_block_decode_noalloc(
    const uint16_t* x, const float* gamma, int64_t h_actual, float eps, const void* router_w,
    int router_w_dtype, const void* router_b, int router_b_dtype, int router_act,
    int act_before_topk, int renorm, float renorm_eps, const uint8_t* gu_q, const uint8_t* gu_s,
    const uint8_t* dn_q, const uint8_t* dn_s, const uint16_t* gu_bias, const uint16_t* dn_bias,
    int64_t T, int64_t H, int64_t I, int64_t E, int top_k, int act, const float* clamps,
    int scale_mode, uint16_t* out, float* logits_out, int32_t* topk_idx_out,
    void* const* stage_events, void* stream) {
  clear_error();
  int rc = tkg_check(T, H, I, E, top_k, act, scale_mode);
  if (rc) return rc;
  const size_t need = mxmoe_moe_block_decode_workspace_bytes(T, H, I, E, top_k);
  if (need > (size_t)MXMOE_NOALLOC_SCRATCH_BYTES)
    return set_error(MXMOE_E_WORKSPACE,
                     "moe_block_decode_noalloc: T=%lld, H=%lld, I=%lld, E=%lld, top_k=%d need "
                     "%zu bytes of scratch; the no-allocation entry point holds %zu",
                     (long long)T, (long long)H, (long long)I, (long long)E, top_k, need,
                     (size_t)MXMOE_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  rc = scratch_of_current_device(&ws);
  if (rc) return rc;
  return mxmoe_moe_block_decode(x, gamma, h_actual, eps, router_w, router_w_dtype, router_b,
                                router_b_dtype, router_act, act_before_topk, renorm, renorm_eps,
                                gu_q, gu_s, dn_q, dn_s, gu_bias, dn_bias, T, H, I, E, top_k, act,
                                clamps, scale_mode, out, logits_out, topk_idx_out, ws,
                                (size_t)MXMOE_NOALLOC_SCRATCH_BYTES, stage_events, stream);
}
