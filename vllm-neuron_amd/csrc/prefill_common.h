// Shared by the prefill GEMMs of both weight families (packed MX in expert_prefill.hip,
// bf16 in expert_prefill_bf16.hip): their arguments, the workgroup -> tile schedule's
// grid size, and the epilogue arithmetic with the reference's bf16 roundings.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace mxmoe {

constexpr int kPM = 128;  // slots per M-tile

struct PrefillArgs {
  const uint16_t* a;      // x [T, H] (gate_up) or h [slots, I] (down)
  const uint8_t* wq;      // weights, all experts: packed MX codes, or bf16 [E, K, N]
  const uint8_t* ws;      // packed scales (MX only)
  const uint16_t* bias;   // gate_up: [E, 2, I]; down: [E, H]; may be null
  const int32_t* tp2id;   // token_position_to_id [slots]
  uint16_t* out;          // h [slots, I] or y [slots, H]
  int T, K, N_rows, I, H, B;
  int n_mtiles, n_ntiles;
  int group;              // M-tiles scheduled together (divides n_mtiles)
  const int2* order;      // (first M-tile of a group, its expert) by rank (null: rank order,
                          // expert 0)
  int E;                  // experts: a tile whose expert lies outside [0, E) computes nothing
  int a_by_slot;          // gate_up reads row `slot` of a (pre-scaled rows), not the token's
  int32_t* inv;           // gate_up, N-tile 0: inv[token * E + expert] = slot (null: none)
  ExpertParams p;
};

// Workgroups per GEMM launch: every XCD runs the same number of group ranks.
inline unsigned prefill_grid(int n_mtiles, int n_ntiles, int group) {
  const int n_groups = n_mtiles / group;
  return (unsigned)(8 * group * n_ntiles * ((n_groups + 7) / 8));
}

// The tile a workgroup computes and its slots.  Workgroup -> (XCD, its i-th workgroup) ->
// (group rank, M-tile in the group, N-tile).  Consecutive workgroups of an XCD go to its
// shader engines in turn, so each M-tile of a group takes its N-tiles in a row
// (alternating M-tiles would send the full tiles to half of the engines).  Threads
// 0..127 (waves 0 and 1, whole) fill the slot tables: stok[i] = token of slot m0 + i or
// -1, rowoff[i] = byte offset of the activation row it reads (padding slots read a real
// row: an MFMA output column depends on its own slot only, and padding columns are never
// stored), lastw[w] = last slot of wave w's 64 holding a real token, or -1; the gate_up
// GEMM's N-tile 0 writes the combine's slot of each (token, expert) pair.  False: no tile
// (past the schedule, or an expert id outside [0, E)); the caller returns before any
// barrier.
struct PrefillTileId {
  int m0, e, nt;
};
template <bool GATE_UP>
__device__ __forceinline__ bool prefill_tile_begin(const PrefillArgs& args, int32_t* stok,
                                                   uint32_t* rowoff, int* lastw,
                                                   PrefillTileId& id) {
  const int G = args.group, per_group = G * args.n_ntiles;
  const int xcd = blockIdx.x & 7, local = blockIdx.x >> 3;
  const int rank = (local / per_group) * 8 + xcd;
  const int sub = (local % per_group) / args.n_ntiles, nt = local % args.n_ntiles;
  if (rank >= args.n_mtiles / G) return false;
  int mt = rank * G + sub, e = 0;
  if (args.order) {
    const int2 me = args.order[rank];
    mt = me.x + sub;
    e = me.y;
    if (e < 0 || e >= args.E) return false;  // a caller's out-of-range expert id: no tile
  }
  const int m0 = mt * kPM;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid < kPM) {
    // Without a mapping (plain linear) slot m0 + tid is row m0 + tid of A, real below T.
    int tk = args.tp2id ? args.tp2id[m0 + tid] : (m0 + tid < args.T ? m0 + tid : -1);
    if (tk < 0 || tk >= args.T) tk = -1;
    stok[tid] = tk;
    const uint32_t arow = (GATE_UP && !args.a_by_slot) ? (uint32_t)(tk >= 0 ? tk : 0)
                                                       : (uint32_t)(tk >= 0 ? m0 + tid : m0);
    rowoff[tid] = arow * (uint32_t)args.K * 2u;
    if (GATE_UP && args.inv && nt == 0 && tk >= 0) args.inv[(size_t)tk * args.E + e] = m0 + tid;
    const unsigned long long real = __ballot(tk >= 0);
    if (lane == 0) lastw[wave] = real ? 64 * wave + 63 - __builtin_clzll(real) : -1;
  }
  id.m0 = m0;
  id.e = e;
  id.nt = nt;
  return true;
}

// The GEMMs schedule M-tiles in groups of G consecutive tiles of one block (G = the
// largest power of two up to 16 dividing B / 128): the group's workgroups run one after
// another on one XCD, so a block's second, mostly empty M-tile reads the weight rows
// while the first one's workgroups hold them in L2.
constexpr int kMaxGroupTiles = 16;
inline int prefill_group_tiles(int64_t block_size) {
  const int64_t per = block_size / kPM;
  int g = 1;
  while (g < kMaxGroupTiles && per % (2 * g) == 0) g *= 2;
  return g;
}

// order[r] = (first M-tile of the r-th group by descending weight, ties in M order; the
// group's expert).  The weight of a tile is the number of its 16-slot subtiles whose
// first slot holds a real token (the GEMM's subtile count when real slots come first,
// as the blockwise mapping lays them out; a different layout only changes the
// schedule), a group's the sum over its tiles.  One workgroup: a histogram of the
// weights, then a stable scatter ranked by ballots per weight.
constexpr int kOrderThreads = 1024;
constexpr int kMaxWeights = kMaxGroupTiles * (kPM / 16) + 1;
constexpr int kOrderMaxTiles = 10240;  // 5 B of LDS per M-tile (with the sort tables < 64 KiB)
__device__ __forceinline__ int tile_weight(const int32_t* __restrict__ tp2id, int mt, int T) {
  int w = 0;
#pragma unroll
  for (int s = 0; s < kPM / 16; ++s) {
    const int tk = tp2id[(size_t)mt * kPM + 16 * s];
    w += (tk >= 0 && tk < T) ? 1 : 0;
  }
  return w;
}

constexpr int kOrderWaves = kOrderThreads / 64;
struct OrderLds {
  int hist[kMaxWeights];
  int next[kMaxWeights];  // next free rank per weight
  int cnt[kOrderWaves][kMaxWeights];
};

// One sort over the tile weights and experts staged in LDS (s_w, s_e).
__device__ inline void order_pass(const uint8_t* s_w, const int32_t* s_e, int n_groups, int G,
                           int2* __restrict__ order, OrderLds& L) {
  const int NW = G * (kPM / 16) + 1;  // weights 0 .. 8G
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  auto weight = [&](int g) {
    int w = 0;
    for (int i = 0; i < G; ++i) w += s_w[g * G + i];
    return w;
  };
  for (int v = tid; v < NW; v += kOrderThreads) L.hist[v] = 0;
  __syncthreads();
  for (int base = 0; base < n_groups; base += kOrderThreads) {
    const int g = base + tid;
    if (g < n_groups) atomicAdd(&L.hist[weight(g)], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int r = 0;
    for (int w = NW - 1; w >= 0; --w) {
      L.next[w] = r;
      r += L.hist[w];
    }
  }
  __syncthreads();
  const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int base = 0; base < n_groups; base += kOrderThreads) {
    const int g = base + tid;
    const int w = g < n_groups ? weight(g) : -1;
    int in_wave = 0;
    for (int v = 0; v < NW; ++v) {
      const unsigned long long m = __ballot(w == v);
      if (lane == 0) L.cnt[wave][v] = __popcll(m);
      if (w == v) in_wave = __popcll(m & below);
    }
    __syncthreads();
    if (w >= 0) {
      int r = L.next[w] + in_wave;
      for (int j = 0; j < wave; ++j) r += L.cnt[j][w];
      order[r] = int2{g * G, s_e[g * G]};
    }
    __syncthreads();
    for (int v = tid; v < NW; v += kOrderThreads) {
      int c = 0;
      for (int j = 0; j < kOrderWaves; ++j) c += L.cnt[j][v];
      L.next[v] += c;
    }
    __syncthreads();
  }
}

// Round to bf16 (nearest even) and back: the gfx950 conversion instruction, which
// gives round_bf16's result on every non-NaN input (NaN stays NaN).
__device__ __forceinline__ float rb(float v) { return (float)(__bf16)v; }

// Two floats -> a packed bf16 pair (a low), by the same conversion: one instruction for
// both.  A NaN stays a NaN; these are intermediates that later kernels read as numbers.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

__device__ __forceinline__ float clamp_ref(float v, float lo, float hi) {
  v = (v > hi) ? hi : v;
  v = (v < lo) ? lo : v;
  return v;
}

// Activation on a bf16 value with the reference's bf16 intermediate roundings.  The
// sigmoid uses the hardware exponential and reciprocal (about 1 ulp each in fp32); its
// result is rounded to bf16 right after, so it differs from the correctly rounded
// sigmoid only where that lies within a few fp32 ulps of a bf16 rounding boundary.
__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

template <int ACT>
__device__ __forceinline__ float act_bf16(float g) {
  if constexpr (ACT == kSwish) {
    const float t1 = rb(g * 1.702f);
    const float t2 = rb(sigmoid_fast(t1));
    return rb(g * t2);
  } else if constexpr (ACT == kSiLU) {
    return rb(g * sigmoid_fast(g));
  } else {
    return rb(0.5f * g * (1.0f + erff(g * 0.70710678118654752f)));
  }
}

// gate_up / down GEMM of bf16 expert weights ([E, H, 2, I] and [E, I, H], K-major rows as
// the reference's shard_on_block passes them) over the same schedule and epilogues.
void launch_prefill_gemm_bf16(bool gate_up, const PrefillArgs& a, hipStream_t s);
// The same GEMMs with the decode flow's fp32 arithmetic: gate_up writes h as bf16 (hi in
// a.out, lo in out_lo); down reads h from a.a (hi) and a_lo (lo) and writes y32 fp32.
void launch_decode_gemm_bf16(bool gate_up, const PrefillArgs& a, const uint16_t* a_lo,
                             uint16_t* out_lo, float* y32, hipStream_t s);
int prefill_ntiles_bf16(bool gate_up, int64_t I, int64_t H);

// A token's routed pairs as the fused prefill front end writes them, in top-k order:
// slot[t K + k] (-1: none), sel[t K + k] the expert (-1: none), val[t K + k] the masked
// affinity (the value the masked affinities hold for that expert).
struct CteTokPairs {
  const int32_t* slot;
  const int32_t* sel;
  const float* val;
  int K;
};

// The moe_cte flow (expert_prefill.hip): gate_up GEMM, down GEMM, combine over a blockwise
// mapping.  order_pre: the M-tile groups' schedule already computed (the fused prefill
// router writes it); null: computed from the mapping first.  pairs: the tokens' routed
// pairs (the fused prefill front end writes them; POST_SCALE and NO_SCALE only): the
// combine reads them instead of the (token, expert) -> slot inverse the gate_up GEMM
// otherwise writes; null: the inverse.
int cte_run(const uint16_t* x, const float* affinities_masked, const uint8_t* gu_q,
            const uint8_t* gu_s, const uint8_t* dn_q, const uint8_t* dn_s, int weight_fmt,
            const uint16_t* gu_bias, const uint16_t* dn_bias, const uint16_t* expert_const,
            const int32_t* token_position_to_id, const int32_t* block_to_expert,
            int64_t n_blocks, int64_t block_size, int64_t T, int64_t H, int64_t I, int64_t E,
            int act, const float* clamps, int scale_mode, int out_f32, void* out,
            void* workspace, size_t workspace_bytes, void* const* stage_events,
            const int2* order_pre, hipStream_t s, const CteTokPairs* pairs = nullptr);

}  // namespace mxmoe
