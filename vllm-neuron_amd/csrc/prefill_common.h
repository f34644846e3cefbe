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

}  // namespace mxmoe
