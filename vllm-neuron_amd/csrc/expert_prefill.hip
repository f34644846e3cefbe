// Prefill (context encoding) expert MLP over the blockwise mapping.
//
// Both projections run the same grouped GEMM:
//   workgroup tile = 128 slots (M) x 256 weight rows (N, 16 row groups) over all of K in
//   128-wide chunks; 4 waves, wave w owns row groups 4w..4w+3 (64 rows = 2 gate/up
//   pairs) against all 128 slots (up to 8 MFMA 16x16x32 tiles of 16 slots).  Two
//   workgroups share a CU (66 KB of LDS each, two waves per SIMD), so one computes
//   while the other waits at its barrier, loads its first chunks or stores its tile.
//   Weights bypass LDS: each wave streams its own rows global -> registers through a
//   ring of two chunks (the packed layout is MFMA operand order) and dequantizes them
//   once, with the CDNA4 scaled conversion, right before its MFMAs.
//   Activations are shared: the 128 slots' rows of a chunk (32 KiB of bf16, 16-byte
//   blocks XOR-swizzled by row against bank conflicts) go global -> LDS by direct
//   loads into a ring of two stages, one chunk ahead.  One s_barrier per chunk,
//   preceded by a wait for the wave's own direct loads of the chunk about to be read
//   only (a counted vmcnt, not the full drain of __syncthreads), keeps the weight and
//   activation streams in flight across chunks.  (The ring depth, the waves and row
//   groups per workgroup are the constants kPStages, kPWaves and PFmt below; four
//   stages of 512-row tiles with 8 waves, one workgroup per CU, measured 3 % slower.)
//   M-tiles never straddle blocks (block_size % 128 == 0) so one tile has one expert;
//   tiles whose 128 slots are all padding exit at once, and the waves run only the
//   16-slot tiles up to the last one holding a real slot (rounded to 1, 2, 4 or 8).
//   Scheduling: the grid's workgroups are dealt round-robin over the 8 XCDs, and each
//   XCD's CUs take its workgroups in order.  M-tiles are scheduled in groups (the tiles
//   of one block: 2 at block size 256).  XCD x runs group ranks x, x+8, x+16, ..., each
//   as group x n_ntiles consecutive workgroups, M-tile by M-tile (the workgroups sharing
//   activations or weight rows sit on one L2 at about the same time), where rank r is
//   the r-th group in an order computed on the device from token_position_to_id: most
//   16-slot subtiles first, all-padding groups last.
//   Every XCD gets an equal share of each group size, and the long groups start first
//   (a block of 256 slots holding ~130 tokens is one full tile and one nearly empty
//   one; in M order the empty tail blocks of the mapping would all land on the last
//   XCDs).
// gate_up: A = x rows gathered through token_position_to_id; epilogue = bias,
//          clamps, activation and up * act with the reference's bf16 roundings;
//          writes h [slots, I] bf16.
// down:    A = h rows of the same slots; epilogue = bias with bf16 roundings;
//          writes y [slots, H] bf16.
// combine: out[t] = bf16(sum over experts in ascending id of y * affinity) in fp32.
#include <math.h>

#include <type_traits>
#include <utility>

#include "capi_util.h"
#include "common.h"
#include "prefill_common.h"

namespace mxmoe {

constexpr int kPWaves = 4;
constexpr int kPThreads = 64 * kPWaves;
constexpr int kPDma = kPM / kPWaves / 4;      // direct loads (1 KiB = 4 rows) per wave and chunk

// Weight formats (MXMOE_WFMT_*): MXFP4 (e2m1 pairs, 16 B per lane, row group and 128-wide
// chunk) and MXFP8 (E4M3FN, 32 B per lane in two 16-B halves).  A wave holds 4 row groups
// of MXFP4 or 2 of MXFP8: both are four 16-B registers per chunk, so the register ring,
// the load counts and the waits are the same; an N-tile is 256 or 128 rows.
constexpr int kWFmt4 = 0, kWFmt8 = 1;
template <int F>
struct PFmt {
  static constexpr int RGW = F == kWFmt8 ? 2 : 4;        // row groups per wave
  static constexpr int RG = RGW * kPWaves;                // row groups per N-tile
  static constexpr uint32_t BYTES_PER_K = F == kWFmt8 ? 16u : 8u;  // of a row group
};
constexpr int kPBw = 4;  // 16-B weight registers per chunk and wave
constexpr int kPStages = 2;   // activation chunks in LDS (2 or 4)
constexpr int kPLead = kPStages - 1;  // chunks the direct loads run ahead

// Per-workgroup and per-wave constants of a tile.
struct PrefillTile {
  const char* a;             // activations
  const uint32_t* rowoff;    // LDS: byte offset of each tile row's source row (padding: a
                             // real row), re-read at every chunk (fewer live registers)
  uint32_t a_off[kPDma];     // the same for this lane's rows, in registers (PD = 0 loops)
  const uint8_t* wq;         // this wave's first row group
  const uint8_t* ws;         // this wave's scale quad
  uint32_t rg_bytes;
  int rv;                    // valid row groups of this wave (<= 4)
  int sbyte;                 // the wave's first row group in its scale quad (byte index)
  int K, nc, nfull, tail_q;
};

// One weight chunk of a wave in registers: kPBw x 16 B per lane (MXFP4: row group r in
// w[r]; MXFP8: half h of row group r in w[2r + h]), and the 32-bit scale word of the
// wave's quad of row groups.
struct PrefillB {
  u32x4 w[kPBw];
  uint32_t s[1];
};

// The activation stages are separate arrays of the kernel, chosen at compile time by a
// selector (stage(std::integral_constant<int, S>())): the compiler then tells the stage
// being read from the ones direct loads are filling; through a pointer, or with arrays
// shared by several kernels, it could not and would drain every load before each LDS
// read.
template <int S>
using StageC = std::integral_constant<int, S>;

// Direct loads of chunk c's activations into LDS: wave w brings its kPM / kPWaves rows,
// kPDma x 1 KiB (rows (kPM / kPWaves) w + 4i + lane / 16).  The lane's LDS slot
// (lane % 16) of row r holds
// column block (lane % 16) ^ (r % 16); columns past K read column 0 of the row.  Issued
// from inline assembly (M0 = the 1 KiB's LDS address, 16 B per lane, a 32-bit offset
// from the activations' base in a scalar register pair): the compiler then
// keeps no account of them, which it could only settle, across the loop, with a full
// drain before the stage's first LDS read; the counted barrier waits for them instead.
// The lane's source row offsets (ro): kept in registers by the loops whose fragment reads
// the compiler schedules (PD = 0), else read from LDS before the barrier that precedes
// the direct loads, so that their latency hides behind its wait.
template <int PD>
__device__ __forceinline__ void prefill_rowoffs(const PrefillTile& p, uint32_t (&ro)[kPDma]) {
  const int wave = wave_id(), lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < kPDma; ++i)
    ro[i] = PD == 0 ? p.a_off[i] : p.rowoff[(kPM / kPWaves) * wave + 4 * i + (lane >> 4)];
}

__device__ __forceinline__ void prefill_dma_one(uint8_t* sa, const PrefillTile& p, int c,
                                                const uint32_t (&ro)[kPDma], int i) {
  const int wave = wave_id(), lane = threadIdx.x & 63;
  const int swz = (lane & 15) ^ ((4 * i + (lane >> 4)) & 15);
  const int kcol = c * 128 + swz * 8;
  const uint32_t off = ro[i] + (kcol < p.K ? (uint32_t)kcol * 2u : 0u);
  uint8_t* dst = sa + ((kPM / kPWaves) * wave + 4 * i) * 256;
  const uint32_t lds = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)dst);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(off),
               "s"(p.a)
               : "memory", "m0");
}

__device__ __forceinline__ void prefill_dma(uint8_t* sa, const PrefillTile& p, int c,
                                            const uint32_t (&ro)[kPDma]) {
#pragma unroll
  for (int i = 0; i < kPDma; ++i) prefill_dma_one(sa, p, c, ro, i);
}

// The wave's weights and scales of chunk c (lanes past K re-read lane 0's bytes of the
// chunk, row groups past the tile re-read its last valid one, a quad past the tile the
// first quad's scales), kPLoadsB loads.  They are issued
// from inline assembly, so the compiler does not track them: with direct-to-LDS loads
// in flight as well it cannot count the wait for register loads and would drain every
// load (s_waitcnt vmcnt(0)) before their first use.  The compiler takes the outputs as
// written by the asm statement, while the hardware writes them later: every slot's
// registers must therefore stay operands of a later wait (prefill_wait_b before use,
// the loop's final drain for the last, unused refills), or the compiler could hand a
// register still being loaded to another value.
// Load k of the chunk (k < kPBw: weight register k, else the scale word of the quad).
// MXFP8: half h of chunk c of a row group at c * 2048 + h * 1024, or in a partial last
// chunk of tq blocks at nfull * 2048 + h * 256 tq.
template <int F>
__device__ __forceinline__ void prefill_load_b_one(PrefillB& f, const PrefillTile& p, int c,
                                                   int k) {
  const int lane = threadIdx.x & 63;
  const bool ok = (c < p.nfull) || ((lane >> 4) < p.tail_q);
  const uint32_t lo = ok ? (uint32_t)lane : 0u;
  if (k < kPBw) {
    const int r = F == kWFmt8 ? k >> 1 : k;
    const uint32_t rr = r < p.rv ? r : p.rv - 1;
    uint32_t coff;
    if constexpr (F == kWFmt8) {
      const uint32_t h = (uint32_t)(k & 1);
      coff = c < p.nfull ? (uint32_t)c * 2048u + h * 1024u
                         : (uint32_t)p.nfull * 2048u + h * 256u * (uint32_t)p.tail_q;
    } else {
      coff = (uint32_t)c * 1024u;
    }
    const uint8_t* base = p.wq + rr * p.rg_bytes + coff;
    asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(f.w[k]) : "v"(lo * 16u), "s"(base)
                 : "memory");
  } else {
    const uint8_t* sbase = p.ws + (uint32_t)c * 256u;
    asm volatile("global_load_dword %0, %1, %2" : "=v"(f.s[0]) : "v"(lo * 4u), "s"(sbase)
                 : "memory");
  }
}

constexpr int kPLoadsB = kPBw + 1;  // loads per chunk and wave: weights, scales

template <int F>
__device__ __forceinline__ void prefill_load_b(PrefillB& f, const PrefillTile& p, int c) {
#pragma unroll
  for (int k = 0; k < kPLoadsB; ++k) prefill_load_b_one<F>(f, p, c, k);
}

// Waits until at most N vector memory operations issued after slot f's loads are
// outstanding (loads retire in issue order); the registers are operands, so no use of
// them moves above the wait.
template <int N>
__device__ __forceinline__ void prefill_wait_b(PrefillB& f) {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  static_assert(kPBw == 4, "the operands below are the ring slot's registers");
  asm volatile("s_waitcnt vmcnt(%5)"
               : "+v"(f.w[0]), "+v"(f.w[1]), "+v"(f.w[2]), "+v"(f.w[3]), "+v"(f.s[0])
               : "n"(N)
               : "memory");
}

// Eight MXFP8 (E4M3FN) bytes of two 32-bit words, times the block scale, to bf16 with the
// CDNA4 scaled conversion (two elements per instruction, low 16-bit word first).
__device__ __forceinline__ bf16x8 dequant8_fp8(uint32_t w0, uint32_t w1, float scale) {
  bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, false);
  bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, true);
  bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, false);
  bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, true);
  bf16x8 r = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
  return r;
}

// Row group r's eight weights of MFMA step j in the chunk held by f.
template <int F>
__device__ __forceinline__ bf16x8 prefill_deq(const PrefillB& f, int r, int j, float sc) {
  if constexpr (F == kWFmt8) {
    const u32x4& w = f.w[2 * r + (j >> 1)];
    return dequant8_fp8(w[2 * (j & 1)], w[2 * (j & 1) + 1], sc);
  } else {
    return dequant8(f.w[r][j], sc);
  }
}

struct NoHook {
  __device__ void operator()(int) const {}
};

// acc[r][t] += W[row group r] x A[16-slot tile t] over chunk c.  Lanes past K get a zero
// scale, so their weights add exact zeros.  The compiler-scheduled loop (PD = 0) calls
// hook(i) after the MFMAs of each (step j, fragment t), i = NT j + t: the caller issues its
// loads for later chunks from there, between MFMA groups, instead of in one burst.
template <int F, int NT, int PD, typename Hook = NoHook>
__device__ __forceinline__ void prefill_compute(const uint8_t* sa, const PrefillB& f,
                                                const PrefillTile& p, int c,
                                                f32x4 (&acc)[PFmt<F>::RGW][NT],
                                                const Hook& hook = Hook()) {
  constexpr int RGW = PFmt<F>::RGW;
  const int lane = threadIdx.x & 63, q = lane >> 4;
  const bool kok = (c < p.nfull) || (q < p.tail_q);
  float sc[RGW];
#pragma unroll
  for (int r = 0; r < RGW; ++r)
    sc[r] = kok ? e8m0_to_f32((f.s[0] >> (8 * (p.sbyte + r))) & 0xffu) : 0.0f;
  // Per 32-wide step j: the row groups' weights dequantized once, then the NT activation
  // fragments against them.  The fragments are read from LDS PD steps (j, t) ahead, into
  // a rotating set of registers, so each read has the MFMAs of PD steps to land in.
  if constexpr (PD == 0) {
    // Left to the compiler's schedule (it reads two fragments ahead).
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int blk = (4 * q + j) ^ (lane & 15);
      bf16x8 wf[RGW];
#pragma unroll
      for (int r = 0; r < RGW; ++r) wf[r] = prefill_deq<F>(f, r, j, sc[r]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const u32x4 xv =
            *reinterpret_cast<const u32x4*>(sa + (16 * t + (lane & 15)) * 256 + blk * 16);
#pragma unroll
        for (int r = 0; r < RGW; ++r) acc[r][t] = mfma16(wf[r], as_bf16x8(xv), acc[r][t]);
        hook(NT * j + t);
      }
    }
  } else {
    constexpr int NS = 4 * NT;
    static_assert(PD >= 1 && PD <= NS, "read-ahead distance");
    const uint8_t* rowp = sa + (lane & 15) * 256;
    auto frag = [&](int i) {
      const int j = i / NT, t = i % NT;
      const int blk = (4 * q + j) ^ (lane & 15);
      return *reinterpret_cast<const u32x4*>(rowp + 16 * t * 256 + blk * 16);
    };
    u32x4 xb[PD];
#pragma unroll
    for (int i = 0; i < PD; ++i) xb[i] = frag(i);
    bf16x8 wf[RGW];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      if (i % NT == 0) {
#pragma unroll
        for (int r = 0; r < RGW; ++r) wf[r] = prefill_deq<F>(f, r, i / NT, sc[r]);
      }
      const u32x4 x = xb[i % PD];
      if (i + PD < NS) xb[i % PD] = frag(i + PD);
#pragma unroll
      for (int r = 0; r < RGW; ++r) acc[r][i % NT] = mfma16(wf[r], as_bf16x8(x), acc[r][i % NT]);
    }
    // The compiler's scheduler would pull the reads back next to their MFMAs; these groups
    // keep the order: PD reads, then per step four MFMAs and the read PD steps ahead.
    __builtin_amdgcn_sched_group_barrier(0x100, PD, 0);
#pragma unroll
    for (int i = 0; i < NS - PD; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, RGW, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int i = 0; i < PD; ++i) __builtin_amdgcn_sched_group_barrier(0x008, RGW, 0);
  }
}

// Waits until at most N vector memory operations of this wave are outstanding (loads
// retire in issue order), then for its LDS operations, then meets the other waves.
// Unlike __syncthreads() it does not drain the loads issued for later chunks.
template <int N>
__device__ __forceinline__ void prefill_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// One chunk: chunk c is in stage S % kPStages.  Issue order (the vmcnt arithmetic
// depends on it), with D = kPDma direct loads and L = kPLoadsB weight and
// scale loads per chunk and P = kPLead:
// prologue: weights of chunks 0 and 1 (2 x L), direct loads of chunks 0 .. P - 1 (P x D);
// step c: [barrier] direct loads of chunk c + P (D), [wait] the MFMAs of chunk c, the
// weights of chunk c + 2 (L).
//  - barrier: chunk c's direct loads have landed once at most (P - 1) D later loads are
//    outstanding at step 0 and (P - 1) D + L at later steps (exactly that at step 1,
//    more later: the wait then also covers older loads); a wave without weights issues
//    direct loads only: (P - 1) D at every step;
//  - weights of chunk c: at most 2D + L later loads outstanding (exactly that from step
//    2 on; steps 0 and 1 wait a little longer, once).
// The compiler-scheduled loop (PD = 0, one lead chunk) issues the same loads in the same
// order, spread between its MFMA groups: step c: [barrier] [wait] the MFMAs of chunk c
// with direct load i of chunk c + 1 after MFMA group 2i (i < D) and weight load k of chunk
// c + 2 after group 3 NT + k (k < L), once step j = 3 has dequantized the slot they refill.
// The barrier counts are unchanged; the weights of chunk c then wait with D + L later
// loads outstanding (exactly that from step 2 on, more at step 1; the same at step 0).
// A wave that issues its loads in bursts leaves its MFMA slots idle while they issue; with
// the loads between MFMA groups the two waves of a SIMD keep it busier (gate_up GEMM at
// 4096 tokens of the 120B-shaped layer: about 5 % faster).
constexpr int kPWaitFirst = (kPLead - 1) * kPDma;
constexpr int kPWait = (kPLead - 1) * kPDma + kPLoadsB;
constexpr int kPWaitB = 2 * kPDma + kPLoadsB;
constexpr int kPWaitBSpread = kPDma + kPLoadsB;
template <int F, int S, int NT, bool ACTIVE, bool FIRST, int PD, typename Stage>
__device__ __forceinline__ void prefill_step(const Stage& stage, PrefillB (&f)[2],
                                             const PrefillTile& p, int c,
                                             f32x4 (&acc)[PFmt<F>::RGW][NT]) {
  uint32_t ro[kPDma];
  prefill_rowoffs<PD>(p, ro);
  prefill_barrier<(FIRST || !ACTIVE) ? kPWaitFirst : kPWait>();
  if constexpr (ACTIVE && PD == 0) {
    static_assert(kPLead == 1 && 2 * kPDma <= 3 * NT, "spread loads: one lead chunk, "
                  "direct loads before the weights");
    uint8_t* next = stage(StageC<(S + 1) % kPStages>());
    const int cn = min(c + 1, p.nc - 1), cw = min(c + 2, p.nc - 1);
    prefill_wait_b<kPWaitBSpread>(f[S % 2]);
    auto hook = [&](int i) {
      if (i % 2 == 0 && i / 2 < kPDma) prefill_dma_one(next, p, cn, ro, i / 2);
      if (i >= 3 * NT && i - 3 * NT < kPLoadsB) prefill_load_b_one<F>(f[S % 2], p, cw, i - 3 * NT);
    };
    prefill_compute<F, NT, PD>(stage(StageC<S % kPStages>()), f[S % 2], p, c, acc, hook);
    __builtin_amdgcn_sched_barrier(0);
    return;
  }
  prefill_dma(stage(StageC<(S + kPLead) % kPStages>()), p, min(c + kPLead, p.nc - 1), ro);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (ACTIVE) {
    prefill_wait_b<kPWaitB>(f[S % 2]);
    prefill_compute<F, NT, PD>(stage(StageC<S % kPStages>()), f[S % 2], p, c, acc);
    __builtin_amdgcn_sched_barrier(0);
    prefill_load_b<F>(f[S % 2], p, min(c + 2, p.nc - 1));
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int F, int NT, bool ACTIVE, int PD, typename Stage>
__device__ __forceinline__ void prefill_loop(const Stage& stage, const PrefillTile& p,
                                             f32x4 (&acc)[PFmt<F>::RGW][NT]) {
  PrefillB f[2];
  if constexpr (ACTIVE) {
    prefill_load_b<F>(f[0], p, 0);
    prefill_load_b<F>(f[1], p, min(1, p.nc - 1));
  }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t ro[kPDma];
  prefill_rowoffs<PD>(p, ro);
  prefill_dma(stage(StageC<0>()), p, 0, ro);
  if constexpr (kPLead > 1) prefill_dma(stage(StageC<1>()), p, min(1, p.nc - 1), ro);
  if constexpr (kPLead > 2) prefill_dma(stage(StageC<2>()), p, min(2, p.nc - 1), ro);
  __builtin_amdgcn_sched_barrier(0);
  prefill_step<F, 0, NT, ACTIVE, true, PD>(stage, f, p, 0, acc);
  int c = 1;
  for (; c + 4 <= p.nc; c += 4) {
    prefill_step<F, 1, NT, ACTIVE, false, PD>(stage, f, p, c, acc);
    prefill_step<F, 2, NT, ACTIVE, false, PD>(stage, f, p, c + 1, acc);
    prefill_step<F, 3, NT, ACTIVE, false, PD>(stage, f, p, c + 2, acc);
    prefill_step<F, 0, NT, ACTIVE, false, PD>(stage, f, p, c + 3, acc);
  }
  if (c < p.nc) {
    prefill_step<F, 1, NT, ACTIVE, false, PD>(stage, f, p, c, acc);
    if (c + 1 < p.nc) {
      prefill_step<F, 2, NT, ACTIVE, false, PD>(stage, f, p, c + 1, acc);
      if (c + 2 < p.nc) prefill_step<F, 3, NT, ACTIVE, false, PD>(stage, f, p, c + 2, acc);
    }
  }
  // The loads issued past the last chunk (clamped re-loads) land before the wave goes
  // on: no direct load may still write into LDS once the workgroup is done with it, and
  // the ring's registers are operands here, so the compiler keeps them allocated until
  // their last (unused) loads have written them.
  if constexpr (ACTIVE) {
    prefill_wait_b<0>(f[0]);
    prefill_wait_b<0>(f[1]);
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

// Tiles with 1 or 2 subtiles of 16 slots (a block's nearly empty second tile) have little
// to compute per chunk, so a chunk costs about one load latency.  They run a loop of their
// own: only their 16 NT rows of activations go to LDS, in a ring of kLStages slices of the
// 64 KB the full tiles use as two stages, kLLead chunks ahead; the weights go through a
// ring of kLSlots register chunks (their accumulators leave the registers free), kLSlots
// chunks ahead.  Wave w brings rows 4 (w + 4j) .. 4 (w + 4j) + 3, j < NT.
constexpr int kLLead = 7, kLStages = 8, kLSlots = 8;
static_assert(kLStages > kLLead && (kLStages & (kLStages - 1)) == 0, "light ring");
// The light loop's direct loads give wave w rows 4 (w + 4 j) of subtile j: exactly the
// 16 NT rows of a ring slice with 4 waves.  Any other wave count writes past the slice
// (and past the workgroup's LDS in the last slice of a 2-subtile ring).
static_assert(kPWaves == 4, "the light loop maps each 16-row subtile onto 4 waves");

template <int NT>
__device__ __forceinline__ void prefill_rowoffs_light(const PrefillTile& p, uint32_t (&ro)[NT]) {
  const int wave = wave_id(), lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < NT; ++j) ro[j] = p.rowoff[4 * (wave + 4 * j) + (lane >> 4)];
}

template <int NT>
__device__ __forceinline__ void prefill_dma_light(uint8_t* ring, int slot, const PrefillTile& p,
                                                  int c, const uint32_t (&ro)[NT]) {
  const int wave = wave_id(), lane = threadIdx.x & 63;
  uint8_t* sa = ring + slot * (16 * NT * 256);
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int r4 = 4 * (wave + 4 * j);
    const int swz = (lane & 15) ^ ((r4 + (lane >> 4)) & 15);
    const int kcol = c * 128 + swz * 8;
    const uint32_t off = ro[j] + (kcol < p.K ? (uint32_t)kcol * 2u : 0u);
    uint8_t* dst = sa + r4 * 256;
    const uint32_t lds = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)dst);
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(off),
                 "s"(p.a)
                 : "memory", "m0");
  }
}

// One chunk of the light loop, chunk c in slice c % kLStages and weight slot SB = c %
// kLSlots.  Issue order: prologue: weights of chunks 0 .. kLSlots - 1 (kLSlots x L), direct
// loads of chunks 0 .. kLLead - 1 (kLLead x D); step c: [barrier] direct loads of chunk
// c + kLLead (D), [wait] the MFMAs of chunk c, the weights of chunk c + kLSlots (L); D = NT,
// L = kPLoadsB (0 for a wave without weights).
//  - barrier: chunk c's direct loads have landed once at most (kLLead - 1) D + min(c,
//    kLLead) L later loads are outstanding (exact at every step: BAR);
//  - weights of chunk c: at most kLSlots D + (kLSlots - 1) L (exact from step kLSlots on,
//    a little longer before).
template <int F, int SB, int NT, bool ACTIVE, int BAR>
__device__ __forceinline__ void prefill_step_light(uint8_t* ring, PrefillB (&f)[kLSlots],
                                                   const PrefillTile& p, int c,
                                                   f32x4 (&acc)[PFmt<F>::RGW][NT]) {
  uint32_t ro[NT];
  prefill_rowoffs_light<NT>(p, ro);
  prefill_barrier<BAR>();
  prefill_dma_light<NT>(ring, (c + kLLead) & (kLStages - 1), p, min(c + kLLead, p.nc - 1), ro);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (ACTIVE) {
    prefill_wait_b<kLSlots * NT + (kLSlots - 1) * kPLoadsB>(f[SB]);
    prefill_compute<F, NT, NT>(ring + (c & (kLStages - 1)) * (16 * NT * 256), f[SB], p, c, acc);
    __builtin_amdgcn_sched_barrier(0);
    prefill_load_b<F>(f[SB], p, min(c + kLSlots, p.nc - 1));
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Steps c + I .. c + N - 1 of the light loop, chunk c + i in weight slot (S0 + i) %
// kLSlots with barrier count B + i DB, nested so that a step runs only after the one
// before it and then() only after all of them (every path of the control flow issues the
// loads in the order the counts assume).
template <int F, int NT, bool ACTIVE, int S0, int B, int DB, int I, int N, typename Then>
__device__ __forceinline__ void prefill_light_tail(uint8_t* ring, PrefillB (&f)[kLSlots],
                                                   const PrefillTile& p, int c,
                                                   f32x4 (&acc)[PFmt<F>::RGW][NT],
                                                   const Then& then) {
  if constexpr (I < N) {
    if (c + I < p.nc) {
      prefill_step_light<F, (S0 + I) % kLSlots, NT, ACTIVE, B + I * DB>(ring, f, p, c + I, acc);
      prefill_light_tail<F, NT, ACTIVE, S0, B, DB, I + 1, N>(ring, f, p, c, acc, then);
    }
  } else {
    then();  // every step ran
  }
}

// kLSlots steps c .. c + kLSlots - 1 (all run), slot (S0 + i) % kLSlots, barrier count B.
template <int F, int NT, bool ACTIVE, int S0, int B, int... Is>
__device__ __forceinline__ void prefill_light_block(uint8_t* ring, PrefillB (&f)[kLSlots],
                                                    const PrefillTile& p, int c,
                                                    f32x4 (&acc)[PFmt<F>::RGW][NT],
                                                    std::integer_sequence<int, Is...>) {
  (prefill_step_light<F, (S0 + Is) % kLSlots, NT, ACTIVE, B>(ring, f, p, c + Is, acc), ...);
}

template <int F, int NT, bool ACTIVE>
__device__ __forceinline__ void prefill_loop_light(uint8_t* ring, const PrefillTile& p,
                                                   f32x4 (&acc)[PFmt<F>::RGW][NT]) {
  constexpr int D = NT, L = ACTIVE ? kPLoadsB : 0, B0 = (kLLead - 1) * D;
  static_assert(B0 + kLLead * L < 64 && kLSlots * D + (kLSlots - 1) * L < 64, "vmcnt range");
  static_assert(kLSlots == kLStages && kLLead + 1 == kLSlots, "slots and slices cycle together");
  PrefillB f[kLSlots];
  if constexpr (ACTIVE) {
#pragma unroll
    for (int s = 0; s < kLSlots; ++s) prefill_load_b<F>(f[s], p, min(s, p.nc - 1));
  }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t ro[NT];
  prefill_rowoffs_light<NT>(p, ro);
#pragma unroll
  for (int v = 0; v < kLLead; ++v) prefill_dma_light<NT>(ring, v, p, min(v, p.nc - 1), ro);
  __builtin_amdgcn_sched_barrier(0);
  // Steps 0 .. kLLead - 1 have their own barrier counts (every path issues the loads in the
  // order the counts assume), then blocks of kLSlots steps with the steady count.
  constexpr int BS = B0 + kLLead * L;
  auto steady = [&]() {
    int c = kLLead;
    for (; c + kLSlots <= p.nc; c += kLSlots)
      prefill_light_block<F, NT, ACTIVE, kLLead, BS>(ring, f, p, c, acc,
                                                     std::make_integer_sequence<int, kLSlots>());
    prefill_light_tail<F, NT, ACTIVE, kLLead, BS, 0, 0, kLSlots - 1>(ring, f, p, c, acc,
                                                                     [] {});
  };
  prefill_light_tail<F, NT, ACTIVE, 0, B0, L, 0, kLLead>(ring, f, p, 0, acc, steady);
  // As in prefill_loop: every load has landed before the wave goes on, and the ring's
  // registers are operands of the final wait.
  if constexpr (ACTIVE) {
#pragma unroll
    for (int s = 0; s < kLSlots; ++s) prefill_wait_b<0>(f[s]);
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

// gate_up epilogue: bias, clamps and the activation on the bf16-rounded accumulators
// (the reference's bf16 intermediates), h = up * act(gate) stored as bf16.
template <int F, int ACT, int NT>
__device__ __forceinline__ void gate_up_store(const PrefillArgs& args, const PrefillTile& p,
                                              const f32x4 (&acc)[PFmt<F>::RGW][NT],
                                              const float (&gb)[PFmt<F>::RGW / 2][4],
                                              const float (&ub)[PFmt<F>::RGW / 2][4],
                                              const int32_t* stok, int m0, int rg_first) {
  typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63, q = lane >> 4;
  const int I = args.I;
#pragma unroll
  for (int pp = 0; pp < PFmt<F>::RGW / 2; ++pp) {
    if (2 * pp >= p.rv) continue;
    const int P = rg_first / 2 + pp;  // pair index = 16 intermediate columns
    const int col0 = 16 * P + 4 * q;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int row = 16 * t + (lane & 15);
      if (stok[row] < 0) continue;
      const f32x4 g4 = acc[2 * pp][t], u4 = acc[2 * pp + 1][t];
      float h[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float g = rb(g4[i]), u = rb(u4[i]);
        if (args.bias) {
          g = rb(g + gb[pp][i]);
          u = rb(u + ub[pp][i]);
        }
        g = clamp_ref(g, args.p.gate_lo, args.p.gate_hi);
        u = clamp_ref(u, args.p.up_lo, args.p.up_hi);
        h[i] = u * act_bf16<ACT>(g);
      }
      *reinterpret_cast<u32x2*>(args.out + (size_t)(m0 + row) * I + col0) =
          u32x2{pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3])};
    }
  }
}

template <int F, bool GATE_UP, int NT, bool LIGHT, typename Stage>
__device__ __forceinline__ void prefill_run(const Stage& stage, uint8_t* ring,
                                            const PrefillArgs& args, const PrefillTile& p,
                                            const int32_t* stok, int m0, int e, int rg_first) {
  constexpr int RGW = PFmt<F>::RGW;
  f32x4 acc[RGW][NT];
#pragma unroll
  for (int r = 0; r < RGW; ++r)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (LIGHT)
    prefill_loop_light<F, NT, true>(ring, p, acc);
  else
    // LDS read-ahead distance: 4 steps (NT steps for 1-2 subtiles); the gate_up 8-subtile
    // loop has no registers left for it and keeps the compiler's schedule (0).
    prefill_loop<F, NT, true, GATE_UP && NT == 8 ? 0 : (NT < 4 ? NT : 4)>(stage, p, acc);

  const int lane = threadIdx.x & 63, q = lane >> 4;
  typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
  // The epilogues load their biases first, all in flight together: unconditional loads
  // (a missing bias or a column past the tile reads element 0 of a valid array) and no
  // store before them (the compiler cannot tell the output from the bias, and would
  // wait for every store before a later bias load).
  const uint16_t* bsrc = args.bias ? args.bias : reinterpret_cast<const uint16_t*>(args.wq);
  if (GATE_UP) {
    const int I = args.I;
    float gb[RGW / 2][4], ub[RGW / 2][4];
#pragma unroll
    for (int pp = 0; pp < RGW / 2; ++pp) {
      const int col0 = 16 * (rg_first / 2 + pp) + 4 * q;
      const bool ok = args.bias && 2 * pp < p.rv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const size_t ig = ok ? (size_t)e * 2 * I + col0 + i : 0;
        const size_t iu = ok ? (size_t)e * 2 * I + I + col0 + i : 0;
        gb[pp][i] = bf16_bits_to_f32(bsrc[ig]);
        ub[pp][i] = bf16_bits_to_f32(bsrc[iu]);
      }
    }
    // The activation is uniform: one dispatch, then straight-line code per element.
    if (args.p.act == kSwish)
      gate_up_store<F, kSwish>(args, p, acc, gb, ub, stok, m0, rg_first);
    else if (args.p.act == kSiLU)
      gate_up_store<F, kSiLU>(args, p, acc, gb, ub, stok, m0, rg_first);
    else
      gate_up_store<F, kGELU>(args, p, acc, gb, ub, stok, m0, rg_first);
  } else {
    const int H = args.H;
    float bb[RGW][4];
#pragma unroll
    for (int r = 0; r < RGW; ++r) {
      const int n0 = 16 * (rg_first + r) + 4 * q;
      const bool ok = args.bias && r < p.rv;
#pragma unroll
      for (int i = 0; i < 4; ++i) bb[r][i] = bf16_bits_to_f32(bsrc[ok ? (size_t)e * H + n0 + i : 0]);
    }
#pragma unroll
    for (int r = 0; r < RGW; ++r) {
      if (r >= p.rv) continue;
      const int n0 = 16 * (rg_first + r) + 4 * q;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int row = 16 * t + (lane & 15);
        if (stok[row] < 0) continue;
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          y[i] = acc[r][t][i];
          if (args.bias) y[i] = rb(rb(y[i]) + bb[r][i]);
        }
        *reinterpret_cast<u32x2*>(args.out + (size_t)(m0 + row) * H + n0) =
            u32x2{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
      }
    }
  }
}

template <bool GATE_UP, int F>
__global__ void __launch_bounds__(kPThreads)
    __attribute__((amdgpu_waves_per_eu(2, 2))) prefill_gemm_kernel(
        PrefillArgs args) {
  constexpr int RGW = PFmt<F>::RGW, RG = PFmt<F>::RG;
  constexpr int kS23 = kPStages == 4 ? kPM * 256 : 16;  // stages 2 and 3 exist with 4 stages
  __shared__ __attribute__((aligned(1024))) uint8_t sa01[2][kPM * 256], sa2[kS23], sa3[kS23];
  __shared__ int32_t stok[kPM];
  __shared__ uint32_t s_rowoff[kPM];
  __shared__ int s_lastw[kPM / 64];  // per wave of slots: last slot holding a real token, or -1
  auto stage = [&](auto s_c) -> uint8_t* {
    constexpr int S = decltype(s_c)::value;
    if constexpr (S == 0) return sa01[0];
    else if constexpr (S == 1) return sa01[1];
    else if constexpr (S == 2) return sa2;
    else return sa3;
  };

  PrefillTileId id;
  if (!prefill_tile_begin<GATE_UP>(args, stok, s_rowoff, s_lastw, id)) return;
  const int m0 = id.m0, e = id.e, nt = id.nt;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  __syncthreads();
  const int last = max(s_lastw[0], s_lastw[1]);
  if (last < 0) return;

  PrefillTile p;
  p.K = args.K;
  p.rg_bytes = (uint32_t)p.K * PFmt<F>::BYTES_PER_K;
  const int n_rg_total = args.N_rows / 16;
  const int rg0 = nt * RG;  // a multiple of 4: the tile holds whole scale quads
  const int rg_valid = min(RG, n_rg_total - rg0);
  const int rg_first = rg0 + RGW * wave;
  p.rv = min(RGW, rg_valid - RGW * wave);
  const int rgw = p.rv > 0 ? rg_first : rg0;  // waves without rows point at valid data
  p.wq = args.wq + ((size_t)e * n_rg_total + rgw) * p.rg_bytes;
  p.ws = args.ws + ((size_t)e * ((n_rg_total + 3) / 4) + rgw / 4) * (size_t)(2 * p.K);
  p.sbyte = rgw % 4;
  p.nc = (p.K + 127) / 128;
  p.nfull = p.K / 128;
  p.tail_q = (p.K % 128) / 32;
  p.a = reinterpret_cast<const char*>(args.a);
  p.rowoff = s_rowoff;
  const int ntiles = last / 16 + 1;  // real slots of a block come first
  if (ntiles <= 2) {
    uint8_t* ring = &sa01[0][0];
    if (p.rv <= 0) {
      if (ntiles <= 1) {
        f32x4 none[RGW][1];
        prefill_loop_light<F, 1, false>(ring, p, none);
      } else {
        f32x4 none[RGW][2];
        prefill_loop_light<F, 2, false>(ring, p, none);
      }
      return;
    }
    if (ntiles <= 1)
      prefill_run<F, GATE_UP, 1, true>(stage, ring, args, p, stok, m0, e, rg_first);
    else
      prefill_run<F, GATE_UP, 2, true>(stage, ring, args, p, stok, m0, e, rg_first);
    return;
  }
#pragma unroll
  for (int i = 0; i < kPDma; ++i) p.a_off[i] = s_rowoff[(kPM / kPWaves) * wave + 4 * i + (lane >> 4)];
  if (p.rv <= 0) {
    // No row groups in this tile for this wave: it still brings its share of the
    // activations and meets the barriers.
    f32x4 none[RGW][1];
    prefill_loop<F, 1, false, 1>(stage, p, none);
    return;
  }
  if (ntiles <= 4)
    prefill_run<F, GATE_UP, 4, false>(stage, nullptr, args, p, stok, m0, e, rg_first);
  else
    prefill_run<F, GATE_UP, 8, false>(stage, nullptr, args, p, stok, m0, e, rg_first);
}

// The order of the groups of G M-tiles both GEMMs run.  The tiles' weights and experts
// are read once into LDS (dynamic: 5 B per tile).
__global__ void __launch_bounds__(kOrderThreads) cte_tile_order_kernel(
    const int32_t* __restrict__ tp2id, const int32_t* __restrict__ b2e, int B, int n_mtiles,
    int G, int T, int2* __restrict__ order) {
  extern __shared__ __attribute__((aligned(16))) uint8_t order_dyn[];
  int32_t* s_e = reinterpret_cast<int32_t*>(order_dyn);
  uint8_t* s_w = order_dyn + 4 * (size_t)n_mtiles;
  __shared__ OrderLds L;
  for (int mt = threadIdx.x; mt < n_mtiles; mt += kOrderThreads) {
    s_w[mt] = (uint8_t)tile_weight(tp2id, mt, T);
    s_e[mt] = b2e[(size_t)mt * kPM / B];
  }
  __syncthreads();
  order_pass(s_w, s_e, n_mtiles / G, G, order, L);
}

// inv[t, e] = slot of (t, e) or -1.
// The slot of (token t, expert e), or -1: inv[t * E + e] as the gate_up GEMM wrote it for
// the routed pairs, checked against the mapping (slot in range, its token t and its
// block's expert e), so that stale entries of unrouted pairs count as none and inv needs
// no clearing before a call.
__device__ __forceinline__ int cte_slot_of(const int32_t* __restrict__ inv,
                                           const int32_t* __restrict__ tp2id,
                                           const int32_t* __restrict__ b2e, int64_t n_slots, int B,
                                           int t, int e, int E) {
  const int s = inv[(size_t)t * E + e];
  if (s < 0 || (int64_t)s >= n_slots) return -1;
  return (tp2id[s] == t && b2e[s / B] == e) ? s : -1;
}

// out[t, n] = bf16(sum_e float(y[inv[t,e], n]) * aff[t*E + e]) for e ascending.  One wave
// per token, four tokens per workgroup: the wave compacts the token's (slot, weight) pairs
// in ascending expert order from its row of inv (a ballot per 64 experts) into its own
// LDS list, then each lane sums its 8-column groups over that list.  All of a
// workgroup's tokens are in flight at once (one round of workgroups on the chip at 4096
// tokens), so the dependent loads (inv, mapping, weights, rows of y) overlap.
constexpr int kCombineThreads = 256;
constexpr int kCombineTok = kCombineThreads / 64;
constexpr int kCteMaxE = 1024;
template <typename YT>  // y element: bf16 bits (prefill flow) or fp32 (decode flow)
__global__ void __launch_bounds__(kCombineThreads) cte_combine_kernel(
    const YT* __restrict__ y, const int32_t* __restrict__ inv,
    const int32_t* __restrict__ tp2id, const int32_t* __restrict__ b2e, int64_t n_slots, int B,
    const float* __restrict__ aff, int T, int H, int E, int scale_mode, int out_f32,
    void* __restrict__ out) {
  __shared__ int s_slot[kCombineTok][kCteMaxE];
  __shared__ float s_w[kCombineTok][kCteMaxE];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * kCombineTok + wave;
  const bool live = t < T;
  const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int cnt = 0;
  if (live) {
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const int sl = e < E ? cte_slot_of(inv, tp2id, b2e, n_slots, B, t, e, E) : -1;
      const unsigned long long m = __ballot(sl >= 0);
      if (sl >= 0) {
        const int pos = cnt + __popcll(m & below);
        s_slot[wave][pos] = sl;
        s_w[wave][pos] = scale_mode == MXMOE_SCALE_NO ? 1.0f : aff[(size_t)t * E + e];
      }
      cnt += __popcll(m);
    }
  }
  __syncthreads();
  if (!live) return;
  typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
  for (int n = lane * 8; n < H; n += 64 * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int k = 0; k < cnt; ++k) {
      const float a = s_w[wave][k];
      const YT* row = y + (size_t)s_slot[wave][k] * H + n;
      float v[8];
      if constexpr (sizeof(YT) == 2) {
        const u16x8 b = *reinterpret_cast<const u16x8*>(row);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = bf16_bits_to_f32(b[i]);
      } else {
        const f32x4 lo = *reinterpret_cast<const f32x4*>(row);
        const f32x4 hi = *reinterpret_cast<const f32x4*>(row + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] = lo[i];
          v[4 + i] = hi[i];
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = __fadd_rn(acc[i], __fmul_rn(v[i], a));
    }
    if (out_f32) {
      float* o = static_cast<float*>(out) + (size_t)t * H + n;
      *reinterpret_cast<f32x4*>(o) = f32x4{acc[0], acc[1], acc[2], acc[3]};
      *reinterpret_cast<f32x4*>(o + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
    } else {
      u16x8 r;
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = f32_to_bf16_bits(acc[i]);
      *reinterpret_cast<u16x8*>(static_cast<uint16_t*>(out) + (size_t)t * H + n) = r;
    }
  }
}

// The same combine from the tokens' pairs as the fused prefill front end lists them (slot,
// expert, masked affinity; at most 8, in top-k order): each wave sorts its token's pairs
// by expert id (scalar registers: the token is the wave's), then sums the rows of y in
// that order exactly as cte_combine_kernel does.  No inverse and no mapping reads: the
// rows of y are the only dependent loads.
// KM: the largest top-k the instance serves (4 or 8); the pair entries and the rows of y are
// loaded unconditionally (entries past K re-read entry 0, rows past the token's pairs
// re-read its first row), so that each batch of loads issues together and is waited for
// once: loads under per-entry conditions were each waited for on their own.
// NG: column groups of 512 per pass (each lane 8 columns of a group, KM rows of each in
// flight): 6 at top-4 covers H <= 3,072 in one pass, so a token's rows are one round trip.
template <int KM, int NG>
__global__ void __launch_bounds__(kCombineThreads) cte_combine_tok_kernel(
    const uint16_t* __restrict__ y, const int32_t* __restrict__ tslot,
    const int32_t* __restrict__ tsel, const float* __restrict__ tval, int T, int H, int K,
    int scale_mode, int out_f32, void* __restrict__ out) {
  static_assert(KM == 4 || KM == 8, "pairs per token");
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * kCombineTok + wave_id();
  if (t >= T) return;
  // Lane k < KM loads entry k; the values are then taken into scalar registers.
  const size_t li = (size_t)t * K + (lane < K ? lane : 0);
  const int le = tsel[li], ls = tslot[li];
  const float lw = tval[li];
  int es[KM], ss[KM];
  float ws[KM];
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    const int e = __builtin_amdgcn_readlane(le, k), sl = __builtin_amdgcn_readlane(ls, k);
    const bool ok = k < K && e >= 0 && sl >= 0;
    es[k] = ok ? e : 0x7fffffff;  // pairs that are none sort last
    ss[k] = ok ? sl : 0;
    ws[k] = scale_mode == MXMOE_SCALE_NO ? 1.0f
                                         : __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                                         __builtin_bit_cast(int, lw), k));
  }
  // ascending expert id (ids are distinct): a transposition sort
#pragma unroll
  for (int i = 0; i < KM; ++i)
#pragma unroll
    for (int j = (i & 1); j + 1 < KM; j += 2)
      if (es[j] > es[j + 1]) {
        const int te = es[j], tsl = ss[j];
        const float tw = ws[j];
        es[j] = es[j + 1];
        ss[j] = ss[j + 1];
        ws[j] = ws[j + 1];
        es[j + 1] = te;
        ss[j + 1] = tsl;
        ws[j + 1] = tw;
      }
  int cnt = 0;
#pragma unroll
  for (int k = 0; k < KM; ++k) cnt += es[k] != 0x7fffffff ? 1 : 0;
  // NG column groups of 8 per lane and pass, KM rows each: all NG x KM loads in flight.
  static_assert(NG * KM <= 24, "rows in flight per lane (registers)");
  typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
  for (int n = lane * 8; n < H; n += 64 * 8 * NG) {
    u16x8 b[NG][KM];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int ng = n + 512 * g < H ? n + 512 * g : n;  // a group past H re-reads group 0
#pragma unroll
      for (int k = 0; k < KM; ++k)
        b[g][k] = *reinterpret_cast<const u16x8*>(y + (size_t)ss[k < cnt ? k : 0] * H + ng);
    }
    // Every row is an operand here: the compiler would otherwise sink each load into the
    // condition on its use below and wait for it there, one row at a time.
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if constexpr (KM == 4)
        asm volatile("" ::"v"(b[g][0]), "v"(b[g][1]), "v"(b[g][2]), "v"(b[g][3]));
      else
        asm volatile("" ::"v"(b[g][0]), "v"(b[g][1]), "v"(b[g][2]), "v"(b[g][3]), "v"(b[g][4]),
                     "v"(b[g][5]), "v"(b[g][6]), "v"(b[g][7]));
    }
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int ng = n + 512 * g;
      if (ng >= H) break;
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        if (k >= cnt) break;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          acc[i] = __fadd_rn(acc[i], __fmul_rn(bf16_bits_to_f32(b[g][k][i]), ws[k]));
      }
      if (out_f32) {
        float* o = static_cast<float*>(out) + (size_t)t * H + ng;
        *reinterpret_cast<f32x4*>(o) = f32x4{acc[0], acc[1], acc[2], acc[3]};
        *reinterpret_cast<f32x4*>(o + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
      } else {
        u16x8 r;
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = f32_to_bf16_bits(acc[i]);
        *reinterpret_cast<u16x8*>(static_cast<uint16_t*>(out) + (size_t)t * H + ng) = r;
      }
    }
  }
}

// The affinity of slot p (token tk, expert e) as the reference's pre-scaling modes use it:
// a bf16 tensor (moe_cte.py:518-520, 556-558 multiply bf16 hidden rows / intermediates by
// it), so the fp32 value is rounded to bf16.
__device__ __forceinline__ float slot_affinity_bf16(const float* __restrict__ aff, int tk, int e,
                                                    int E) {
  return round_bf16(aff[(size_t)tk * E + e]);
}

// PRE_SCALE: xs[p] = bf16(x[token(p)] * a(p)) for every real slot p (moe_cte.py:518-520);
// padding slots are left as they are (the GEMM reads but never stores them).  One
// workgroup per slot, 8 columns per thread.
__global__ void __launch_bounds__(256) cte_prescale_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ aff,
    const int32_t* __restrict__ tp2id, const int32_t* __restrict__ b2e, int B, int T, int E,
    int H, uint16_t* __restrict__ xs) {
  const int64_t p = blockIdx.x;
  const int tk = tp2id[p];
  const int e = b2e[p / B];
  if (tk < 0 || tk >= T || e < 0 || e >= E) return;
  const float a = slot_affinity_bf16(aff, tk, e, E);
  for (int n = threadIdx.x * 8; n < H; n += 256 * 8) {
    const u16x8 v = *reinterpret_cast<const u16x8*>(x + (size_t)tk * H + n);
    u16x8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = f32_to_bf16_bits(bf16_bits_to_f32(v[i]) * a);
    *reinterpret_cast<u16x8*>(xs + (size_t)p * H + n) = r;
  }
}

// PRE_SCALE_DELAYED: h[p] = bf16(h[p] * a(p)) for every real slot (moe_cte.py:556-558).
__global__ void __launch_bounds__(256) cte_scale_h_kernel(
    uint16_t* __restrict__ h, const float* __restrict__ aff, const int32_t* __restrict__ tp2id,
    const int32_t* __restrict__ b2e, int B, int T, int E, int I) {
  const int64_t p = blockIdx.x;
  const int tk = tp2id[p];
  const int e = b2e[p / B];
  if (tk < 0 || tk >= T || e < 0 || e >= E) return;
  const float a = slot_affinity_bf16(aff, tk, e, E);
  for (int n = threadIdx.x * 8; n < I; n += 256 * 8) {
    u16x8 v = *reinterpret_cast<const u16x8*>(h + (size_t)p * I + n);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = f32_to_bf16_bits(bf16_bits_to_f32(v[i]) * a);
    *reinterpret_cast<u16x8*>(h + (size_t)p * I + n) = v;
  }
}

// Combine of the pre-scaling modes (moe_cte.py:576-579): out[t] = sum over ALL experts e
// in ascending order of y_e, with the bf16 running sum of the reference (a bf16 output
// tensor, each addition rounded).  A routed expert contributes its slot's y, any other
// expert its output for a zero input, expert_const[e] (the down bias under
// PRE_SCALE_DELAYED, y_e(0) under PRE_SCALE), or nothing when expert_const is null.
// Grid (T, column chunks of 2048); 8 columns per thread.
__global__ void __launch_bounds__(256) cte_combine_dense_bf16_kernel(
    const uint16_t* __restrict__ y, const int32_t* __restrict__ inv,
    const int32_t* __restrict__ tp2id, const int32_t* __restrict__ b2e, int64_t n_slots, int B,
    const uint16_t* __restrict__ expert_const, int H, int E, int out_f32, void* __restrict__ out) {
  const int t = blockIdx.x;
  const int n = blockIdx.y * 2048 + threadIdx.x * 8;
  if (n >= H) return;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int e = 0; e < E; ++e) {
    const int slot = cte_slot_of(inv, tp2id, b2e, n_slots, B, t, e, E);
    const uint16_t* src = slot >= 0 ? y + (size_t)slot * H
                                    : (expert_const ? expert_const + (size_t)e * H : nullptr);
    if (!src) continue;
    const u16x8 v = *reinterpret_cast<const u16x8*>(src + n);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = round_bf16(acc[i] + bf16_bits_to_f32(v[i]));
  }
  if (out_f32) {
    float* o = static_cast<float*>(out) + (size_t)t * H + n;
    *reinterpret_cast<f32x4*>(o) = f32x4{acc[0], acc[1], acc[2], acc[3]};
    *reinterpret_cast<f32x4*>(o + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
  } else {
    u16x8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = f32_to_bf16_bits(acc[i]);
    *reinterpret_cast<u16x8*>(static_cast<uint16_t*>(out) + (size_t)t * H + n) = r;
  }
}

struct CteWs {
  uint16_t* h;
  uint16_t* y;
  int32_t* inv;
  int2* order;
  uint16_t* xs;  // PRE_SCALE: the scaled activation row of every slot
};

static size_t cte_carve(void* base, size_t cap, int64_t T, int64_t H, int64_t I, int64_t E,
                        int64_t n_slots, int scale_mode, CteWs* w) {
  Carver cv(base, cap);
  CteWs c;
  c.h = cv.take<uint16_t>(n_slots * I);
  c.y = cv.take<uint16_t>(n_slots * H);
  c.inv = cv.take<int32_t>(T * E);
  c.order = cv.take<int2>(n_slots / kPM);
  c.xs = cv.take<uint16_t>(scale_mode == MXMOE_SCALE_PRE ? n_slots * H : 0);
  if (w) *w = c;
  return cv.off + 256;
}

// N-tiles of a projection with `rows` output rows, and its launch, per weight format.
static int prefill_ntiles(int64_t rows, int fmt) {
  const int rg = fmt == kWFmt8 ? PFmt<kWFmt8>::RG : PFmt<kWFmt4>::RG;
  return (int)((rows / 16 + rg - 1) / rg);
}

static void launch_prefill_gemm(bool gate_up, int fmt, const PrefillArgs& a, hipStream_t s) {
  const dim3 g(prefill_grid(a.n_mtiles, a.n_ntiles, a.group));
  if (fmt == kWFmt8) {
    if (gate_up)
      hipLaunchKernelGGL((prefill_gemm_kernel<true, kWFmt8>), g, dim3(kPThreads), 0, s, a);
    else
      hipLaunchKernelGGL((prefill_gemm_kernel<false, kWFmt8>), g, dim3(kPThreads), 0, s, a);
  } else {
    if (gate_up)
      hipLaunchKernelGGL((prefill_gemm_kernel<true, kWFmt4>), g, dim3(kPThreads), 0, s, a);
    else
      hipLaunchKernelGGL((prefill_gemm_kernel<false, kWFmt4>), g, dim3(kPThreads), 0, s, a);
  }
}

// Decode with bf16 expert weights: the routed top-k as dense affinities [T, E] (zero
// where not selected; expert ids outside [0, E) skipped), one workgroup per token.
__global__ void __launch_bounds__(256) tkg_bf16_scatter_kernel(const int32_t* __restrict__ idx,
                                                               const float* __restrict__ val,
                                                               int E, int K, float* __restrict__ aff) {
  const int t = blockIdx.x;
  for (int e = threadIdx.x; e < E; e += 256) aff[(size_t)t * E + e] = 0.0f;
  __syncthreads();
  if (threadIdx.x < K) {
    const int e = idx[(size_t)t * K + threadIdx.x];
    if (e >= 0 && e < E) aff[(size_t)t * E + e] = val[(size_t)t * K + threadIdx.x];
  }
}

constexpr int kTkgBf16Block = 128;  // one M-tile per block: decode batches are small
struct TkgBf16Ws {
  float *aff, *aff_m;
  int32_t *tp2id, *b2e, *cond, *inv;
  void* bw;
  size_t bw_bytes;
  int2* order;
  uint16_t *h_hi, *h_lo;
  float* y;
  int64_t n_blocks;
};

static size_t tkg_bf16_carve(void* base, size_t cap, int64_t T, int64_t H, int64_t I, int64_t E,
                             int K, TkgBf16Ws* w) {
  Carver cv(base, cap);
  TkgBf16Ws c;
  c.n_blocks = blockwise_n_blocks(T, E, K, kTkgBf16Block);
  const int64_t n_slots = c.n_blocks * kTkgBf16Block;
  c.aff = cv.take<float>(T * E);
  c.aff_m = cv.take<float>(T * E);
  c.tp2id = cv.take<int32_t>(n_slots);
  c.b2e = cv.take<int32_t>(c.n_blocks);
  c.cond = cv.take<int32_t>(c.n_blocks);
  c.inv = cv.take<int32_t>(T * E);
  c.bw_bytes = mxmoe_blockwise_workspace_bytes(T, E);
  c.bw = cv.take<char>(c.bw_bytes);
  c.order = cv.take<int2>(n_slots / kPM);
  c.h_hi = cv.take<uint16_t>(n_slots * I);
  c.h_lo = cv.take<uint16_t>(n_slots * I);
  c.y = cv.take<float>(n_slots * H);
  if (w) *w = c;
  return cv.off + 256;
}

}  // namespace mxmoe

using namespace mxmoe;

// Batches whose experts hold few 16-token tiles (the MXFP4 decode's one-tile rule) stream
// the weights item by item (tkg_bf16_stream); larger ones run the blockwise GEMMs.
static bool tkg_bf16_streams(int64_t T, int64_t E, int top_k) {
  return (T <= 16 || T * top_k <= 8 * E) && T <= 1024 && E <= 512 && top_k <= 8;
}

extern "C" size_t mxmoe_moe_tkg_bf16_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                                                     int top_k) {
  if (T < 1 || E < 1 || top_k < 1) return 256;
  if (tkg_bf16_streams(T, E, top_k)) return tkg_bf16_stream_workspace(T, H, I, E, top_k);
  return tkg_bf16_carve(nullptr, ~(size_t)0, T, H, I, E, top_k, nullptr);
}

extern "C" int mxmoe_moe_tkg_bf16(const uint16_t* x, const int32_t* topk_idx,
                                  const float* topk_val, const uint16_t* gu_w,
                                  const uint16_t* dn_w, const uint16_t* gu_bias,
                                  const uint16_t* dn_bias, int64_t T, int64_t H, int64_t I,
                                  int64_t E, int top_k, int act, const float* clamps,
                                  int scale_mode, uint16_t* out, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  clear_error();
  MXMOE_REQUIRE(x && topk_idx && topk_val && gu_w && dn_w && out && workspace,
                "moe_tkg_bf16: null pointer");
  MXMOE_REQUIRE(T >= 1 && E >= 1 && E <= kCteMaxE && top_k >= 1 && top_k <= 256,
                "moe_tkg_bf16: bad T/E/top_k (E at most %d, top_k at most 256)", kCteMaxE);
  MXMOE_REQUIRE(H % 32 == 0 && I % 32 == 0 && H >= 32 && I >= 32,
                "moe_tkg_bf16: H=%lld and I=%lld must be multiples of 32", (long long)H,
                (long long)I);
  MXMOE_REQUIRE(act >= 0 && act <= 2, "moe_tkg_bf16: unknown activation %d", act);
  MXMOE_REQUIRE(scale_mode == MXMOE_SCALE_POST || scale_mode == MXMOE_SCALE_NO,
                "moe_tkg_bf16: unsupported scale mode %d", scale_mode);
  MXMOE_REQUIRE((uintptr_t)gu_w % 16 == 0 && (uintptr_t)dn_w % 16 == 0,
                "moe_tkg_bf16: bf16 weights must be 16-byte aligned");
  // both decode flows address one expert's weights through a buffer resource (32-bit size
  // and offsets): its gate_up, H x 2I bf16, stays under 4 GiB
  MXMOE_REQUIRE((double)H * (double)I * 4.0 < 4294967296.0,
                "moe_tkg_bf16: a bf16 expert's gate_up (H=%lld x 2I=%lld) exceeds 4 GiB",
                (long long)H, (long long)(2 * I));
  if (tkg_bf16_streams(T, E, top_k))
    return tkg_bf16_stream(x, topk_idx, topk_val, gu_w, dn_w, gu_bias, dn_bias, T, H, I, E, top_k,
                           act, clamps, scale_mode, out, workspace, workspace_bytes,
                           as_stream(stream));
  const int64_t n_slots = blockwise_n_blocks(T, E, top_k, kTkgBf16Block) * kTkgBf16Block;
  const int64_t kmax = H > I ? H : I;
  MXMOE_REQUIRE(n_slots / kPM <= kOrderMaxTiles && n_slots * kmax * 2 < ((int64_t)1 << 32) &&
                    T * H * 2 < ((int64_t)1 << 32),
                "moe_tkg_bf16: %lld tokens x %d experts exceed one call", (long long)T, top_k);
  const size_t need = tkg_bf16_carve(nullptr, ~(size_t)0, T, H, I, E, top_k, nullptr);
  if (workspace_bytes < need)
    return set_error(MXMOE_E_WORKSPACE, "moe_tkg_bf16: workspace %zu < %zu", workspace_bytes,
                     need);
  TkgBf16Ws w;
  tkg_bf16_carve(workspace, workspace_bytes, T, H, I, E, top_k, &w);
  hipStream_t s = as_stream(stream);

  hipLaunchKernelGGL(tkg_bf16_scatter_kernel, dim3((unsigned)T), dim3(256), 0, s, topk_idx,
                     topk_val, (int)E, top_k, w.aff);
  int rc = mxmoe_blockwise_mapping(w.aff, nullptr, T, E, top_k, kTkgBf16Block, w.n_blocks,
                                   w.aff_m, w.tp2id, w.b2e, w.cond, nullptr, w.bw, w.bw_bytes,
                                   stream);
  if (rc != MXMOE_OK) return rc;

  PrefillArgs a = {};
  a.tp2id = w.tp2id;
  a.T = (int)T;
  a.I = (int)I;
  a.H = (int)H;
  a.B = kTkgBf16Block;
  a.n_mtiles = (int)(n_slots / kPM);
  a.group = prefill_group_tiles(kTkgBf16Block);
  a.order = w.order;
  a.E = (int)E;
  a.a_by_slot = 0;
  a.inv = w.inv;
  a.p.gate_lo = clamps ? clamps[0] : -INFINITY;
  a.p.gate_hi = clamps ? clamps[1] : INFINITY;
  a.p.up_lo = clamps ? clamps[2] : -INFINITY;
  a.p.up_hi = clamps ? clamps[3] : INFINITY;
  a.p.act = act;
  hipLaunchKernelGGL(cte_tile_order_kernel, dim3(1), dim3(kOrderThreads),
                     (size_t)a.n_mtiles * 5, s, w.tp2id, w.b2e, kTkgBf16Block, a.n_mtiles,
                     a.group, (int)T, w.order);
  // gate_up: A = x (K = H), rows = 2I; h as (hi, lo)
  a.a = x;
  a.wq = reinterpret_cast<const uint8_t*>(gu_w);
  a.bias = gu_bias;
  a.out = w.h_hi;
  a.K = (int)H;
  a.N_rows = (int)(2 * I);
  a.n_ntiles = prefill_ntiles_bf16(true, I, H);
  launch_decode_gemm_bf16(true, a, nullptr, w.h_lo, nullptr, s);
  // down: A = h (K = I) in two passes, rows = H; y fp32
  a.a = w.h_hi;
  a.inv = nullptr;
  a.wq = reinterpret_cast<const uint8_t*>(dn_w);
  a.bias = dn_bias;
  a.out = nullptr;
  a.K = (int)I;
  a.N_rows = (int)H;
  a.n_ntiles = prefill_ntiles_bf16(false, I, H);
  launch_decode_gemm_bf16(false, a, w.h_lo, nullptr, w.y, s);
  hipLaunchKernelGGL(cte_combine_kernel<float>,
                     dim3((unsigned)((T + kCombineTok - 1) / kCombineTok)),
                     dim3(kCombineThreads), 0, s, w.y, w.inv, w.tp2id, w.b2e, n_slots,
                     kTkgBf16Block, w.aff, (int)T, (int)H, (int)E, scale_mode, 0, out);
  return check_launch("moe_tkg_bf16");
}

extern "C" size_t mxmoe_moe_cte_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                                                int64_t block_size, int64_t n_blocks,
                                                int scale_mode) {
  return cte_carve(nullptr, ~(size_t)0, T, H, I, E, block_size * n_blocks, scale_mode, nullptr);
}

namespace mxmoe {

int cte_run(const uint16_t* x, const float* affinities_masked, const uint8_t* gu_q,
            const uint8_t* gu_s, const uint8_t* dn_q, const uint8_t* dn_s, int weight_fmt,
            const uint16_t* gu_bias, const uint16_t* dn_bias, const uint16_t* expert_const,
            const int32_t* token_position_to_id, const int32_t* block_to_expert,
            int64_t n_blocks, int64_t block_size, int64_t T, int64_t H, int64_t I, int64_t E,
            int act, const float* clamps, int scale_mode, int out_f32, void* out,
            void* workspace, size_t workspace_bytes, void* const* stage_events,
            const int2* order_pre, hipStream_t s, const CteTokPairs* pairs) {
  const bool bf16w = weight_fmt == MXMOE_WFMT_BF16;
  // the affinities are read by the pre-scaling modes and the inverse-table combine only
  const bool need_aff = !(pairs && pairs->K <= 8 && scale_mode == MXMOE_SCALE_POST);
  MXMOE_REQUIRE(x && (affinities_masked || !need_aff) && gu_q && dn_q &&
                    (bf16w || (gu_s && dn_s)) && token_position_to_id && block_to_expert &&
                    out && workspace,
                "moe_cte: null pointer");
  MXMOE_REQUIRE(T >= 1 && E >= 1 && E <= kCteMaxE && n_blocks >= 1,
                "moe_cte: bad T/E/n_blocks (E at most %d)", kCteMaxE);
  MXMOE_REQUIRE(block_size >= 128 && block_size % 128 == 0,
                "moe_cte: block_size=%lld must be a multiple of 128", (long long)block_size);
  MXMOE_REQUIRE(H % 32 == 0 && I % 32 == 0 && H >= 32 && I >= 32,
                "moe_cte: H=%lld and I=%lld must be multiples of 32", (long long)H, (long long)I);
  MXMOE_REQUIRE(act >= 0 && act <= 2, "moe_cte: unknown activation %d", act);
  MXMOE_REQUIRE(weight_fmt == MXMOE_WFMT_MXFP4 || weight_fmt == MXMOE_WFMT_MXFP8 || bf16w,
                "moe_cte: unknown weight format %d", weight_fmt);
  // bf16 weight rows are read 16 bytes at a time, through buffer resources of one expert
  // (32-bit sizes and offsets)
  MXMOE_REQUIRE(!bf16w || ((uintptr_t)gu_q % 16 == 0 && (uintptr_t)dn_q % 16 == 0),
                "moe_cte: bf16 weights must be 16-byte aligned");
  MXMOE_REQUIRE(!bf16w || (double)H * (double)I * 4.0 < 4294967296.0,
                "moe_cte: a bf16 expert's gate_up (H=%lld x 2I=%lld) exceeds 4 GiB",
                (long long)H, (long long)(2 * I));
  MXMOE_REQUIRE(scale_mode == MXMOE_SCALE_POST || scale_mode == MXMOE_SCALE_NO ||
                    scale_mode == MXMOE_SCALE_PRE || scale_mode == MXMOE_SCALE_PRE_DELAYED,
                "moe_cte: unsupported scale mode %d", scale_mode);
  const int64_t n_slots = n_blocks * block_size;
  MXMOE_REQUIRE(n_slots / kPM <= kOrderMaxTiles,
                "moe_cte: %lld slots exceed the %d M-tiles of 128 slots one call schedules",
                (long long)n_slots, kOrderMaxTiles);
  // The GEMMs address activation rows with 32-bit byte offsets from one base.
  const int64_t kmax = H > I ? H : I;
  MXMOE_REQUIRE(n_slots * kmax * 2 < ((int64_t)1 << 32) && T * H * 2 < ((int64_t)1 << 32),
                "moe_cte: %lld slots x %lld columns (or %lld tokens) exceed the 4 GiB of "
                "activation rows one call addresses",
                (long long)n_slots, (long long)kmax, (long long)T);
  const size_t need = cte_carve(nullptr, ~(size_t)0, T, H, I, E, n_slots, scale_mode, nullptr);
  if (workspace_bytes < need)
    return set_error(MXMOE_E_WORKSPACE, "moe_cte: workspace %zu < %zu", workspace_bytes, need);
  CteWs w;
  cte_carve(workspace, workspace_bytes, T, H, I, E, n_slots, scale_mode, &w);
  const bool pre = scale_mode == MXMOE_SCALE_PRE, delayed = scale_mode == MXMOE_SCALE_PRE_DELAYED;
  auto mark = [&](int i) {
    mark_event(stage_events, i, s);
  };

  PrefillArgs a;
  a.tp2id = token_position_to_id;
  a.T = (int)T;
  a.I = (int)I;
  a.H = (int)H;
  a.B = (int)block_size;
  a.n_mtiles = (int)(n_slots / kPM);
  a.group = prefill_group_tiles(block_size);
  a.order = order_pre ? order_pre : w.order;
  a.E = (int)E;
  a.a_by_slot = pre ? 1 : 0;
  const bool tok_pairs = pairs && pairs->K <= 8 && !pre && !delayed;
  a.inv = tok_pairs ? nullptr : w.inv;
  a.p.gate_lo = clamps ? clamps[0] : -INFINITY;
  a.p.gate_hi = clamps ? clamps[1] : INFINITY;
  a.p.up_lo = clamps ? clamps[2] : -INFINITY;
  a.p.up_hi = clamps ? clamps[3] : INFINITY;
  a.p.act = act;

  // gate_up: A = x (K = H), rows = 2I; under PRE_SCALE the scaled row of every slot
  if (pre)
    hipLaunchKernelGGL(cte_prescale_kernel, dim3((unsigned)n_slots), dim3(256), 0, s, x,
                       affinities_masked, token_position_to_id, block_to_expert,
                       (int)block_size, (int)T, (int)E, (int)H, w.xs);
  a.a = pre ? w.xs : x;
  a.wq = gu_q;
  a.ws = gu_s;
  a.bias = gu_bias;
  a.out = w.h;
  a.K = (int)H;
  a.N_rows = (int)(2 * I);
  a.n_ntiles = bf16w ? prefill_ntiles_bf16(true, I, H) : prefill_ntiles(2 * I, weight_fmt);
  if (!order_pre)
    hipLaunchKernelGGL(cte_tile_order_kernel, dim3(1), dim3(kOrderThreads),
                       (size_t)a.n_mtiles * 5, s, token_position_to_id, block_to_expert,
                       (int)block_size, a.n_mtiles, a.group, (int)T, w.order);
  mark(0);
  if (bf16w)
    launch_prefill_gemm_bf16(true, a, s);
  else
    launch_prefill_gemm(true, weight_fmt, a, s);
  mark(1);
  if (delayed)
    hipLaunchKernelGGL(cte_scale_h_kernel, dim3((unsigned)n_slots), dim3(256), 0, s, w.h,
                       affinities_masked, token_position_to_id, block_to_expert,
                       (int)block_size, (int)T, (int)E, (int)I);
  // down: A = h (K = I), rows = H
  a.a = w.h;
  a.a_by_slot = 0;
  a.inv = nullptr;
  a.wq = dn_q;
  a.ws = dn_s;
  a.bias = dn_bias;
  a.out = w.y;
  a.K = (int)I;
  a.N_rows = (int)H;
  a.n_ntiles = bf16w ? prefill_ntiles_bf16(false, I, H) : prefill_ntiles(H, weight_fmt);
  if (bf16w)
    launch_prefill_gemm_bf16(false, a, s);
  else
    launch_prefill_gemm(false, weight_fmt, a, s);
  mark(2);
  if (pre || delayed)
    hipLaunchKernelGGL(cte_combine_dense_bf16_kernel,
                       dim3((unsigned)T, (unsigned)((H + 2047) / 2048)), dim3(256), 0, s, w.y,
                       w.inv, token_position_to_id, block_to_expert, n_slots, (int)block_size,
                       expert_const, (int)H, (int)E, out_f32, out);
  else if (tok_pairs && pairs->K <= 4)
    hipLaunchKernelGGL((cte_combine_tok_kernel<4, 6>),
                       dim3((unsigned)((T + kCombineTok - 1) / kCombineTok)),
                       dim3(kCombineThreads), 0, s, w.y, pairs->slot, pairs->sel, pairs->val,
                       (int)T, (int)H, pairs->K, scale_mode, out_f32, out);
  else if (tok_pairs)
    hipLaunchKernelGGL((cte_combine_tok_kernel<8, 2>),
                       dim3((unsigned)((T + kCombineTok - 1) / kCombineTok)),
                       dim3(kCombineThreads), 0, s, w.y, pairs->slot, pairs->sel, pairs->val,
                       (int)T, (int)H, pairs->K, scale_mode, out_f32, out);
  else
    hipLaunchKernelGGL(cte_combine_kernel<uint16_t>,
                       dim3((unsigned)((T + kCombineTok - 1) / kCombineTok)),
                       dim3(kCombineThreads), 0, s, w.y, w.inv, token_position_to_id,
                       block_to_expert, n_slots, (int)block_size, affinities_masked, (int)T,
                       (int)H, (int)E, scale_mode, out_f32, out);
  mark(3);
  return check_launch("moe_cte");
}

}  // namespace mxmoe

extern "C" int mxmoe_moe_cte(const uint16_t* x, const float* affinities_masked,
                             const uint8_t* gu_q, const uint8_t* gu_s, const uint8_t* dn_q,
                             const uint8_t* dn_s, int weight_fmt, const uint16_t* gu_bias,
                             const uint16_t* dn_bias, const uint16_t* expert_const,
                             const int32_t* token_position_to_id,
                             const int32_t* block_to_expert, int64_t n_blocks, int64_t block_size,
                             int64_t T, int64_t H, int64_t I, int64_t E, int act,
                             const float* clamps, int scale_mode, int out_f32, void* out,
                             void* workspace, size_t workspace_bytes, void* const* stage_events,
                             void* stream) {
  clear_error();
  return cte_run(x, affinities_masked, gu_q, gu_s, dn_q, dn_s, weight_fmt, gu_bias, dn_bias,
                 expert_const, token_position_to_id, block_to_expert, n_blocks, block_size, T, H,
                 I, E, act, clamps, scale_mode, out_f32, out, workspace, workspace_bytes,
                 stage_events, nullptr, as_stream(stream));
}

// The linear for few rows of x (M <= kLinSmallM, MXFP4).  The tiled GEMM above gives such
// an x one M-tile, so W's N / 256 N-tiles are its only workgroups (23 for N = 5,760, about
// 40 us each, MFMA-issue bound on one wave per SIMD).  Here a workgroup is 12 waves, one
// row group (16 rows of W) each, against one 16-row tile of x: ceil(N / 192) x ceil(M / 16)
// workgroups (240 for 128 x 5,760, one per CU), the x tiles of one block of W rows on one
// XCD (the dispatcher deals workgroup i to XCD i % 8), so that its L2 serves those W rows
// to all of them.  K goes in slabs of up to kLinSlab chunks, each one round trip: every
// wave issues its row group's weight and scale loads for the whole slab (registers) and
// its share of the x tile's slab as direct global -> LDS loads (no registers; 16-byte
// blocks XOR-swizzled by row), waits for all of them, and after the barrier runs the
// slab's MFMAs.  Per accumulator the arithmetic is the tiled GEMM's: the same lane -> K
// mapping, chunks in order, steps j = 0..3 in order, lanes past K with scale 0, the same
// bf16 conversion; so the output is the same, bit for bit.
namespace mxmoe {

constexpr int kLinWaves = 12;
constexpr int kLinSlab = 24;  // chunks per K slab: 96 + 24 registers of weights and scales
constexpr int kLinSmallM = 256;
constexpr int kLinDma = 4 * kLinSlab / kLinWaves;  // 1 KiB direct loads per wave and slab
static_assert(kLinDma * kLinWaves == 4 * kLinSlab, "a slab's x tile: 4 KiB per chunk");

__global__ void __launch_bounds__(64 * kLinWaves) linear_small_kernel(
    const uint16_t* __restrict__ x, int M, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, int N, int K, int n_tiles, uint16_t* __restrict__ y) {
  // LDS: chunk c of the slab at c * 4 KiB, row r (of 16) at r * 256 B in it, 16-byte slot s
  // of the row holding the row's column block s ^ r
  extern __shared__ __attribute__((aligned(16))) uint8_t lin_lds[];
  const int lane = threadIdx.x & 63, q = lane >> 4, r16 = lane & 15;
  const int wave = wave_id();
  const int n_rg = N / 16;
  // workgroup i: XCD i % 8 takes the row blocks i % 8, i % 8 + 8, ..., each with its
  // n_tiles x tiles in a row; ids past the last row block exit at once (the whole workgroup)
  const int xcd = (int)blockIdx.x % 8, k = (int)blockIdx.x / 8;
  const int rb = xcd + 8 * (k / n_tiles);
  if (rb * kLinWaves >= n_rg) return;
  const int rg_raw = rb * kLinWaves + wave;
  const bool rg_ok = rg_raw < n_rg;
  const int rg = rg_ok ? rg_raw : n_rg - 1;  // waves past N load a real row group, store nothing
  const int m0 = (k % n_tiles) * 16;
  const int nc = (K + 127) / 128, nfull = K / 128, tail_q = (K % 128) / 32;
  const uint8_t* wbase = wq + (size_t)rg * ((size_t)K * 8);
  const uint8_t* sbase = ws + (size_t)(rg / 4) * ((size_t)K * 2);
  const int sshift = 8 * (rg % 4);
  // this lane's x row in direct load i of a chunk (rows 4i .. 4i + 3, 16 lanes each) and
  // its source column block (slot lane % 16 of row r holds block (lane % 16) ^ r)
  const int drow = lane >> 4;  // + 4 * (load index % 4)
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < nc; c0 += kLinSlab) {
    const int ns = min(kLinSlab, nc - c0);
    if (c0 > 0) __syncthreads();  // the last slab's LDS is read before it is refilled
    // The x tile's slab: wave w issues loads d = w, w + 12, ... < 4 ns, load d = (chunk
    // d / 4, rows 4 (d % 4) ..), 1 KiB to LDS offset d * 1 KiB; loads u < kLinDma / 2 hold
    // chunks 0 .. 11 of the slab, the others chunks 12 .. 23.
    auto xdma = [&](int u) {
      const int d = wave + kLinWaves * u;
      if (d < 4 * ns) {
        const int row = 4 * (d & 3) + drow;
        const int col = (c0 + (d >> 2)) * 128 + 8 * (r16 ^ row);
        const int m = min(m0 + row, M - 1);
        const uint32_t off = 2u * ((uint32_t)m * (uint32_t)K + (uint32_t)(col < K ? col : 0));
        const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(
            const __attribute__((address_space(3))) uint8_t*)(lin_lds + d * 1024));
        asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(off),
                     "s"(x)
                     : "memory", "m0");
      }
    };
    // The slab's weights and scales (chunks past the slab re-read its last one; lanes past
    // K read lane 0's bytes, which the zero scale cancels).
    u32x4 wv[kLinSlab];
    uint32_t sv[kLinSlab];
    auto wload = [&](int i) {
      const int c = c0 + min(i, ns - 1);
      const uint32_t lo = (c < nfull || q < tail_q) ? (uint32_t)lane : 0u;
      wv[i] = *reinterpret_cast<const u32x4*>(wbase + (size_t)c * 1024 + lo * 16u);
      sv[i] = *reinterpret_cast<const uint32_t*>(sbase + (size_t)c * 256 + lo * 4u);
    };
    // Issue order: the first half's x and weights, the second half's x, then its weights
    // (2 x 12 loads, always issued); waiting until at most those 24 are outstanding leaves
    // every x block landed (the direct loads are not counted by the compiler), and the
    // first half's MFMAs run while the second half's weights arrive (the compiler waits
    // for each weight register it counts before its first use).
#pragma unroll
    for (int u = 0; u < kLinDma / 2; ++u) xdma(u);
#pragma unroll
    for (int i = 0; i < kLinSlab / 2; ++i) wload(i);
#pragma unroll
    for (int u = kLinDma / 2; u < kLinDma; ++u) xdma(u);
#pragma unroll
    for (int i = kLinSlab / 2; i < kLinSlab; ++i) wload(i);
    static_assert(kLinSlab == 24 && kLinDma == 8, "the wait below counts 2 x 12 loads");
    asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
    __syncthreads();
    const uint8_t* xr = lin_lds + r16 * 256;
#pragma unroll
    for (int i = 0; i < kLinSlab; ++i) {
      if (i < ns) {
        const int c = c0 + i;
        const bool kok = c < nfull || q < tail_q;
        const float sc = kok ? e8m0_to_f32((sv[i] >> sshift) & 0xffu) : 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const u32x4 xf =
              *reinterpret_cast<const u32x4*>(xr + i * 4096 + (((4 * q + j) ^ r16) << 4));
          acc = mfma16(dequant8(wv[i][j], sc), as_bf16x8(xf), acc);
        }
      }
    }
  }
  // Lane (q, r16): W rows 16 rg + 4q .. + 3 of x row m0 + r16.
  const int m = m0 + r16;
  if (rg_ok && m < M)
    *reinterpret_cast<u32x2*>(y + (size_t)m * N + 16 * rg + 4 * q) =
        u32x2{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
}

}  // namespace mxmoe

extern "C" int mxmoe_linear(const uint16_t* x, int64_t M, const uint8_t* wq, const uint8_t* ws,
                            int weight_fmt, int64_t N, int64_t K, uint16_t* y, void* stream) {
  clear_error();
  MXMOE_REQUIRE(x && wq && ws && y, "linear: null pointer");
  MXMOE_REQUIRE(weight_fmt == MXMOE_WFMT_MXFP4 || weight_fmt == MXMOE_WFMT_MXFP8,
                "linear: unknown weight format %d", weight_fmt);
  MXMOE_REQUIRE(M >= 0 && N >= 16 && N % 16 == 0 && K >= 32 && K % 32 == 0,
                "linear: N=%lld must be a multiple of 16 and K=%lld of 32", (long long)N,
                (long long)K);
  if (M == 0) return MXMOE_OK;
  if (weight_fmt == MXMOE_WFMT_MXFP4 && M <= kLinSmallM) {
    MXMOE_REQUIRE(M * K * 2 < ((int64_t)1 << 32), "linear: x of %lld x %lld too large",
                  (long long)M, (long long)K);
    const int nc = (int)((K + 127) / 128);
    const size_t lds = (size_t)std::min(kLinSlab, nc) * 4096;
    const int n_rb = (int)((N / 16 + kLinWaves - 1) / kLinWaves);
    const int n_tiles = (int)((M + 15) / 16);
    hipLaunchKernelGGL(linear_small_kernel, dim3((unsigned)(8 * ((n_rb + 7) / 8) * n_tiles)),
                       dim3(64 * kLinWaves), lds, as_stream(stream), x, (int)M, wq, ws, (int)N,
                       (int)K, n_tiles, y);
    return check_launch("linear");
  }
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
  a.E = 1;
  a.a_by_slot = 0;
  a.n_mtiles = (int)((M + kPM - 1) / kPM);
  a.n_ntiles = prefill_ntiles(N, weight_fmt);
  a.group = 1;
  a.p.gate_lo = -INFINITY;
  a.p.gate_hi = INFINITY;
  a.p.up_lo = -INFINITY;
  a.p.up_hi = INFINITY;
  launch_prefill_gemm(false, weight_fmt, a, as_stream(stream));
  return check_launch("linear");
}
