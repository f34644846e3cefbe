// Expert GEMMs of bf16 expert weights (prefill and decode): the reference's shard_on_block operands
// (vllm_neuron/functional/moe/moe_cte.py:117-124, model_bf16.py:1360-1391), gate_up
// [E, H, 2, I] and down [E, I, H], each expert's rows running along K.  Same blockwise
// schedule (tile order, XCD groups), slot tables and epilogues as the MX GEMMs, which
// stream packed codes instead.
//
// Workgroup tile: 128 slots x 128 output columns over K in 64-wide chunks, 4 waves in a
// 2 x 2 grid (wave w: slots 64 (w & 1) .. +63, columns 64 (w >> 1) .. +63), each wave
// 4 x 4 MFMA 16x16x32 tiles.  The weights are the MFMA's A operand (rows = output
// columns) and the slots' activations its B operand, so a lane ends with 4 consecutive
// output columns of one slot (one 8-byte store).  Both operands pass through LDS, in two
// stages of one chunk each (32 KiB: 64 KiB per workgroup, two workgroups per CU):
//   activations: 128 rows x 128 B, 16-byte blocks XOR-swizzled by row pair;
//   weights: row-major as in memory (64 rows x 256 B), 32-byte column groups XOR-swizzled
//     by row; a lane's 8 K-values of one column come from two transposing LDS reads
//     (ds_read_b64_tr_b16).
// Global -> register loads are bounds-checked buffer loads issued in a fixed order, two
// chunks ahead of the MFMAs; one barrier per chunk orders the stages.
// gate_up N-tile: 64 intermediate columns as 4 pairs of 16-column tiles (gate, up) so
// that a lane holds gate and up of the same columns; down N-tile: 128 columns of H.
// Two flows share the GEMMs (template F32):
//   prefill (moe_cte, moe_cte.py:448-581): the bf16 result of every op, h bf16, y bf16;
//   decode (moe_block_tkg.py:223-297): fp32 throughout; gate_up writes h as an exact-to-
//   16-bits pair hi + lo of bf16 arrays, the down GEMM runs K twice (hi rows, then lo
//   rows against the same weight rows: bf16 products are exact in fp32) and writes y fp32.

#include <math.h>

#include "capi_util.h"
#include "common.h"
#include "prefill_common.h"

namespace mxmoe {

constexpr int kBN = 128;               // output columns per N-tile
constexpr int kBK = 64;                // K per chunk
constexpr int kBThreads = 256;
constexpr int kBGateUpCols = kBN / 2;  // intermediate columns of a gate_up N-tile
constexpr int kBArow = kBK * 2;        // bytes of an activation row's chunk (8 blocks of 16 B)
constexpr int kBWrow = kBN * 2;        // bytes of a weight row's chunk (128 columns)
constexpr int kBAbytes = kPM * kBArow;                 // 16 KiB
constexpr int kBStage = kBAbytes + kBK * kBWrow;       // + 16 KiB of weights
static_assert(kPM * (kBArow / 16) == 4 * kBThreads, "4 activation blocks per thread and chunk");
static_assert(kBK * (kBWrow / 16) == 4 * kBThreads, "4 weight blocks per thread and chunk");

// The decode flow's extra operands (null in the prefill flow).
struct Bf16Args {
  PrefillArgs p;
  const uint16_t* a_lo;  // down: lo part of h [slots, I]
  uint16_t* out_lo;      // gate_up: lo part of h [slots, I]
  float* y32;            // down: y [slots, H] fp32
};

// Activation stage: row r (slot), 16-byte block b of its 64 K-values, XOR-swizzled so
// that the 16 rows an operand read touches (two per 256-byte bank window) hit distinct banks.
__device__ __forceinline__ uint32_t a_off(int r, int b) {
  return (uint32_t)r * kBArow + (uint32_t)((b ^ ((r >> 1) & 7)) << 4);
}
// Weight stage: row k (K), column n of the N-tile, row-major as in memory; the 32-byte
// groups of 16 columns are XOR-swizzled by k so that the 16 rows one transposing read
// touches (k = 8 g + j and + 4, g, j = 0..3) spread over 8 distinct groups.
__device__ __forceinline__ uint32_t w_swz(int k) { return (uint32_t)((k & 3) | (((k >> 3) & 1) << 2)); }
__device__ __forceinline__ uint32_t w_off(int k, int n) {
  return (uint32_t)kBAbytes + (uint32_t)k * kBWrow +
         ((((uint32_t)(n >> 4)) ^ w_swz(k)) << 5) + (uint32_t)((n & 15) << 1);
}

// One chunk's global -> register loads of a thread: 4 activation blocks (rows tid / 8 +
// 32 i, block tid % 8) and 4 weight blocks (rows tid / 16 + 16 j, columns 8 (tid % 16) ..),
// as bounds-checked buffer loads: a block whose data is not wanted (past K, columns past
// the projection, slots after the tile's last real one) gets an offset past the resource's
// range, which returns zeros without a memory access.  Every load is issued, in a fixed
// order: loads under a lane condition would make the compiler wait for all outstanding
// loads where the paths meet.
struct BChunk {
  u32x4 a[4];
  u32x4 w[4];
};
constexpr uint32_t kBOff = 0xFFFFFFF0u;  // past every resource's range (each is < 4 GiB, in 64-byte rows)
// Raw buffer resource over [p, p + bytes): stride 0, the gfx9-family data format word.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t bf16_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ void bf16_load(BChunk& r, __amdgpu_buffer_rsrc_t ra,
                                          const uint32_t (&aoff)[4], __amdgpu_buffer_rsrc_t rw,
                                          uint32_t wcol, bool wcol_ok, uint32_t ldw, int K, int kc,
                                          int last) {
  const int tid = threadIdx.x;
  const int ab = tid & 7, ar = tid >> 3, kr = tid >> 4;
  const bool a_ok = kc + 8 * ab < K;  // K % 32 == 0: a block is whole or past K
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool ok = a_ok && ar + 32 * i <= last;
    const uint32_t o = ok ? aoff[i] + (uint32_t)(kc + 8 * ab) * 2u : kBOff;
    r.a[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, (int)o, 0, 0));
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int k = kc + kr + 16 * j;
    const uint32_t o = (wcol_ok && k < K) ? ((uint32_t)k * ldw + wcol) * 2u : kBOff;
    r.w[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)o, 0, 0));
  }
}

__device__ __forceinline__ void bf16_store_lds(const BChunk& r, uint8_t* st) {
  const int tid = threadIdx.x;
  const int ab = tid & 7, ar = tid >> 3, nb = tid & 15, kr = tid >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(st + a_off(ar + 32 * i, ab)) = r.a[i];
#pragma unroll
  for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4*>(st + w_off(kr + 16 * j, 8 * nb)) = r.w[j];
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
// 4 K-values (rows k, k + 1, k + 2, k + 3 of column n + lane % 16) of the weight stage by
// gfx950's transposing LDS read: in each 16-lane group, lane 4 j + q reads row k + j,
// columns n + 4 q .. + 3, and lane i receives column n + i of the 4 rows.
__device__ __forceinline__ s16x4 w_tr(const uint8_t* st, int k, int n) {
  const int li = threadIdx.x & 15;
  const uint8_t* p = st + w_off(k + (li >> 2), n + 4 * (li & 3));
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)((__attribute__((address_space(3))) uint8_t*)p));
}

// One chunk's MFMAs of a wave: 2 K-steps of 32, each 4 weight operands (two transposing
// reads each) and 4 activation operands (one 16-byte read each; lane l: row l % 16 of the
// subtile, K-values 8 (l / 16) .. + 7 of the step).
__device__ __forceinline__ void bf16_compute(const uint8_t* st, int fh, int sh,
                                             f32x4 (&acc)[4][4]) {
  const int lane = threadIdx.x & 63, li = lane & 15, lq = lane >> 4;
#pragma unroll
  for (int ks = 0; ks < kBK / 32; ++ks) {
    bf16x8 wa[4], xb[4];
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const int k = 32 * ks + 8 * lq, n = 64 * fh + 16 * f;
      const s16x4 lo = w_tr(st, k, n), hi = w_tr(st, k + 4, n);
      const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      wa[f] = __builtin_bit_cast(bf16x8, v);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
      xb[s] = as_bf16x8(*reinterpret_cast<const u32x4*>(st + a_off(64 * sh + 16 * s + li,
                                                                   4 * ks + lq)));
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int s = 0; s < 4; ++s) acc[f][s] = mfma16(wa[f], xb[s], acc[f][s]);
  }
}

// gate_up epilogue of a wave: pairs (f = 0, 1) and (2, 3) are the gate and up tiles of
// intermediate columns c0 + 16 p ..; bias, clamps and activation with the reference's
// bf16 roundings (as the MX gate_up epilogue), h = up * act(gate) as bf16.
template <int ACT>
__device__ __forceinline__ void bf16_gate_up_store(const PrefillArgs& args, const f32x4 (&acc)[4][4],
                                                   const int32_t* stok, int m0, int e, int c0,
                                                   int sh) {
  const int lane = threadIdx.x & 63, li = lane & 15, lq = lane >> 4;
  const int I = args.I;
#pragma unroll
  for (int pp = 0; pp < 2; ++pp) {
    const int col0 = c0 + 16 * pp + 4 * lq;
    if (col0 >= I) continue;
    float gb[4] = {0.f, 0.f, 0.f, 0.f}, ub[4] = {0.f, 0.f, 0.f, 0.f};
    if (args.bias) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        gb[i] = bf16_bits_to_f32(args.bias[(size_t)e * 2 * I + col0 + i]);
        ub[i] = bf16_bits_to_f32(args.bias[(size_t)e * 2 * I + I + col0 + i]);
      }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int row = 64 * sh + 16 * s + li;
      if (stok[row] < 0) continue;
      const f32x4 g4 = acc[2 * pp][s], u4 = acc[2 * pp + 1][s];
      float h[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float g = rb(g4[i]), u = rb(u4[i]);
        if (args.bias) {
          g = rb(g + gb[i]);
          u = rb(u + ub[i]);
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

// down epilogue of a wave: columns n0 + 16 f + 4 (l / 16) .., bias with bf16 roundings.
__device__ __forceinline__ void bf16_down_store(const PrefillArgs& args, const f32x4 (&acc)[4][4],
                                                const int32_t* stok, int m0, int e, int n0,
                                                int sh) {
  const int lane = threadIdx.x & 63, li = lane & 15, lq = lane >> 4;
  const int H = args.H;
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int n = n0 + 16 * f + 4 * lq;
    if (n >= H) continue;
    float bb[4] = {0.f, 0.f, 0.f, 0.f};
    if (args.bias) {
#pragma unroll
      for (int i = 0; i < 4; ++i) bb[i] = bf16_bits_to_f32(args.bias[(size_t)e * H + n + i]);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int row = 64 * sh + 16 * s + li;
      if (stok[row] < 0) continue;
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        y[i] = acc[f][s][i];
        if (args.bias) y[i] = rb(rb(y[i]) + bb[i]);
      }
      *reinterpret_cast<u32x2*>(args.out + (size_t)(m0 + row) * H + n) =
          u32x2{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
    }
  }
}

__device__ __forceinline__ float clamp_f32(float v, float lo, float hi) {
  v = (v > hi) ? hi : v;  // torch.clamp: NaN stays NaN
  v = (v < lo) ? lo : v;
  return v;
}

// The decode flow's activation in fp32 (moe_block_tkg.py:250-263).
__device__ __forceinline__ float act_fp32(float g, int act) {
  if (act == kSwish) return g * (1.0f / (1.0f + expf(-(g * 1.702f))));
  if (act == kSiLU) return g / (1.0f + expf(-g));
  return 0.5f * g * (1.0f + erff(g * 0.70710678118654752f));
}

// Decode-flow gate_up epilogue: fp32 bias, clamps and activation, h = up * act(gate) as
// the bf16 pair (hi, lo).
__device__ __forceinline__ void bf16_gate_up_store_f32(const Bf16Args& b, const f32x4 (&acc)[4][4],
                                                       const int32_t* stok, int m0, int e, int c0,
                                                       int sh) {
  const PrefillArgs& args = b.p;
  const int lane = threadIdx.x & 63, li = lane & 15, lq = lane >> 4;
  const int I = args.I;
#pragma unroll
  for (int pp = 0; pp < 2; ++pp) {
    const int col0 = c0 + 16 * pp + 4 * lq;
    if (col0 >= I) continue;
    float gb[4] = {0.f, 0.f, 0.f, 0.f}, ub[4] = {0.f, 0.f, 0.f, 0.f};
    if (args.bias) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        gb[i] = bf16_bits_to_f32(args.bias[(size_t)e * 2 * I + col0 + i]);
        ub[i] = bf16_bits_to_f32(args.bias[(size_t)e * 2 * I + I + col0 + i]);
      }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int row = 64 * sh + 16 * s + li;
      if (stok[row] < 0) continue;
      uint16_t hi[4], lo[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float g = clamp_f32(acc[2 * pp][s][i] + gb[i], args.p.gate_lo, args.p.gate_hi);
        const float u = clamp_f32(acc[2 * pp + 1][s][i] + ub[i], args.p.up_lo, args.p.up_hi);
        split_bf16(u * act_fp32(g, args.p.act), hi[i], lo[i]);
      }
      typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
      const size_t o = (size_t)(m0 + row) * I + col0;
      *reinterpret_cast<u16x4*>(args.out + o) = u16x4{hi[0], hi[1], hi[2], hi[3]};
      *reinterpret_cast<u16x4*>(b.out_lo + o) = u16x4{lo[0], lo[1], lo[2], lo[3]};
    }
  }
}

// Decode-flow down epilogue: y = acc + bias in fp32.
__device__ __forceinline__ void bf16_down_store_f32(const Bf16Args& b, const f32x4 (&acc)[4][4],
                                                    const int32_t* stok, int m0, int e, int n0,
                                                    int sh) {
  const PrefillArgs& args = b.p;
  const int lane = threadIdx.x & 63, li = lane & 15, lq = lane >> 4;
  const int H = args.H;
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int n = n0 + 16 * f + 4 * lq;
    if (n >= H) continue;
    f32x4 bb = {0.f, 0.f, 0.f, 0.f};
    if (args.bias) {
#pragma unroll
      for (int i = 0; i < 4; ++i) bb[i] = bf16_bits_to_f32(args.bias[(size_t)e * H + n + i]);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int row = 64 * sh + 16 * s + li;
      if (stok[row] < 0) continue;
      *reinterpret_cast<f32x4*>(b.y32 + (size_t)(m0 + row) * H + n) = acc[f][s] + bb;
    }
  }
}

template <bool GATE_UP, bool F32>
__global__ void __launch_bounds__(kBThreads)
    __attribute__((amdgpu_waves_per_eu(2, 2))) prefill_gemm_bf16_kernel(Bf16Args bargs) {
  const PrefillArgs& args = bargs.p;
  __shared__ __attribute__((aligned(1024))) uint8_t s_st[2][kBStage];
  __shared__ int32_t stok[kPM];
  __shared__ uint32_t s_rowoff[kPM];
  __shared__ int s_lastw[kPM / 64];
  PrefillTileId id;
  if (!prefill_tile_begin<GATE_UP>(args, stok, s_rowoff, s_lastw, id)) return;
  const int m0 = id.m0, e = id.e, nt = id.nt;
  __syncthreads();
  const int last = max(s_lastw[0], s_lastw[1]);
  if (last < 0) return;  // all 128 slots are padding (uniform over the workgroup)

  const int tid = threadIdx.x, wave = wave_id();
  const int fh = wave >> 1, sh = wave & 1;
  const bool active = last >= 64 * sh;  // this wave's 64 slots hold a real one
  const int K = args.K;
  // Weight rows: gate_up [E, H, 2, I] (a row = 2I: gate columns, then up), down [E, I, H].
  const size_t ldw = GATE_UP ? 2 * (size_t)args.I : (size_t)args.H;
  // This thread's weight column group (8 columns) of the N-tile.
  const int nb = tid & 15;
  int scol;
  bool wcol_ok;
  if (GATE_UP) {
    const int jn = nb >> 1;  // 16-column tile: pair jn / 2, gate (even) or up (odd)
    const int icol = nt * kBGateUpCols + 16 * (jn >> 1) + 8 * (nb & 1);
    wcol_ok = icol < args.I;
    scol = (jn & 1 ? args.I : 0) + (wcol_ok ? icol : 0);
  } else {
    const int n = nt * kBN + 8 * nb;
    wcol_ok = n < args.H;
    scol = wcol_ok ? n : 0;
  }
  // Buffer resources: this expert's weights (K rows of ldw), the activation rows (tokens,
  // or slots when the rows are per slot) and, for the decode flow's down GEMM, the lo rows.
  const __amdgpu_buffer_rsrc_t rw = bf16_rsrc(
      reinterpret_cast<const uint16_t*>(args.wq) + (size_t)e * K * ldw, (uint32_t)(K * ldw * 2));
  const uint32_t a_rows = (GATE_UP && !args.a_by_slot) ? (uint32_t)args.T
                                                       : (uint32_t)args.n_mtiles * kPM;
  const __amdgpu_buffer_rsrc_t ra = bf16_rsrc(args.a, a_rows * (uint32_t)K * 2u);
  uint32_t aoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) aoff[i] = s_rowoff[(tid >> 3) + 32 * i];
  f32x4 acc[4][4];
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[f][s] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nc = (K + kBK - 1) / kBK;
  // The decode flow's down GEMM runs its chunks twice: hi rows of h, then lo rows.
  constexpr bool TWO = F32 && !GATE_UP;
  const int ncc = TWO ? 2 * nc : nc;
  const __amdgpu_buffer_rsrc_t ra_lo =
      TWO ? bf16_rsrc(bargs.a_lo, a_rows * (uint32_t)K * 2u) : ra;
  auto load = [&](BChunk& r, int cc) {
    cc = min(cc, ncc - 1);  // past the last chunk: a re-read that is never stored
    const bool lo = TWO && cc >= nc;
    bf16_load(r, lo ? ra_lo : ra, aoff, rw, (uint32_t)scol, wcol_ok, (uint32_t)ldw, K,
              (lo ? cc - nc : cc) * kBK, last);
  };
  // Two LDS stages (chunk c in stage c % 2) and two register chunks: while chunk c's MFMAs
  // run, the loads of chunks c + 1 and c + 2 are in flight; chunk c + 1 goes to LDS after
  // them, and one barrier per chunk orders the stages.
  // Every load is issued unconditionally, in a fixed order (chunks past the last re-read
  // the last one): with loads on some paths only, the compiler could not count the loads
  // still in flight and would wait for all of them before each store.
  BChunk r0, r1;
  load(r0, 0);
  load(r1, 1);
  bf16_store_lds(r0, s_st[0]);
  load(r0, 2);
  __syncthreads();
  // Stores past the last chunk write re-read data that no compute reads.
  for (int c = 0; c < ncc; c += 2) {
    if (active) bf16_compute(s_st[0], fh, sh, acc);
    bf16_store_lds(r1, s_st[1]);
    __syncthreads();
    load(r1, c + 3);
    if (active && c + 1 < ncc) bf16_compute(s_st[1], fh, sh, acc);
    bf16_store_lds(r0, s_st[0]);
    __syncthreads();
    load(r0, c + 4);
  }
  if (!active) return;
  if constexpr (F32) {
    if (GATE_UP)
      bf16_gate_up_store_f32(bargs, acc, stok, m0, e, nt * kBGateUpCols + 32 * fh, sh);
    else
      bf16_down_store_f32(bargs, acc, stok, m0, e, nt * kBN + 64 * fh, sh);
    return;
  }
  if (GATE_UP) {
    const int c0 = nt * kBGateUpCols + 32 * fh;
    if (args.p.act == kSwish)
      bf16_gate_up_store<kSwish>(args, acc, stok, m0, e, c0, sh);
    else if (args.p.act == kSiLU)
      bf16_gate_up_store<kSiLU>(args, acc, stok, m0, e, c0, sh);
    else
      bf16_gate_up_store<kGELU>(args, acc, stok, m0, e, c0, sh);
  } else {
    bf16_down_store(args, acc, stok, m0, e, nt * kBN + 64 * fh, sh);
  }
}

int prefill_ntiles_bf16(bool gate_up, int64_t I, int64_t H) {
  return gate_up ? (int)((I + kBGateUpCols - 1) / kBGateUpCols) : (int)((H + kBN - 1) / kBN);
}

void launch_prefill_gemm_bf16(bool gate_up, const PrefillArgs& a, hipStream_t s) {
  const dim3 g(prefill_grid(a.n_mtiles, a.n_ntiles, a.group));
  const Bf16Args b = {a, nullptr, nullptr, nullptr};
  if (gate_up)
    hipLaunchKernelGGL((prefill_gemm_bf16_kernel<true, false>), g, dim3(kBThreads), 0, s, b);
  else
    hipLaunchKernelGGL((prefill_gemm_bf16_kernel<false, false>), g, dim3(kBThreads), 0, s, b);
}

void launch_decode_gemm_bf16(bool gate_up, const PrefillArgs& a, const uint16_t* a_lo,
                             uint16_t* out_lo, float* y32, hipStream_t s) {
  const dim3 g(prefill_grid(a.n_mtiles, a.n_ntiles, a.group));
  const Bf16Args b = {a, a_lo, out_lo, y32};
  if (gate_up)
    hipLaunchKernelGGL((prefill_gemm_bf16_kernel<true, true>), g, dim3(kBThreads), 0, s, b);
  else
    hipLaunchKernelGGL((prefill_gemm_bf16_kernel<false, true>), g, dim3(kBThreads), 0, s, b);
}

}  // namespace mxmoe
