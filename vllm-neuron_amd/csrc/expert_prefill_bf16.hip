// Expert GEMMs of bf16 expert weights (prefill and decode): the reference's shard_on_block operands
// (vllm_neuron/functional/moe/moe_cte.py:117-124, model_bf16.py:1360-1391), gate_up
// [E, H, 2, I] and down [E, I, H], each expert's rows running along K.  Same blockwise
// schedule (tile order, XCD groups), slot tables and epilogues as the MX GEMMs, which
// stream packed codes instead.
//
// Workgroup tile: 128 slots x 128 output columns over K in 128-wide chunks, 4 waves in a
// 2 x 2 grid (wave w: slots 64 (w & 1) .. +63, columns 64 (w >> 1) .. +63), each wave
// 4 x 4 MFMA 16x16x32 tiles.  The weights are the MFMA's A operand (rows = output
// columns) and the slots' activations its B operand, so a lane ends with 4 consecutive
// output columns of one slot (one 8-byte store).  Both operands pass through LDS, one
// chunk at a time:
//   activations: 128 rows x 256 B, 16-byte blocks XOR-swizzled by row (the 16 rows an
//     operand read touches then hit distinct banks);
//   weights: transposed, [column][k] (256 B per column, the same swizzle), so a lane's
//     8 K-values of a column are one 16-byte LDS read.  A thread loads an 8 (k) x 8
//     (column) block with 8 row loads of 16 B (16 lanes read 256 contiguous bytes of a
//     row), transposes it in registers with byte permutes and writes 8 columns of 16 B.
// The next chunk's global loads are issued before the current chunk's MFMAs and land in
// registers while they run; LDS is refilled between two barriers.  64 KiB of LDS per
// workgroup: two workgroups per CU.
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
constexpr int kBK = 128;               // K per chunk
constexpr int kBRow = kBK * 2;         // bytes of one LDS row (a slot's or a column's chunk)
constexpr int kBThreads = 256;
constexpr int kBGateUpCols = kBN / 2;  // intermediate columns of a gate_up N-tile
static_assert(kBThreads == 16 * 16, "one 8 x 8 weight block per thread and chunk");
static_assert(kPM * (kBRow / 16) == 8 * kBThreads, "8 activation blocks per thread and chunk");

// The decode flow's extra operands (null in the prefill flow).
struct Bf16Args {
  PrefillArgs p;
  const uint16_t* a_lo;  // down: lo part of h [slots, I]
  uint16_t* out_lo;      // gate_up: lo part of h [slots, I]
  float* y32;            // down: y [slots, H] fp32
};

// LDS byte offset of 16-byte block `blk` (0..15) of row `row`.
__device__ __forceinline__ uint32_t bsw(int row, int blk) {
  return (uint32_t)row * kBRow + (uint32_t)((blk ^ (row & 15)) << 4);
}

// in[r] = 8 bf16 of row r (word w = columns 2w, 2w + 1) -> out[j] = 8 bf16 of column j
// (word v = rows 2v, 2v + 1; the lower row in the low half).
__device__ __forceinline__ void transpose8x8(const u32x4 (&in)[8], u32x4 (&out)[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint32_t a = in[2 * v][w], b = in[2 * v + 1][w];
      out[2 * w][v] = __builtin_amdgcn_perm(b, a, 0x05040100u);      // low halves
      out[2 * w + 1][v] = __builtin_amdgcn_perm(b, a, 0x07060302u);  // high halves
    }
}

// One chunk's global -> register loads of a thread: 8 activation blocks (rows
// tid / 16 + 16 i, block tid % 16) and an 8 x 8 weight block (rows 8 (tid / 16) ..,
// columns of group tid % 16).  Past K, for columns past the projection and for slots
// after the tile's last real one (padding: its outputs are never stored), zeros.
struct BChunk {
  u32x4 a[8];
  u32x4 w[8];
};

template <bool GATE_UP>
__device__ __forceinline__ void bf16_load(BChunk& r, const char* abase, const uint32_t (&aoff)[8],
                                          const uint16_t* wsrc, bool wcol_ok, size_t ldw, int K,
                                          int kc, int last) {
  const int tid = threadIdx.x;
  const int blk = tid & 15, kb = tid >> 4;
  const u32x4 z = {0u, 0u, 0u, 0u};
  const bool a_ok = kc + 8 * blk < K;  // K % 32 == 0: a block is whole or past K
#pragma unroll
  for (int i = 0; i < 8; ++i)
    r.a[i] = (a_ok && kb + 16 * i <= last)
                 ? *reinterpret_cast<const u32x4*>(abase + aoff[i] + (size_t)(kc + 8 * blk) * 2)
                 : z;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int k = kc + 8 * kb + j;
    r.w[j] = (wcol_ok && k < K) ? *reinterpret_cast<const u32x4*>(wsrc + (size_t)k * ldw) : z;
  }
}

__device__ __forceinline__ void bf16_store_lds(const BChunk& r, uint8_t* sa, uint8_t* sw) {
  const int tid = threadIdx.x;
  const int blk = tid & 15, kb = tid >> 4;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    *reinterpret_cast<u32x4*>(sa + bsw(kb + 16 * i, blk)) = r.a[i];
  u32x4 t[8];
  transpose8x8(r.w, t);
#pragma unroll
  for (int j = 0; j < 8; ++j) *reinterpret_cast<u32x4*>(sw + bsw(8 * blk + j, kb)) = t[j];
}

// One chunk's MFMAs of a wave: 4 K-steps of 32, each 4 weight and 4 activation operand
// reads (lane l: row l % 16 of the tile, K-values 8 (l / 16) .. + 7 of the step).  All 4
// subtiles run: skipping those past the tile's last real slot branched around each MFMA
// and measured 15 % slower.
__device__ __forceinline__ void bf16_compute(const uint8_t* sa, const uint8_t* sw, int fh, int sh,
                                             f32x4 (&acc)[4][4]) {
  const int lane = threadIdx.x & 63, li = lane & 15, lq = lane >> 4;
#pragma unroll
  for (int ks = 0; ks < kBK / 32; ++ks) {
    const int blk = 4 * ks + lq;
    bf16x8 wa[4], xb[4];
#pragma unroll
    for (int f = 0; f < 4; ++f)
      wa[f] = as_bf16x8(*reinterpret_cast<const u32x4*>(sw + bsw(64 * fh + 16 * f + li, blk)));
#pragma unroll
    for (int s = 0; s < 4; ++s)
      xb[s] = as_bf16x8(*reinterpret_cast<const u32x4*>(sa + bsw(64 * sh + 16 * s + li, blk)));
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        acc[f][s] = mfma16(wa[f], xb[s], acc[f][s]);
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
  __shared__ __attribute__((aligned(1024))) uint8_t s_a[kPM * kBRow], s_w[kBN * kBRow];
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
  const uint16_t* wbase = reinterpret_cast<const uint16_t*>(args.wq) + (size_t)e * K * ldw + scol;
  uint32_t aoff[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) aoff[i] = s_rowoff[(tid >> 4) + 16 * i];
  const char* abase = reinterpret_cast<const char*>(args.a);

  f32x4 acc[4][4];
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[f][s] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nc = (K + kBK - 1) / kBK;
  // The decode flow's down GEMM runs its chunks twice: hi rows of h, then lo rows.
  constexpr bool TWO = F32 && !GATE_UP;
  const int ncc = TWO ? 2 * nc : nc;
  const char* abase_lo = TWO ? reinterpret_cast<const char*>(bargs.a_lo) : abase;
  BChunk r;
  bf16_load<GATE_UP>(r, abase, aoff, wbase, wcol_ok, ldw, K, 0, last);
  bf16_store_lds(r, s_a, s_w);
  __syncthreads();
  for (int c = 0; c < ncc; ++c) {
    const bool more = c + 1 < ncc;
    if (more) {
      const int cn = c + 1;
      const bool lo = TWO && cn >= nc;
      bf16_load<GATE_UP>(r, lo ? abase_lo : abase, aoff, wbase, wcol_ok, ldw, K,
                         (lo ? cn - nc : cn) * kBK, last);
    }
    if (active) bf16_compute(s_a, s_w, fh, sh, acc);
    __syncthreads();
    if (more) {
      bf16_store_lds(r, s_a, s_w);
      __syncthreads();
    }
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
