// Shared device helpers for the MXFP4 MoE kernels (gfx950 / CDNA4 only).
//
// Weight tile layout ("row-group/chunk" layout), produced once at load time by
// vllm_neuron_amd.weights.pack_mxfp4 from the OCP/HF checkpoint layout
// (blocks [N, K/32, 16] uint8 low-nibble-first + scales [N, K/32] uint8 E8M0):
//   * rows are grouped by 16 (row group rg = n / 16);
//   * K is cut into chunks of 128 elements (64 bytes per row), the last chunk
//     may hold 1..3 blocks of 32;
//   * inside a chunk, lane l of a wave owns row rg*16 + (l % 16) and K-block
//     4*c + l/16: its 16 bytes are stored at  rg*(K*8) + c*1024 + l*16, so a wave
//     reads one chunk of one row group with a single coalesced 1 KiB load;
//   * scales keep row groups four at a time (quad q = rg / 4, r = rg % 4): the
//     E8M0 byte of that lane is at q*(2K) + c*256 + 4*l + r, so one 32-bit load
//     per lane gives the scales of a quad's four row groups; a partial last quad
//     is padded with zero bytes.
// A row group therefore occupies K*8 data bytes and a quad 2K scale bytes.
//
// MFMA operand convention (v_mfma_f32_16x16x32_bf16): A lane l holds row l%16,
// B lane l holds column l%16, and both hold 8 K-values chosen by (l/16, element).
// Only the pairing between A and B matters for a dot product, so every kernel
// feeds lane l of both operands the same 8 K-indices
//   k = 128*c + 32*(l/16) + 8*j + [0..7]     for MFMA j in 0..3 of chunk c,
// which for the weights is dword j of the lane's 16 bytes.
// D lane l, element i holds row 4*(l/16)+i, column l%16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

namespace mxmoe {

constexpr int kChunkK = 128;       // K elements per chunk
constexpr int kChunkBytes = 1024;  // data bytes per chunk of a row group
constexpr int kRowGroup = 16;

// Wave index inside the workgroup as a wave-uniform (scalar) value, so branches
// on it stay scalar instead of turning into EXEC-mask divergence.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float((uint32_t)b << 16);
}

// Round-to-nearest-even float -> bf16 bits.  NaN maps to 0xFFFF, the pattern the
// reference's CPU conversion of float32 tensors to bfloat16 produces.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xFFFFu;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

// Round-to-nearest-even float -> fp16 bits (overflow to +-inf, as a tensor cast does).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Element types of the C-ABI (MXMOE_DT_*): 0 fp32, 1 fp16, 2 bf16.
enum Dt : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

// How the router multiplies its 16-bit operands (router_logits_kernel).
constexpr int kOpBF16 = 0, kOpF16 = 1, kOpExact = 2;

// f rounded to the precision of dt (a cast to dt and back to fp32).
__device__ __forceinline__ float round_to(float f, int dt) {
  if (dt == kF16) return (float)(_Float16)f;
  if (dt == kBF16) return round_bf16(f);
  return f;
}

// Element i of an array of element type dt, as fp32 (exact).  Branch-free: two 16-bit
// loads that are always issued (an fp32 element's halves, or the 16-bit element twice),
// so that several calls' loads issue together instead of one basic block per load.
__device__ __forceinline__ float load_as_f32(const void* p, size_t i, int dt) {
  const uint16_t* h = static_cast<const uint16_t*>(p);
  const bool f32 = dt == kF32;
  const uint16_t b0 = h[f32 ? 2 * i : i], b1 = h[f32 ? 2 * i + 1 : i];
  const float v16 = dt == kF16 ? f16_bits_to_f32(b0) : bf16_bits_to_f32(b0);
  return f32 ? __uint_as_float((uint32_t)b0 | ((uint32_t)b1 << 16)) : v16;
}

// Element i of an optional array p (null: 0.0f) as fp32.  Its loads are always issued (from
// `fallback`, any array of at least i + 1 floats, when p is null) and the value is masked
// by a bit-and, so that no branch puts the loads in a block of their own.
__device__ __forceinline__ float load_opt_f32(const void* p, size_t i, int dt,
                                              const void* fallback) {
  const float v = load_as_f32(p ? p : fallback, i, p ? dt : kF32);
  return __uint_as_float(__float_as_uint(v) & (p ? 0xffffffffu : 0u));
}

// Eight 16-bit values (a 16-byte load) in one type, as eight of another.
__device__ __forceinline__ bf16x8 f16x8_to_bf16x8(u32x4 v) {  // RNE, like a tensor cast
  const u16x8 h = __builtin_bit_cast(u16x8, v);
  u16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = f32_to_bf16_bits(f16_bits_to_f32(h[i]));
  return __builtin_bit_cast(bf16x8, r);
}

__device__ __forceinline__ f16x8 bf16x8_to_f16x8(u32x4 v) {  // RNE, like a tensor cast
  const u16x8 h = __builtin_bit_cast(u16x8, v);
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (_Float16)bf16_bits_to_f32(h[i]);
  return r;
}

// fp16 values as an exact sum hi + lo of two bf16 values: hi is the value rounded to
// bf16 (8 significant bits), lo the remainder (at most 3 more bits, also exact), so
// products with bf16 operands stay exact in fp32 over two bf16 MFMAs.
__device__ __forceinline__ void f16x8_split_bf16(u32x4 v, bf16x8& hi, bf16x8& lo) {
  const u16x8 h = __builtin_bit_cast(u16x8, v);
  u16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float f = f16_bits_to_f32(h[i]);
    a[i] = f32_to_bf16_bits(f);
    b[i] = f32_to_bf16_bits(f - bf16_bits_to_f32(a[i]));
  }
  hi = __builtin_bit_cast(bf16x8, a);
  lo = __builtin_bit_cast(bf16x8, b);
}

__device__ __forceinline__ f32x4 mfma16_f16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// E8M0 exponent byte -> float 2^(s-127); s = 0 gives the subnormal 2^-127 and
// s = 255 gives +inf (the value 2^128 overflows float).
__device__ __forceinline__ float e8m0_to_f32(uint32_t s) {
  return __uint_as_float(s ? (s << 23) : 0x00400000u);
}

// Four bytes (8 e2m1 codes, low nibble = even element) times the block scale,
// converted to 8 bf16 with the CDNA4 scaled-conversion instruction.
__device__ __forceinline__ bf16x8 dequant8(uint32_t w, float scale) {
  bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
  bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
  bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
  bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
  bf16x8 r = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
  return r;
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  return __builtin_bit_cast(bf16x8, v);
}

// Split a float into a bf16 high part and a bf16 remainder so that hi + lo carries
// ~16 significant bits; two MFMAs over (hi, lo) give fp32-grade products.
__device__ __forceinline__ void split_bf16(float v, uint16_t& hi, uint16_t& lo) {
  hi = f32_to_bf16_bits(v);
  lo = f32_to_bf16_bits(v - bf16_bits_to_f32(hi));
}

__device__ __forceinline__ float sigmoid_f32(float x) {
  return 1.0f / (1.0f + expf(-x));
}

// Activation kinds, numbered like the C-ABI (include/mxfp4_moe.h).
enum Act : int { kSiLU = 0, kGELU = 1, kSwish = 2 };

struct ExpertParams {
  float gate_lo, gate_hi, up_lo, up_hi;  // clamps; +-inf when absent
  int act;
};

}  // namespace mxmoe
