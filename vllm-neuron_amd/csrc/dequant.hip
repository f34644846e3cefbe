// MXFP4 dequantization (bit-exact with the reference loader), MXFP8 dequantization (the
// MX definition), the hardware conversion probes and the MFMA operand-layout probe; also
// the error plumbing of the C-ABI.
#include <string.h>

#include "capi_util.h"
#include "common.h"

namespace mxmoe {

static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = 0; }

// One e2m1 code times 2^e as bf16 bits, built with integer arithmetic so no
// floating-point mode (denormal flushing) can interfere.  The reference computes
// bf16(float(v) * float(2^e)) (torch.ldexp into a bf16 buffer); v * 2^e is exact
// whenever it is finite, 2^128 overflows float (scale byte 255) giving +-inf, or
// NaN for a zero code, and results at or above 2^128 round to +-inf.
__device__ __forceinline__ uint16_t e2m1_ldexp_bf16(uint32_t code, uint32_t s) {
  const uint32_t sign = (code & 8u) << 12;  // bit 15
  const uint32_t mag = code & 7u;
  if (s == 255u) return mag == 0u ? (uint16_t)0xFFFFu : (uint16_t)(sign | 0x7F80u);
  if (mag == 0u) return (uint16_t)sign;
  // mag: 1 -> 0.5, 2 -> 1, 3 -> 1.5, 4 -> 2, 5 -> 3, 6 -> 4, 7 -> 6 = m * 2^x, m in {1, 1.5}
  const int x = (mag == 1u) ? -1 : (int)(mag >> 1) - 1;
  const uint32_t half = (mag >= 2u) ? (mag & 1u) : 0u;  // mantissa 1.5
  const int E = x + (int)s - 127;                     // unbiased exponent of the result
  if (E >= -126) {
    if (E + 127 >= 255) return (uint16_t)(sign | 0x7F80u);
    return (uint16_t)(sign | ((uint32_t)(E + 127) << 7) | (half << 6));
  }
  // Subnormal: value = (m * 2^(E+133)) * 2^-133, an integer count of the bf16 ulp.
  const uint32_t m2 = half ? 3u : 2u;  // 2m
  const int sh = E + 133 - 1;          // m * 2^(E+133) = (2m) * 2^(E+132)
  return (uint16_t)(sign | (m2 << sh));
}

// blocks [rows*G][16] bytes, scales [rows*G]; one thread per 4 bytes -> 8 bf16.
__global__ void __launch_bounds__(256) dequant_kernel(const uint32_t* __restrict__ blocks,
                                                      const uint8_t* __restrict__ scales,
                                                      uint16_t* __restrict__ out, int64_t n_words,
                                                      int hw) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_words) return;
  const uint32_t w = blocks[i];
  const uint32_t s = scales[i >> 2];  // 4 words per 32-element block
  u16x8 r;
  if (hw) {
    bf16x8 v = dequant8(w, e8m0_to_f32(s));
    r = __builtin_bit_cast(u16x8, v);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) r[k] = e2m1_ldexp_bf16((w >> (4 * k)) & 15u, s);
  }
  *reinterpret_cast<u16x8*>(out + i * 8) = r;
}

// One E4M3FN code times 2^(s - 127) as bf16 bits, by integer arithmetic (the MX value:
// scale byte 255 and the codes S.1111.111 are NaN; no infinities in E4M3FN).  The code is
// M x 2^X with an integer M < 16, so the product is exact in float32 (its smallest value,
// 2^-136, is a float32 subnormal; its largest overflows to +-inf) and rounds once to
// bf16: exactly for normal results, to the nearest even multiple of 2^-133 below 2^-126.
__device__ __forceinline__ uint16_t e4m3_ldexp_bf16(uint32_t code, uint32_t s) {
  const uint32_t sign = (code & 0x80u) << 8;
  const uint32_t e = (code >> 3) & 15u, m = code & 7u;
  if (s == 255u || (e == 15u && m == 7u)) return (uint16_t)(sign | 0x7FC0u);
  if (e == 0u && m == 0u) return (uint16_t)sign;
  const uint32_t M = e ? 8u + m : m;
  const int X = (e ? (int)e - 10 : -9) + (int)s - 127;  // value = M * 2^X
  const int L = 32 - __clz(M);                            // bit length of M, 1..4
  const int E = X + L - 1;                                 // unbiased exponent
  if (E > 127) return (uint16_t)(sign | 0x7F80u);
  if (E >= -126) {
    const uint32_t frac = (M << (8 - L)) & 0x7Fu;          // L - 1 <= 3 fraction bits
    return (uint16_t)(sign | ((uint32_t)(E + 127) << 7) | frac);
  }
  const int sh = X + 133;  // value / 2^-133 = M * 2^sh
  if (sh >= 0) return (uint16_t)(sign | (M << sh));
  const int k = -sh;  // 1..3
  const uint32_t q = M >> k, rem = M & ((1u << k) - 1u), half = 1u << (k - 1);
  const uint32_t r = q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
  return (uint16_t)(sign | r);
}

// codes [rows*G][32] bytes, scales [rows*G]; one thread per 8 codes -> 8 bf16.  hw: the
// CDNA4 scaled fp8 conversion the GEMMs use, else e4m3_ldexp_bf16.
__global__ void __launch_bounds__(256) dequant_fp8_kernel(const uint2* __restrict__ codes,
                                                          const uint8_t* __restrict__ scales,
                                                          uint16_t* __restrict__ out,
                                                          int64_t n_pairs, int hw) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_pairs) return;
  const uint2 w = codes[i];
  const uint32_t s = scales[i >> 2];  // 4 x 8 codes per 32-element block
  u16x8 r;
  if (hw) {
    const float sc = e8m0_to_f32(s);
    const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, sc, false);
    const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, sc, true);
    const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, sc, false);
    const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, sc, true);
    const bf16x8 v = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    r = __builtin_bit_cast(u16x8, v);
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      r[k] = e4m3_ldexp_bf16((w.x >> (8 * k)) & 0xFFu, s);
      r[4 + k] = e4m3_ldexp_bf16((w.y >> (8 * k)) & 0xFFu, s);
    }
  }
  *reinterpret_cast<u16x8*>(out + i * 8) = r;
}

static int run_dequant_fp8(const uint8_t* codes, const uint8_t* scales, uint16_t* out,
                           int64_t rows, int64_t K, void* stream, int hw) {
  clear_error();
  MXMOE_REQUIRE(codes && scales && out, "dequant_mxfp8: null pointer");
  MXMOE_REQUIRE(rows >= 0 && K >= 0 && K % 32 == 0,
                "dequant_mxfp8: K=%lld must be a multiple of 32", (long long)K);
  const int64_t n_pairs = rows * (K / 8);
  if (n_pairs == 0) return MXMOE_OK;
  hipLaunchKernelGGL(dequant_fp8_kernel, dim3((unsigned)((n_pairs + 255) / 256)), dim3(256), 0,
                     as_stream(stream), reinterpret_cast<const uint2*>(codes), scales, out,
                     n_pairs, hw);
  return check_launch("dequant_mxfp8");
}

__global__ void mfma_probe_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                  float* __restrict__ d) {
  const int l = threadIdx.x;
  const int row = l & 15, kq = (l >> 4) * 8;
  u16x8 av, bv;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    av[k] = a[row * 32 + kq + k];
    bv[k] = b[row * 32 + kq + k];
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = mfma16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv), acc);
#pragma unroll
  for (int i = 0; i < 4; ++i) d[(4 * (l >> 4) + i) * 16 + (l & 15)] = acc[i];
}

static int run_dequant(const uint8_t* blocks, const uint8_t* scales, uint16_t* out, int64_t rows,
                       int64_t K, void* stream, int hw) {
  clear_error();
  MXMOE_REQUIRE(blocks && scales && out, "dequant: null pointer");
  MXMOE_REQUIRE(rows >= 0 && K >= 0 && K % 32 == 0, "dequant: K=%lld must be a multiple of 32",
                (long long)K);
  const int64_t n_words = rows * (K / 8);
  if (n_words == 0) return MXMOE_OK;
  const int64_t grid = (n_words + 255) / 256;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)grid), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint32_t*>(blocks), scales, out, n_words, hw);
  return check_launch("dequant");
}

}  // namespace mxmoe

using namespace mxmoe;

extern "C" int mxmoe_version(void) { return 100; }

extern "C" const char* mxmoe_last_error(void) { return g_err; }

extern "C" int mxmoe_dequant_bf16(const uint8_t* blocks, const uint8_t* scales, uint16_t* out,
                                  int64_t rows, int64_t K, void* stream) {
  return run_dequant(blocks, scales, out, rows, K, stream, 0);
}

extern "C" int mxmoe_probe_hw_dequant(const uint8_t* blocks, const uint8_t* scales,
                                      uint16_t* out, int64_t rows, int64_t K, void* stream) {
  return run_dequant(blocks, scales, out, rows, K, stream, 1);
}

extern "C" int mxmoe_dequant_mxfp8_bf16(const uint8_t* codes, const uint8_t* scales,
                                        uint16_t* out, int64_t rows, int64_t K, void* stream) {
  return run_dequant_fp8(codes, scales, out, rows, K, stream, 0);
}

extern "C" int mxmoe_probe_hw_dequant_fp8(const uint8_t* codes, const uint8_t* scales,
                                          uint16_t* out, int64_t rows, int64_t K,
                                          void* stream) {
  return run_dequant_fp8(codes, scales, out, rows, K, stream, 1);
}

extern "C" int mxmoe_probe_mfma(const uint16_t* a, const uint16_t* b, float* d, void* stream) {
  clear_error();
  MXMOE_REQUIRE(a && b && d, "probe_mfma: null pointer");
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(1), dim3(64), 0, as_stream(stream), a, b, d);
  return check_launch("probe_mfma");
}
