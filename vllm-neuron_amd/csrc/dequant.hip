// MXFP4 dequantization (bit-exact with the reference loader), the hardware
// conversion probe and the MFMA operand-layout probe; also the error plumbing of
// the C-ABI.
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

extern "C" int mxmoe_probe_mfma(const uint16_t* a, const uint16_t* b, float* d, void* stream) {
  clear_error();
  MXMOE_REQUIRE(a && b && d, "probe_mfma: null pointer");
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(1), dim3(64), 0, as_stream(stream), a, b, d);
  return check_launch("probe_mfma");
}
