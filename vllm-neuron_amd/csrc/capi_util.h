// Host-side helpers shared by the C-ABI entry points: per-thread error text,
// argument checks, HIP status propagation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/mxfp4_moe.h"

namespace mxmoe {

int set_error(int code, const char* fmt, ...);
void clear_error();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Status of the launches just issued on the stream (does not synchronize).
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MXMOE_E_HIP, "%s: %s", what, hipGetErrorString(e));
  return MXMOE_OK;
}

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Profiling marks: ev is null or an array of hipEvent_t handles supplied by the caller.
inline void mark_event(void* const* ev, int i, hipStream_t s) {
  if (ev) (void)hipEventRecord(reinterpret_cast<hipEvent_t>(ev[i]), s);
}

// Operands and roundings of one router call (router.hip).  Dtypes are MXMOE_DT_* codes;
// op is how the 16-bit operands are multiplied (kOpBF16, kOpF16 or kOpExact, common.h);
// the bias, the logits and the activation outputs are rounded to bias_rnd, logit_rnd and
// act_rnd (MXMOE_DT_F32 leaves them in fp32).
struct RouterSpec {
  const uint16_t* x = nullptr;  // [T, H]
  int x_dt = MXMOE_DT_BF16;
  const uint16_t* w = nullptr;  // [E, H]
  int w_dt = MXMOE_DT_BF16;
  const void* bias = nullptr;  // [E] or null
  int bias_dt = MXMOE_DT_BF16;
  int op = 0;
  int bias_rnd = MXMOE_DT_F32, logit_rnd = MXMOE_DT_F32, act_rnd = MXMOE_DT_F32;
};

int router_check(const RouterSpec& r);

// Router logits + top-k + activation (router.hip); affinities / aff16 may be null.
int router_run(const RouterSpec& r, int64_t T, int64_t H, int64_t E, int top_k, int act,
               int act_before_topk, int renorm, float renorm_eps, float* logits,
               float* affinities, uint16_t* aff16, int32_t* topk_idx, float* topk_val,
               hipStream_t s);

// RMSNorm of bf16 rows into bf16 or fp16 (router.hip): the mean square over the first ha
// columns (all_cols = 0; columns >= ha written as 0) or over all H columns divided by ha
// (all_cols = 1).
int rmsnorm_run(const uint16_t* x, const float* gamma, int64_t T, int64_t H, int64_t ha,
                int all_cols, float eps, int out_dt, uint16_t* out, hipStream_t s);

// Decode with bf16 expert weights by streaming items (expert_decode.hip): the routing,
// tiles, activation and combine of the MXFP4 decode, for batches whose experts hold few
// 16-token tiles.
size_t tkg_bf16_stream_workspace(int64_t T, int64_t H, int64_t I, int64_t E, int K);
int tkg_bf16_stream(const uint16_t* x, const int32_t* topk_idx, const float* topk_val,
                    const uint16_t* gu_w, const uint16_t* dn_w, const uint16_t* gu_bias,
                    const uint16_t* dn_bias, int64_t T, int64_t H, int64_t I, int64_t E,
                    int top_k, int act, const float* clamps, int scale_mode, uint16_t* out,
                    void* workspace, size_t workspace_bytes, hipStream_t s);

// Blocks of the blockwise mapping of T tokens with top_k experts each over E experts at
// block size B: the reference's bound (moe_blockwise.py:343-349), at most one block per
// routed slot.
inline int64_t blockwise_n_blocks(int64_t T, int64_t E, int top_k, int64_t B) {
  const int64_t total = T * (top_k < E ? top_k : E);
  int64_t nb = (total - (E - 1) + B - 1) / B;
  if (total - (E - 1) <= 0) nb = (total - (E - 1)) / B;  // ceil of a non-positive value
  nb += E - 1;
  return nb > total ? total : nb;
}

// Bump allocator over a caller-provided workspace.
struct Carver {
  char* base;
  size_t cap;
  size_t off = 0;
  Carver(void* b, size_t c) : base(static_cast<char*>(b)), cap(c) {}
  template <typename T>
  T* take(size_t count) {
    off = align_up(off, 256);
    T* p = reinterpret_cast<T*>(base + off);
    off += count * sizeof(T);
    return p;
  }
  bool ok() const { return off <= cap; }
};

}  // namespace mxmoe

#define MXMOE_REQUIRE(cond, ...)                                    \
  do {                                                              \
    if (!(cond)) return ::mxmoe::set_error(MXMOE_E_INVALID, __VA_ARGS__); \
  } while (0)
