// Token -> expert permutation.
//
// (1) Blockwise mapping for the prefill path, bit-exact with the reference torch
//     flow: a stable counting sort of routed (token, expert) pairs by expert, each
//     expert's run padded with -1 to a multiple of the block size.
//     Chunks of 256 tokens (4 waves x 64).  Inside a chunk every wave builds one
//     64-bit token mask per expert in LDS (atomicOr of the lane bit); the rank of a
//     token among the chunk's tokens of an expert is popcounts of the earlier
//     waves' masks plus popcount(own mask & lanes below).  Per-chunk counts are
//     scanned per expert, experts are scanned into block offsets, then tokens are
//     scattered.  No step depends on atomic ordering, so the result is unique.
// (2) The decode routing for moe_tkg: same ranking inside one workgroup, from
//     top-k indices, producing per-expert slot lists and per-token slot lists.
#include "capi_util.h"
#include "common.h"

namespace mxmoe {

constexpr int kChunkTok = 256;
constexpr int kMaxE = 1024;

__device__ __forceinline__ bool routed(const float* aff_row, int e) { return aff_row[e] != 0.0f; }

// Pass 1: per-chunk expert counts and the masked affinities.
__global__ void __launch_bounds__(256) bw_count_kernel(const float* __restrict__ aff,
                                                       const uint8_t* __restrict__ pmask, int T,
                                                       int E, float* __restrict__ aff_masked,
                                                       int32_t* __restrict__ chunk_counts) {
  extern __shared__ unsigned long long masks[];  // [4][E]
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < 4 * E; i += 256) masks[i] = 0ull;
  __syncthreads();
  const int t = blockIdx.x * kChunkTok + threadIdx.x;
  if (t < T) {
    const float* row = aff + (size_t)t * E;
    float* mrow = aff_masked + (size_t)t * E;
    const float pm = pmask ? (pmask[t] ? 1.0f : 0.0f) : 1.0f;
    for (int e = 0; e < E; ++e) {
      const float a = row[e];
      mrow[e] = pmask ? a * pm : a;
      if (a != 0.0f) atomicOr(&masks[wave * E + e], 1ull << lane);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 256) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) c += __popcll(masks[w * E + e]);
    chunk_counts[(size_t)blockIdx.x * E + e] = c;
  }
}

// Pass 2 (one workgroup of 1024 threads): per-expert chunk prefix, block counts,
// block offsets, block_to_expert, conditions.
__global__ void __launch_bounds__(1024) bw_scan_kernel(
    int32_t* __restrict__ chunk_counts, int n_chunks, int E, int B, int N,
    int32_t* __restrict__ expert_pos, int32_t* __restrict__ block_to_expert,
    int32_t* __restrict__ conditions, int32_t* __restrict__ expert_counts) {
  __shared__ int cum[kMaxE];  // inclusive cumulative blocks per expert
  __shared__ int wsum[16];
  const int e = threadIdx.x;
  int total = 0, nb = 0;
  if (e < E) {
    for (int c = 0; c < n_chunks; ++c) {
      const int v = chunk_counts[(size_t)c * E + e];
      chunk_counts[(size_t)c * E + e] = total;  // exclusive prefix within the expert
      total += v;
    }
    nb = (total + B - 1) / B;
    if (expert_counts) expert_counts[e] = total;
  }
  // Inclusive block scan over experts: wave scan, then across waves.
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int v = nb;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(v, off);
    if (lane >= off) v += o;
  }
  if (lane == 63) wsum[wave] = v;
  __syncthreads();
  int pre = 0;
  for (int w = 0; w < wave; ++w) pre += wsum[w];
  v += pre;
  if (e < E) {
    cum[e] = v;
    expert_pos[e] = (v - nb) * B;  // first slot of the expert's run
  }
  __syncthreads();
  const int used = cum[E - 1];
  for (int n = threadIdx.x; n < N; n += 1024) {
    // block_to_expert[n] = #{e < E-1 : n >= cum[e]}  (cum is non-decreasing)
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (cum[mid] <= n) lo = mid + 1;
      else hi = mid;
    }
    block_to_expert[n] = lo;
    // A block inside a run holds at least one token; blocks past the runs are empty.
    conditions[n] = n < used ? 1 : 0;
  }
}

// Pass 3: scatter token ids.  token_position_to_id was filled with -1 beforehand.
__global__ void __launch_bounds__(256) bw_scatter_kernel(
    const float* __restrict__ aff, int T, int E, const int32_t* __restrict__ chunk_prefix,
    const int32_t* __restrict__ expert_pos, int32_t* __restrict__ tp2id, int64_t n_slots) {
  extern __shared__ unsigned long long masks[];  // [4][E]
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < 4 * E; i += 256) masks[i] = 0ull;
  __syncthreads();
  const int t = blockIdx.x * kChunkTok + threadIdx.x;
  const float* row = aff + (size_t)min(t, T - 1) * E;
  if (t < T)
    for (int e = 0; e < E; ++e)
      if (routed(row, e)) atomicOr(&masks[wave * E + e], 1ull << lane);
  __syncthreads();
  if (t >= T) return;
  const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int e = 0; e < E; ++e) {
    if (!routed(row, e)) continue;
    int rank = chunk_prefix[(size_t)blockIdx.x * E + e];
    for (int w = 0; w < wave; ++w) rank += __popcll(masks[w * E + e]);
    rank += __popcll(masks[wave * E + e] & below);
    const int64_t pos = (int64_t)expert_pos[e] + rank;
    if (pos < n_slots) tp2id[pos] = t;
  }
}

__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace mxmoe

using namespace mxmoe;

static size_t bw_ws(int64_t T, int64_t E) {
  const int64_t nch = (T + kChunkTok - 1) / kChunkTok;
  return align_up((size_t)(nch * E) * 4, 256) + align_up((size_t)E * 4, 256) + 256;
}

extern "C" size_t mxmoe_blockwise_workspace_bytes(int64_t T, int64_t E) { return bw_ws(T, E); }

extern "C" int mxmoe_blockwise_mapping(const float* affinities, const uint8_t* padding_mask,
                                       int64_t T, int64_t E, int top_k, int64_t block_size,
                                       int64_t n_blocks, float* affinities_masked,
                                       int32_t* token_position_to_id, int32_t* block_to_expert,
                                       int32_t* conditions, int32_t* expert_counts,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  MXMOE_REQUIRE(affinities && affinities_masked && token_position_to_id && block_to_expert &&
                    conditions && workspace,
                "blockwise_mapping: null pointer");
  MXMOE_REQUIRE(T >= 1 && E >= 1 && E <= kMaxE, "blockwise_mapping: T=%lld E=%lld out of range",
                (long long)T, (long long)E);
  MXMOE_REQUIRE(block_size >= 1 && top_k >= 1, "blockwise_mapping: bad block_size/top_k");
  const int64_t total = T * (top_k < E ? top_k : E);
  int64_t nb = (total - (E - 1) + block_size - 1) / block_size;
  if (total - (E - 1) <= 0) nb = (total - (E - 1)) / block_size;  // ceil of a non-positive value
  nb += E - 1;
  if (nb > total) nb = total;
  MXMOE_REQUIRE(n_blocks == nb, "blockwise_mapping: n_blocks=%lld, expected %lld",
                (long long)n_blocks, (long long)nb);
  if (workspace_bytes < bw_ws(T, E))
    return set_error(MXMOE_E_WORKSPACE, "blockwise_mapping: workspace %zu < %zu", workspace_bytes,
                     bw_ws(T, E));
  Carver cv(workspace, workspace_bytes);
  const int64_t nch = (T + kChunkTok - 1) / kChunkTok;
  int32_t* chunk_counts = cv.take<int32_t>(nch * E);
  int32_t* expert_pos = cv.take<int32_t>(E);
  hipStream_t s = as_stream(stream);
  const int64_t n_slots = n_blocks * block_size;
  hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)((n_slots + 255) / 256)), dim3(256), 0, s,
                     token_position_to_id, n_slots, -1);
  const size_t lds = (size_t)4 * E * sizeof(unsigned long long);
  hipLaunchKernelGGL(bw_count_kernel, dim3((unsigned)nch), dim3(256), lds, s, affinities,
                     padding_mask, (int)T, (int)E, affinities_masked, chunk_counts);
  hipLaunchKernelGGL(bw_scan_kernel, dim3(1), dim3(1024), 0, s, chunk_counts, (int)nch, (int)E,
                     (int)block_size, (int)n_blocks, expert_pos, block_to_expert, conditions,
                     expert_counts);
  hipLaunchKernelGGL(bw_scatter_kernel, dim3((unsigned)nch), dim3(256), lds, s, affinities,
                     (int)T, (int)E, chunk_counts, expert_pos, token_position_to_id, n_slots);
  return check_launch("blockwise_mapping");
}
