// Token -> expert permutation for the prefill path (blockwise mapping), bit-exact with
// the reference torch flow: a stable counting sort of the routed (token, expert) pairs
// by expert, each expert's run padded with -1 to a multiple of the block size.
//
// Chunks of 64 tokens, one workgroup of 256 threads each: four threads per token read
// its affinity row with 16-byte loads (each nonzero sets the token's bit in a 64-bit
// LDS mask of its expert).  The rank of a pair among the chunk's tokens of its expert
// is popcount(mask & tokens below); per-chunk counts are scanned per expert (one wave
// per expert, lanes over chunks), experts are scanned into block offsets, and the pairs
// are scattered.  No step depends on atomic ordering, so the result is unique.
#include "capi_util.h"
#include "common.h"
#include "permute_dev.h"

namespace mxmoe {

constexpr int kBwThreads = 256;

// Calls f(e, a) for the nonzero affinities of row t handled by thread quarter q
// (four threads per row; 16-byte loads when E is a multiple of 4).
template <typename F>
__device__ __forceinline__ void for_row_quarter(const float* __restrict__ row, int E, int q, F f) {
  if ((E & 3) == 0) {
    const f32x4* r4 = reinterpret_cast<const f32x4*>(row);
    for (int i = q; i < E / 4; i += 4) {
      const f32x4 v = r4[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) f(4 * i + j, v[j]);
    }
  } else {
    for (int e = q; e < E; e += 4) f(e, row[e]);
  }
}

// Pass 1: per-chunk expert masks and counts, and the masked affinities; the workgroups
// also fill token_position_to_id with -1 (the scatter, two kernels later, writes the
// real slots).  counts are stored expert-major: counts[e * n_chunks + c].
__global__ void __launch_bounds__(kBwThreads) bw_count_kernel(
    const float* __restrict__ aff, const uint8_t* __restrict__ pmask, int T, int E,
    int n_chunks, float* __restrict__ aff_masked, int32_t* __restrict__ counts,
    unsigned long long* __restrict__ chunk_masks, int32_t* __restrict__ tp2id,
    int64_t n_slots) {
  extern __shared__ unsigned long long masks[];  // [E]
  const int tid = threadIdx.x, tl = tid >> 2, q = tid & 3, c = blockIdx.x;
  for (int64_t i = (int64_t)c * kBwThreads + tid; i < n_slots; i += (int64_t)n_chunks * kBwThreads)
    tp2id[i] = -1;
  for (int i = tid; i < E; i += kBwThreads) masks[i] = 0ull;
  __syncthreads();
  const int t = c * kChunkTok + tl;
  if (t < T) {
    const float* row = aff + (size_t)t * E;
    float* mrow = aff_masked + (size_t)t * E;
    const float pm = pmask ? (pmask[t] ? 1.0f : 0.0f) : 1.0f;
    for_row_quarter(row, E, q, [&](int e, float a) {
      mrow[e] = pmask ? a * pm : a;
      if (a != 0.0f) atomicOr(&masks[e], 1ull << tl);
    });
  }
  __syncthreads();
  for (int e = tid; e < E; e += kBwThreads) {
    const unsigned long long m = masks[e];
    counts[(size_t)e * n_chunks + c] = __popcll(m);
    chunk_masks[(size_t)c * E + e] = m;
  }
}

// Pass 2 (one workgroup of 1024 threads): per-expert exclusive prefix over chunks, block
// counts, block offsets, block_to_expert, conditions (bw_scan_body).
__global__ void __launch_bounds__(1024) bw_scan_kernel(
    int32_t* __restrict__ counts, int n_chunks, int E, int B, int N,
    int32_t* __restrict__ expert_pos, int32_t* __restrict__ block_to_expert,
    int32_t* __restrict__ conditions, int32_t* __restrict__ expert_counts) {
  __shared__ int cum[kMaxE], tot[kMaxE], wsum[16];
  bw_scan_body(counts, n_chunks, E, B, N, expert_pos, block_to_expert, conditions,
               expert_counts, cum, tot, wsum);
}

// Pass 3: scatter token ids.  token_position_to_id was filled with -1 by pass 1.
__global__ void __launch_bounds__(kBwThreads) bw_scatter_kernel(
    const float* __restrict__ aff, int T, int E, int n_chunks,
    const int32_t* __restrict__ prefix, const unsigned long long* __restrict__ chunk_masks,
    const int32_t* __restrict__ expert_pos, int32_t* __restrict__ tp2id, int64_t n_slots) {
  const int tid = threadIdx.x, tl = tid >> 2, q = tid & 3, c = blockIdx.x;
  const int t = c * kChunkTok + tl;
  if (t >= T) return;
  const unsigned long long below = (tl == 0) ? 0ull : (~0ull >> (64 - tl));
  for_row_quarter(aff + (size_t)t * E, E, q, [&](int e, float a) {
    if (a == 0.0f) return;
    const int rank = prefix[(size_t)e * n_chunks + c] +
                     __popcll(chunk_masks[(size_t)c * E + e] & below);
    const int64_t pos = (int64_t)expert_pos[e] + rank;
    if (pos < n_slots) tp2id[pos] = t;
  });
}

// Passes 2 and 3 in one launch for mappings whose chunk masks are few (every workgroup
// reads all of them): one workgroup of 1024 threads per chunk c, and one more (c =
// n_chunks) for the block tables.  Each reads every chunk mask and forms the per-expert
// totals (integer sums in LDS, so the atomics' order is free) and scans the experts' block
// counts into the first slot of each run, expert_pos[e], as bw_scan_body does.  A chunk's
// workgroup also sums pre[e], the expert's tokens in earlier chunks, keeps its own chunk's
// masks in LDS and writes its pairs: thread e walks the set bits of its expert's mask, the
// token of the r-th bit at slot expert_pos[e] + pre[e] + r, bw_scatter_kernel's slot.  The
// last workgroup writes block_to_expert, conditions and expert_counts as bw_scan_body.
constexpr int kPlaceMaxMasks = 32768;  // 256 KB of masks per workgroup at most
__global__ void __launch_bounds__(1024) bw_place_kernel(
    const unsigned long long* __restrict__ chunk_masks, int n_chunks, int E, int B, int N,
    int32_t* __restrict__ tp2id, int64_t n_slots, int32_t* __restrict__ block_to_expert,
    int32_t* __restrict__ conditions, int32_t* __restrict__ expert_counts) {
  __shared__ int tot[kMaxE], pre[kMaxE], cum[kMaxE], wsum[16];
  __shared__ unsigned long long own[kMaxE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = blockIdx.x;
  const bool place = c < n_chunks;
  for (int e = tid; e < E; e += 1024) tot[e] = pre[e] = 0;
  __syncthreads();
  const int nm = n_chunks * E;
  for (int i0 = 0; i0 < nm; i0 += 8 * 1024) {
    unsigned long long m[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * 1024 + tid;
      m[u] = i < nm ? chunk_masks[i] : 0ull;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * 1024 + tid;
      const int n = __popcll(m[u]);
      if (place && i / E == c) own[i % E] = m[u];
      if (n) {
        const int e = i % E;
        atomicAdd(&tot[e], n);
        if (i / E < c) atomicAdd(&pre[e], n);
      }
    }
  }
  __syncthreads();
  // Inclusive scan of the block counts over experts: wave scan, then across waves.
  const int e = tid;
  const int nb = e < E ? (tot[e] + B - 1) / B : 0;
  int v = nb;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(v, off);
    if (lane >= off) v += o;
  }
  if (lane == 63) wsum[wave] = v;
  __syncthreads();
  for (int w = 0; w < wave; ++w) v += wsum[w];
  if (e < E) cum[e] = v;
  __syncthreads();
  if (place) {
    if (e < E) {
      unsigned long long m = own[e];
      int64_t pos = (int64_t)(v - nb) * B + pre[e];
      while (m) {
        const int bit = __ffsll((long long)m) - 1;
        m &= m - 1;
        if (pos < n_slots) tp2id[pos] = c * kChunkTok + bit;
        ++pos;
      }
    }
    return;
  }
  if (e < E && expert_counts) expert_counts[e] = tot[e];
  const int used = cum[E - 1];
  for (int n = tid; n < N; n += 1024) {
    int lo = 0, hi = E - 1;  // #{e < E - 1 : n >= cum[e]} (cum is non-decreasing)
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (cum[mid] <= n) lo = mid + 1;
      else hi = mid;
    }
    block_to_expert[n] = lo;
    if (conditions) conditions[n] = n < used ? 1 : 0;
  }
}

}  // namespace mxmoe

using namespace mxmoe;

static size_t bw_ws(int64_t T, int64_t E) {
  const int64_t nch = (T + kChunkTok - 1) / kChunkTok;
  return align_up((size_t)(nch * E) * 4, 256) + align_up((size_t)(nch * E) * 8, 256) +
         align_up((size_t)E * 4, 256) + 256;
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
  const int64_t nb = blockwise_n_blocks(T, E, top_k, block_size);
  MXMOE_REQUIRE(n_blocks == nb, "blockwise_mapping: n_blocks=%lld, expected %lld",
                (long long)n_blocks, (long long)nb);
  if (workspace_bytes < bw_ws(T, E))
    return set_error(MXMOE_E_WORKSPACE, "blockwise_mapping: workspace %zu < %zu", workspace_bytes,
                     bw_ws(T, E));
  Carver cv(workspace, workspace_bytes);
  const int64_t nch = (T + kChunkTok - 1) / kChunkTok;
  int32_t* counts = cv.take<int32_t>(nch * E);
  unsigned long long* chunk_masks = cv.take<unsigned long long>(nch * E);
  int32_t* expert_pos = cv.take<int32_t>(E);
  hipStream_t s = as_stream(stream);
  const int64_t n_slots = n_blocks * block_size;
  const size_t lds = (size_t)E * sizeof(unsigned long long);
  hipLaunchKernelGGL(bw_count_kernel, dim3((unsigned)nch), dim3(kBwThreads), lds, s, affinities,
                     padding_mask, (int)T, (int)E, (int)nch, affinities_masked, counts,
                     chunk_masks, token_position_to_id, n_slots);
  if (nch * E <= kPlaceMaxMasks) {
    hipLaunchKernelGGL(bw_place_kernel, dim3((unsigned)nch + 1), dim3(1024), 0, s, chunk_masks,
                       (int)nch, (int)E, (int)block_size, (int)n_blocks, token_position_to_id,
                       n_slots, block_to_expert, conditions, expert_counts);
    return check_launch("blockwise_mapping");
  }
  hipLaunchKernelGGL(bw_scan_kernel, dim3(1), dim3(1024), 0, s, counts, (int)nch, (int)E,
                     (int)block_size, (int)n_blocks, expert_pos, block_to_expert, conditions,
                     expert_counts);
  hipLaunchKernelGGL(bw_scatter_kernel, dim3((unsigned)nch), dim3(kBwThreads), 0, s, affinities,
                     (int)T, (int)E, (int)nch, counts, chunk_masks, expert_pos,
                     token_position_to_id, n_slots);
  return check_launch("blockwise_mapping");
}
