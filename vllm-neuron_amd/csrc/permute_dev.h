// Device helpers of the blockwise mapping shared by the standalone mapping kernels
// (permute.hip) and the fused prefill front end (prefill_front.hip).
#pragma once

#include "common.h"

namespace mxmoe {

constexpr int kChunkTok = 64;  // tokens per chunk of the mapping (one 64-bit mask per expert)
constexpr int kMaxE = 1024;

// The scan step of the mapping, by one workgroup of 1024 threads: per-expert exclusive
// prefix over chunks (in place in counts, expert-major [e * n_chunks + c]; one wave per
// expert, lanes over chunks), per-expert totals into tot[] and block counts, their
// inclusive scan over experts into cum[] (LDS, kMaxE entries each), expert_pos[e] = first
// slot of expert e's run, block_to_expert[n] = #{e < E - 1 : n >= cum[e]}, and where not
// null conditions[n] (block inside the runs) and expert_counts[e].  Ends with a barrier.
__device__ inline void bw_scan_body(int32_t* __restrict__ counts, int n_chunks, int E, int B,
                                    int N, int32_t* __restrict__ expert_pos,
                                    int32_t* __restrict__ block_to_expert,
                                    int32_t* __restrict__ conditions,
                                    int32_t* __restrict__ expert_counts, int* cum, int* tot,
                                    int* wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Wave w scans experts w, w + 16, ...; EB of them at a time, their loads in flight
  // together.
  constexpr int EB = 8;
  for (int e0 = wave; e0 < E; e0 += 16 * EB) {
    int run[EB];
#pragma unroll
    for (int u = 0; u < EB; ++u) run[u] = 0;
    for (int c0 = 0; c0 < n_chunks; c0 += 64) {
      const int c = c0 + lane;
      int v[EB];
#pragma unroll
      for (int u = 0; u < EB; ++u) {
        const int e = e0 + 16 * u;
        v[u] = (e < E && c < n_chunks) ? counts[(size_t)e * n_chunks + c] : 0;
      }
#pragma unroll
      for (int u = 0; u < EB; ++u) {
        const int e = e0 + 16 * u;
        int x = v[u];
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int o = __shfl_up(x, off);
          if (lane >= off) x += o;
        }
        // exclusive prefix within the expert
        if (e < E && c < n_chunks) counts[(size_t)e * n_chunks + c] = run[u] + x - v[u];
        run[u] += __shfl(x, 63);
      }
    }
#pragma unroll
    for (int u = 0; u < EB; ++u)
      if (lane == 0 && e0 + 16 * u < E) tot[e0 + 16 * u] = run[u];
  }
  __syncthreads();
  const int e = tid;
  int nb = 0;
  if (e < E) {
    const int total = tot[e];
    nb = (total + B - 1) / B;
    if (expert_counts) expert_counts[e] = total;
  }
  // Inclusive block scan over experts: wave scan, then across waves.
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
  for (int n = tid; n < N; n += 1024) {
    // block_to_expert[n] = #{e < E-1 : n >= cum[e]}  (cum is non-decreasing)
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (cum[mid] <= n) lo = mid + 1;
      else hi = mid;
    }
    block_to_expert[n] = lo;
    // A block inside a run holds at least one token; blocks past the runs are empty.
    if (conditions) conditions[n] = n < used ? 1 : 0;
  }
  __syncthreads();
}

}  // namespace mxmoe
