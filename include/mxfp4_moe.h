/*
 * C-ABI of the MI355X (gfx950) MXFP4 mixture-of-experts expert path.
 *
 * One shared library (libmxmoe.so) with plain pointers, sizes and an explicit
 * HIP stream.  Every entry point returns 0 on success or a negative MXMOE_E_*
 * code; mxmoe_last_error() returns a message for the calling thread's last
 * failure.  No entry point allocates device memory: outputs and workspaces are
 * caller-allocated device buffers (sizes from the *_workspace_bytes queries).
 * The library keeps no mutable global state besides the per-thread error text,
 * so calls on different streams may run concurrently.
 *
 * Data conventions
 *   bf16       uint16_t bit patterns.
 *   MXFP4      OCP e2m1 codes, two per byte with the even element in the low
 *              nibble, one E8M0 scale byte (bias 127) per 32 elements along K.
 *   packed     weights in the row-group/chunk tile layout produced at load time
 *              by vllm_neuron_amd.weights.pack_mxfp4 (rows grouped by 16, K cut
 *              into 128-element chunks; see vllm-neuron_amd/csrc/common.h).
 *              Scales keep row groups four at a time (one 32-bit word per lane
 *              and chunk covers a quad).  A [N, K] matrix takes N*K/2 data
 *              bytes and ceil(N/64)*2K scale bytes.
 *              Fused gate_up matrices alternate 16-row groups of gate and up
 *              rows: [gate 0..15, up 0..15, gate 16..31, up 16..31, ...].
 *   clamps     float[4] = {gate_lo, gate_hi, up_lo, up_hi}; pass -INFINITY /
 *              +INFINITY for an absent limit.
 *   act        MXMOE_ACT_*; scale_mode MXMOE_SCALE_*.
 *
 * Shape limits checked by every entry point: K and N multiples of 32 and 16;
 * top_k <= 8; E <= 1024.
 */
#ifndef MXFP4_MOE_H_
#define MXFP4_MOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXMOE_OK 0
#define MXMOE_E_INVALID (-1)     /* bad shape / argument */
#define MXMOE_E_HIP (-2)         /* HIP runtime error */
#define MXMOE_E_WORKSPACE (-3)   /* workspace too small */
#define MXMOE_E_UNSUPPORTED (-4) /* valid but unsupported configuration */

#define MXMOE_ACT_SILU 0
#define MXMOE_ACT_GELU 1
#define MXMOE_ACT_SWISH 2 /* g * sigmoid(1.702 g) */

#define MXMOE_SCALE_POST 0    /* out += y * affinity */
#define MXMOE_SCALE_NO 1      /* out += y for selected experts */

#define MXMOE_ROUTER_SOFTMAX 0
#define MXMOE_ROUTER_SIGMOID 1


/* Library version (major*10000 + minor*100 + patch). */
int mxmoe_version(void);

/* Message for the calling thread's last failed call ("" if none). */
const char* mxmoe_last_error(void);

/*
 * MXFP4 -> bf16 dequantization, bit-exact with the reference loader.
 * Replaces: vllm_neuron/model/gpt_oss/weight_loaders_bf16.py:264-316
 * (_dequantize_mxfp4_to_bf16).  blocks [rows, K/32, 16], scales [rows, K/32]
 * (checkpoint layout) -> out bf16 [rows, K].
 */
int mxmoe_dequant_bf16(const uint8_t* blocks, const uint8_t* scales, uint16_t* out,
                       int64_t rows, int64_t K, void* stream);

/*
 * Weight-only MXFP4 linear: y[M, N] = bf16(x[M, K] . W[N, K]^T), fp32 accumulation,
 * W packed.  Replaces one expert projection of the MXFP4 path as the reference CPU
 * flow computes it: dequantize at load (weight_loaders_bf16.py:264-316), then the bf16
 * matmul with fp32 accumulation (vllm_neuron/functional/moe/moe_cte.py:536-537).
 */
int mxmoe_linear(const uint16_t* x, int64_t M, const uint8_t* wq, const uint8_t* ws,
                 int64_t N, int64_t K, uint16_t* y, void* stream);

/*
 * Router: logits = x . W^T (+ bias) in fp32, top-k, activation, scatter.
 * Replaces: vllm_neuron/functional/moe/router.py:690-796 (_nki_router_impl, the
 * nkilib router_topk call at :773-794) and the router stage of nkilib moe_block_tkg
 * (moe_block_tkg.py:474-512); semantics of the torch flows at router.py:383-565 and
 * moe_block_tkg.py:152-204.
 * x bf16 [T, H]; w bf16 [E, H] (the storage of router_weights[H, E] = W.T);
 * bias bf16 [E] or NULL.  act_before_topk = 0: top-k on logits, then the
 * activation over the k selected values; = 1: activation over all E logits, then
 * top-k.  renorm = 1 divides the k values by (their sum + renorm_eps).
 * Outputs: logits fp32 [T, E] (always written), affinities fp32 [T, E] (zeros except
 * the k selected), topk_idx int32 [T, k] and topk_val fp32 [T, k] (final values, in
 * descending order; equal values pick the lower expert id).
 */
size_t mxmoe_router_workspace_bytes(int64_t T, int64_t E);
int mxmoe_router_topk(const uint16_t* x, const uint16_t* w, const uint16_t* bias, int64_t T,
                      int64_t H, int64_t E, int top_k, int act, int act_before_topk, int renorm,
                      float renorm_eps, float* logits, float* affinities, int32_t* topk_idx,
                      float* topk_val, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Fused RMSNorm for the decode block: x_norm = bf16(gamma * x * rsqrt(mean(x[:h_actual]^2)
 * + eps)), columns >= h_actual set to 0.
 * Replaces the RMSNorm front-end of vllm_neuron/functional/moe/moe_block_tkg.py:134-150
 * (inside nkilib moe_block_tkg, called at :474-512).  x, out bf16 [T, H]; gamma fp32 [H].
 */
int mxmoe_rmsnorm(const uint16_t* x, const float* gamma, int64_t T, int64_t H, int64_t h_actual,
                  float eps, uint16_t* out, void* stream);

/*
 * Blockwise token -> expert mapping, bit-exact with the reference torch flow.
 * Replaces: vllm_neuron/functional/moe/moe_blockwise.py:159-291 (nkilib
 * find_nonzero_indices + indexed_flatten) with the semantics of :294-400.
 * affinities fp32 [T, E]; padding_mask uint8 [T] or NULL (1 = real token).
 * n_blocks must equal the reference bound (moe_blockwise.py:343-349).
 * Outputs: affinities_masked fp32 [T*E], token_position_to_id int32 [n_blocks*B],
 * block_to_expert int32 [n_blocks], conditions int32 [n_blocks],
 * expert_counts int32 [E] (tokens per expert; may be NULL).
 */
size_t mxmoe_blockwise_workspace_bytes(int64_t T, int64_t E);
int mxmoe_blockwise_mapping(const float* affinities, const uint8_t* padding_mask, int64_t T,
                            int64_t E, int top_k, int64_t block_size, int64_t n_blocks,
                            float* affinities_masked, int32_t* token_position_to_id,
                            int32_t* block_to_expert, int32_t* conditions,
                            int32_t* expert_counts, void* workspace, size_t workspace_bytes,
                            void* stream);

/*
 * Prefill expert MLP over the blockwise mapping (grouped gate_up GEMM with fused
 * MXFP4 dequant, bias, clamps, activation; down GEMM with bias; affinity-weighted
 * combine in ascending expert order).  bf16 intermediates as in the reference.
 * Replaces: vllm_neuron/functional/moe/moe_cte.py:650-732 (_torch_compatible_moe_cte_kernel
 * -> nkilib moe_cte shard_on_block_mx); semantics of the torch flow at :448-581.
 * x bf16 [>=T, H]; affinities_masked fp32 [T*E]; gu_q/gu_s packed [E][2I x H];
 * dn_q/dn_s packed [E][H x I]; gu_bias bf16 [E, 2, I] or NULL; dn_bias bf16 [E, H]
 * or NULL; out [T, H] in bf16, or fp32 when out_f32 = 1 (the dtype of the reference
 * torch flow's result).  stage_events: NULL, or 4 hipEvent_t recorded on the stream
 * before the gate_up GEMM, after it, after the down GEMM and after the combine.
 */
size_t mxmoe_moe_cte_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                                     int64_t block_size, int64_t n_blocks);
int mxmoe_moe_cte(const uint16_t* x, const float* affinities_masked, const uint8_t* gu_q,
                  const uint8_t* gu_s, const uint8_t* dn_q, const uint8_t* dn_s,
                  const uint16_t* gu_bias, const uint16_t* dn_bias,
                  const int32_t* token_position_to_id, const int32_t* block_to_expert,
                  int64_t n_blocks, int64_t block_size, int64_t T, int64_t H, int64_t I,
                  int64_t E, int act, const float* clamps, int scale_mode, int out_f32,
                  void* out, void* workspace, size_t workspace_bytes, void* const* stage_events,
                  void* stream);

/*
 * Decode expert MLP given routing: weight-streaming grouped GEMMs over the selected
 * experts only, fp32 intermediates (the down GEMM consumes a hi/lo bf16 split of
 * the fp32 activations), ascending-expert fp32 combine, bf16 output.
 * Replaces: vllm_neuron/functional/moe/moe_tkg.py:157-190 (moe_tkg_wrapper -> nkilib
 * moe_tkg) and the expert part of moe_block_tkg (moe_block_tkg.py:474-512); semantics
 * of the torch flow at moe_block_tkg.py:223-297.
 * x bf16 [T, H]; topk_idx int32 [T, k]; topk_val fp32 [T, k] (the affinity of each
 * selected expert); expert ids outside [0, E) are skipped (expert parallelism).
 * stage_events: NULL, or 5 hipEvent_t recorded on the stream before the routing
 * kernel, after it, after the gate_up kernel, after the down kernel, after the combine.
 */
size_t mxmoe_moe_tkg_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int top_k);
int mxmoe_moe_tkg(const uint16_t* x, const int32_t* topk_idx, const float* topk_val,
                  const uint8_t* gu_q, const uint8_t* gu_s, const uint8_t* dn_q,
                  const uint8_t* dn_s, const uint16_t* gu_bias, const uint16_t* dn_bias,
                  int64_t T, int64_t H, int64_t I, int64_t E, int top_k, int act,
                  const float* clamps, int scale_mode, uint16_t* out, void* workspace,
                  size_t workspace_bytes, void* const* stage_events, void* stream);

/*
 * Whole decode expert layer in one call: router (as mxmoe_router_topk) on x, then the
 * mxmoe_moe_tkg pipeline on the selected experts.  The counterpart of the router +
 * expert stages of nkilib moe_block_tkg (vllm_neuron/functional/moe/moe_block_tkg.py:474-512)
 * for an already-normalized input; semantics of moe_block_tkg.py:152-297.
 * router_w bf16 [E, H], router_b bf16 [E] or NULL; logits_out fp32 [T, E] or NULL.
 * stage_events: NULL, or 6 hipEvent_t recorded before the router and after the router,
 * routing, gate_up, down and combine kernels.  For T <= 16 one kernel takes the top-k
 * and routes the batch: the events after the router and after routing then both follow
 * it (routing shows no time of its own).
 */
size_t mxmoe_moe_decode_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int top_k);
int mxmoe_moe_decode(const uint16_t* x, const uint16_t* router_w, const uint16_t* router_b,
                     int router_act, int act_before_topk, int renorm, float renorm_eps,
                     const uint8_t* gu_q, const uint8_t* gu_s, const uint8_t* dn_q,
                     const uint8_t* dn_s, const uint16_t* gu_bias, const uint16_t* dn_bias,
                     int64_t T, int64_t H, int64_t I, int64_t E, int top_k, int act,
                     const float* clamps, int scale_mode, uint16_t* out, float* logits_out,
                     void* workspace, size_t workspace_bytes, void* const* stage_events,
                     void* stream);

/*
 * The decode MoE block in one call: RMSNorm (as mxmoe_rmsnorm: variance over the first
 * h_actual columns, bf16 result, columns past h_actual zero) into the workspace, then
 * mxmoe_moe_decode on the normalized rows.  Replaces the RMSNorm + router + expert
 * stages of nkilib moe_block_tkg (vllm_neuron/functional/moe/moe_block_tkg.py:474-512;
 * semantics of :134-297) for one expert-parallel rank holding every expert.
 * x bf16 [T, H] (not normalized); gamma fp32 [H]; the rest as mxmoe_moe_decode.
 * stage_events: NULL, or 7 hipEvent_t: before the RMSNorm, then the 6 of
 * mxmoe_moe_decode.
 */
size_t mxmoe_moe_block_decode_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                                              int top_k);
int mxmoe_moe_block_decode(const uint16_t* x, const float* gamma, int64_t h_actual, float eps,
                           const uint16_t* router_w, const uint16_t* router_b, int router_act,
                           int act_before_topk, int renorm, float renorm_eps, const uint8_t* gu_q,
                           const uint8_t* gu_s, const uint8_t* dn_q, const uint8_t* dn_s,
                           const uint16_t* gu_bias, const uint16_t* dn_bias, int64_t T, int64_t H,
                           int64_t I, int64_t E, int top_k, int act, const float* clamps,
                           int scale_mode, uint16_t* out, float* logits_out, void* workspace,
                           size_t workspace_bytes, void* const* stage_events, void* stream);

/*
 * Diagnostics (no counterpart in the reference): they pin the hardware behaviour
 * the kernels rely on.  mxmoe_probe_hw_dequant runs the CDNA4 scaled fp4->bf16
 * conversion the GEMMs use over blocks/scales like mxmoe_dequant_bf16;
 * mxmoe_probe_mfma multiplies A bf16 [16, 32] by B^T (B bf16 [16, 32]) with one
 * v_mfma_f32_16x16x32_bf16 using the library's operand convention -> D fp32 [16, 16].
 */
int mxmoe_probe_hw_dequant(const uint8_t* blocks, const uint8_t* scales, uint16_t* out,
                           int64_t rows, int64_t K, void* stream);
int mxmoe_probe_mfma(const uint16_t* a, const uint16_t* b, float* d, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MXFP4_MOE_H_ */
