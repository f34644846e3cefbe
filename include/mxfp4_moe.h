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

#define MXMOE_SCALE_POST 0         /* out += y * affinity */
#define MXMOE_SCALE_NO 1           /* out += y for selected experts */
#define MXMOE_SCALE_PRE 2          /* moe_cte: x * affinity before gate_up, bf16 sum of all experts */
#define MXMOE_SCALE_PRE_DELAYED 3  /* moe_cte: act(g) * u * affinity before down, bf16 sum */

#define MXMOE_ROUTER_SOFTMAX 0
#define MXMOE_ROUTER_SIGMOID 1

/* Element types (dtype arguments). */
#define MXMOE_DT_F32 0
#define MXMOE_DT_F16 1
#define MXMOE_DT_BF16 2

/* Expert weight formats (weight_fmt arguments), both in this library's packed layout with
 * E8M0 scales per 32 elements along K: MXFP4 (e2m1 pairs, [rows/16, 8K] bytes) and MXFP8
 * (E4M3FN, [rows/16, 16K] bytes); the scales are packed alike ([ceil(rows/64), 2K]). */
#define MXMOE_WFMT_MXFP4 0
#define MXMOE_WFMT_MXFP8 1
/* bf16 expert weights as the reference's shard_on_block takes them (moe_cte.py:117-124):
 * gate_up [E, H, 2, I] and down [E, I, H], rows along K, no scales (mxmoe_moe_cte only). */
#define MXMOE_WFMT_BF16 2


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
 * MXFP8 -> bf16: element = E4M3FN(code) x 2^(scale - 127), one rounding to bf16, scale byte
 * 255 and the NaN codes -> NaN (the OCP MX definition; the reference names MXFP8 weights
 * for moe_cte's MX kernel, moe_cte.py:136-138, with no CPU flow to follow).  codes
 * [rows, K/32, 32] uint8, scales [rows, K/32] -> out bf16 [rows, K].
 */
int mxmoe_dequant_mxfp8_bf16(const uint8_t* codes, const uint8_t* scales, uint16_t* out,
                             int64_t rows, int64_t K, void* stream);

/*
 * Weight-only MX linear: y[M, N] = bf16(x[M, K] . W[N, K]^T), fp32 accumulation, W packed
 * in weight_fmt (MXMOE_WFMT_*).  Replaces one expert projection of the MX path as the
 * reference CPU flow computes it: dequantize at load (weight_loaders_bf16.py:264-316), then
 * the bf16 matmul with fp32 accumulation (vllm_neuron/functional/moe/moe_cte.py:536-537).
 */
int mxmoe_linear(const uint16_t* x, int64_t M, const uint8_t* wq, const uint8_t* ws,
                 int weight_fmt, int64_t N, int64_t K, uint16_t* y, void* stream);

/*
 * Router: logits = x . W^T (+ bias), top-k, activation, scatter.
 * Replaces: vllm_neuron/functional/moe/router.py:690-796 (_nki_router_impl, the
 * nkilib router_topk call at :773-794); semantics of the torch flows at router.py:383-565,
 * computed as torch computes them in compute_dtype (router.py:422-426):
 *   MXMOE_DT_F32   the operands and products exactly as in an fp32 matmul (x bf16; W bf16
 *                  or fp16, fp16 weights split exactly into two bf16 operands), fp32 logits
 *                  and activations;
 *   MXMOE_DT_F16   x and W cast to fp16, fp16 products summed in fp32, the bias cast to fp16
 *                  and added in fp32, the logit rounded to fp16 once; every activation
 *                  output, renorm sum and quotient rounded to fp16 (one rounding per op);
 *   MXMOE_DT_BF16  the same with bf16.
 * x [T, H] (x_dtype bf16, or fp16 with compute_dtype fp16); w [E, H] (the storage of
 * router_weights[H, E] = W.T; w_dtype bf16 or fp16); bias [E] (bias_dtype any) or NULL.
 * act_before_topk = 0: top-k on logits, then the activation over the k selected values;
 * = 1: activation over all E logits, then top-k.  renorm = 1 divides the k values by
 * (their sum + renorm_eps).
 * Outputs: logits fp32 [T, E] (always written; values of compute_dtype), affinities fp32
 * [T, E] (zeros except the k selected), topk_idx int32 [T, k] and topk_val fp32 [T, k]
 * (final values, in descending order; equal values pick the lower expert id).
 */
size_t mxmoe_router_workspace_bytes(int64_t T, int64_t E);
int mxmoe_router_topk(const void* x, int x_dtype, const void* w, int w_dtype, const void* bias,
                      int bias_dtype, int64_t T, int64_t H, int64_t E, int top_k, int act,
                      int act_before_topk, int renorm, float renorm_eps, int compute_dtype,
                      float* logits, float* affinities, int32_t* topk_idx, float* topk_val,
                      void* workspace, size_t workspace_bytes, void* stream);

/*
 * RMSNorm of bf16 rows: out = gamma * (x * inv), inv = 1 / sqrt(ss / h_actual + eps), fp32
 * arithmetic, rounded to out_dtype (MXMOE_DT_BF16 or MXMOE_DT_F16).
 *   all_cols = 0: ss sums x^2 over the first h_actual columns and columns >= h_actual
 *                 are written as 0 (vllm_neuron/functional/moe/moe_block_tkg.py:134-150,
 *                 the RMSNorm front end of nkilib moe_block_tkg called at :474-512);
 *   all_cols = 1: ss sums x^2 over all H columns and every column is normalized
 *                 (rmsnorm_router_topk_tkg.py:249-257; router.py:680-687 with h_actual = H).
 * x [T, H] bf16; gamma fp32 [H]; out [T, H].
 */
int mxmoe_rmsnorm(const uint16_t* x, const float* gamma, int64_t T, int64_t H, int64_t h_actual,
                  int all_cols, float eps, int out_dtype, uint16_t* out, void* stream);

/*
 * Fused RMSNorm + router top-k of the decode front end, quantization NONE.
 * Replaces: vllm_neuron/functional/moe/rmsnorm_router_topk_tkg.py:33-45 (the nkilib
 * kernel behind it); semantics of its torch flow at :214-279: the RMSNorm as
 * mxmoe_rmsnorm with all_cols = 1, rounded to mm_dtype (MXMOE_DT_F16 or MXMOE_DT_BF16)
 * into norm_out [T, H]; logits = norm . cast(W, mm_dtype) in fp32 + cast(bias, mm_dtype);
 * top-k on the fp32 logits, the activation over the k selected values (fp32), scattered
 * into affinities [T, E] bf16 (zeros elsewhere); topk_idx int32 [T, k].
 * router_w [E, H] (w_dtype bf16 or fp16), router_b [E] (b_dtype any) or NULL.
 */
size_t mxmoe_rmsnorm_router_topk_workspace_bytes(int64_t T, int64_t E, int top_k);
int mxmoe_rmsnorm_router_topk(const uint16_t* x, const float* gamma, int64_t h_actual, float eps,
                              const void* router_w, int w_dtype, const void* router_b,
                              int b_dtype, int64_t T, int64_t H, int64_t E, int top_k, int act,
                              int mm_dtype, uint16_t* norm_out, int32_t* topk_idx,
                              uint16_t* affinities, void* workspace, size_t workspace_bytes,
                              void* stream);

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
 * MXFP4 dequant, bias, clamps, activation; down GEMM with bias; combine).  bf16
 * intermediates as in the reference.
 * Replaces: vllm_neuron/functional/moe/moe_cte.py:650-732 (_torch_compatible_moe_cte_kernel
 * -> nkilib moe_cte shard_on_block_mx); semantics of the torch flow at :448-581.
 * x bf16 [>=T, H]; affinities_masked fp32 [T*E]; gu_q/gu_s packed [E][2I x H];
 * dn_q/dn_s packed [E][H x I], both in weight_fmt (MXMOE_WFMT_MXFP4, or MXMOE_WFMT_MXFP8:
 * the MxFP8 weights of the reference's shard_on_block_mx kernel, moe_cte.py:136-138);
 * with MXMOE_WFMT_BF16, gu_q is bf16 [E, H, 2, I] and dn_q bf16 [E, I, H] (the
 * shard_on_block operands of the bf16 model, model_bf16.py:1360-1391; 16-byte aligned)
 * and gu_s / dn_s are ignored (may be NULL);
 * gu_bias bf16 [E, 2, I] or NULL; dn_bias bf16 [E, H] or NULL; out [T, H] in bf16, or
 * fp32 when out_f32 = 1.
 * scale_mode:
 *   MXMOE_SCALE_POST         out = sum of y * affinity over the routed experts, in
 *                            ascending expert order, fp32 (:572-575);
 *   MXMOE_SCALE_PRE          gate_up on bf16(x * affinity) (:518-520);
 *   MXMOE_SCALE_PRE_DELAYED  the activation times bf16 affinity before the down GEMM
 *                            (:556-558);
 *   for both pre-scaling modes the affinity is taken as bf16 and out is the bf16 running
 *   sum over ALL E experts in ascending order (:576-579): a routed expert adds its y, any
 *   other expert expert_const[e] (bf16 [E, H]: its output for a zero input, i.e. the down
 *   bias under PRE_SCALE_DELAYED and y_e(0) under PRE_SCALE; NULL adds nothing).
 * stage_events: NULL, or 4 hipEvent_t recorded on the stream before the gate_up GEMM,
 * after it, after the down GEMM and after the combine.
 */
size_t mxmoe_moe_cte_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                                     int64_t block_size, int64_t n_blocks, int scale_mode);
int mxmoe_moe_cte(const uint16_t* x, const float* affinities_masked, const uint8_t* gu_q,
                  const uint8_t* gu_s, const uint8_t* dn_q, const uint8_t* dn_s, int weight_fmt,
                  const uint16_t* gu_bias, const uint16_t* dn_bias, const uint16_t* expert_const,
                  const int32_t* token_position_to_id, const int32_t* block_to_expert,
                  int64_t n_blocks, int64_t block_size, int64_t T, int64_t H, int64_t I,
                  int64_t E, int act, const float* clamps, int scale_mode, int out_f32,
                  void* out, void* workspace, size_t workspace_bytes, void* const* stage_events,
                  void* stream);

/*
 * Whole prefill expert layer in one call: router on x, blockwise mapping (block_size),
 * then the mxmoe_moe_cte pipeline with POST_SCALE.  The counterpart of the call sequence
 * of the GPT-OSS MXFP4 prefill layer, vllm_neuron/model/gpt_oss/model_mxfp4.py:1337-1433
 * (NF.router -> NF.build_blockwise_mapping -> NF.moe_cte shard_on_block_mx, skip_token)
 * for an already-normalized input on one rank holding every expert.
 * Router arguments as mxmoe_router_topk (router_compute_dtype is its compute_dtype;
 * x is bf16); the logits are bit-identical to its.  padding_mask uint8 [T] or NULL as
 * mxmoe_blockwise_mapping; the mapping equals its result.  Weights, biases, act,
 * clamps, out_f32 and out as mxmoe_moe_cte (weight_fmt MXMOE_WFMT_MXFP4 or
 * MXMOE_WFMT_MXFP8).
 * stage_events: NULL, or 5 hipEvent_t recorded before the router, after the mapping
 * (before the gate_up GEMM), after the gate_up GEMM, after the down GEMM and after the
 * combine.
 */
size_t mxmoe_moe_prefill_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int top_k,
                                         int64_t block_size);
int mxmoe_moe_prefill(const uint16_t* x, const void* router_w, int router_w_dtype,
                      const void* router_b, int router_b_dtype, int router_act,
                      int act_before_topk, int renorm, float renorm_eps, int router_compute_dtype,
                      const uint8_t* padding_mask, const uint8_t* gu_q, const uint8_t* gu_s,
                      const uint8_t* dn_q, const uint8_t* dn_s, int weight_fmt,
                      const uint16_t* gu_bias, const uint16_t* dn_bias, int64_t T, int64_t H,
                      int64_t I, int64_t E, int top_k, int64_t block_size, int act,
                      const float* clamps, int out_f32, void* out, void* workspace,
                      size_t workspace_bytes, void* const* stage_events, void* stream);

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
 * mxmoe_moe_tkg for bf16 expert weights: the decode flow of the reference's torch path
 * (moe_block_tkg.py:223-297; the bf16 GPT-OSS model's decode call, model_bf16.py:
 * 1199-1252, passes bf16 weights [E_L, H, 2, I] and [E_L, I, H]) with fp32 intermediates
 * (h carried as an exact-to-16-bits bf16 pair into the down GEMM) and the ascending-expert
 * fp32 combine, bf16 output.  The selected experts are mapped blockwise (block 128) and
 * run the MFMA GEMMs of the bf16 moe_cte path.
 * Replaces: the nkilib moe_block_tkg / moe_tkg kernels for bf16 weights
 * (moe_block_tkg.py:474-512, moe_tkg.py:157-190).
 * x bf16 [T, H]; topk_idx int32 [T, k]; topk_val fp32 [T, k]; expert ids outside [0, E)
 * are skipped; gu_w bf16 [E, H, 2, I], dn_w bf16 [E, I, H] (16-byte aligned); gu_bias
 * bf16 [E, 2, I] or NULL, dn_bias bf16 [E, H] or NULL; scale_mode MXMOE_SCALE_POST or
 * MXMOE_SCALE_NO.
 */
size_t mxmoe_moe_tkg_bf16_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                                          int top_k);
int mxmoe_moe_tkg_bf16(const uint16_t* x, const int32_t* topk_idx, const float* topk_val,
                       const uint16_t* gu_w, const uint16_t* dn_w, const uint16_t* gu_bias,
                       const uint16_t* dn_bias, int64_t T, int64_t H, int64_t I, int64_t E,
                       int top_k, int act, const float* clamps, int scale_mode, uint16_t* out,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * Whole decode expert layer in one call: router on x, then the mxmoe_moe_tkg pipeline on
 * the selected experts.  The counterpart of the router + expert stages of nkilib
 * moe_block_tkg (vllm_neuron/functional/moe/moe_block_tkg.py:474-512) for an
 * already-normalized input; semantics of moe_block_tkg.py:152-297: fp32 router logits
 * (router_w [E, H] bf16 or fp16 by router_w_dtype, every product exact; router_b [E] of
 * router_b_dtype or NULL), then the fp32 expert math.
 * logits_out fp32 [T, E] or NULL; topk_idx_out int32 [T, k] or NULL (the experts the
 * front end selected per token, descending score, equal scores -> lower id).
 * stage_events: NULL, or 6 hipEvent_t recorded before the router and after the router,
 * routing, gate_up, down and combine kernels.  For T <= 16 one kernel takes the top-k
 * and routes the batch: the events after the router and after routing then both follow
 * it (routing shows no time of its own).
 */
size_t mxmoe_moe_decode_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int top_k);
int mxmoe_moe_decode(const uint16_t* x, const void* router_w, int router_w_dtype,
                     const void* router_b, int router_b_dtype, int router_act,
                     int act_before_topk, int renorm, float renorm_eps, const uint8_t* gu_q,
                     const uint8_t* gu_s, const uint8_t* dn_q, const uint8_t* dn_s,
                     const uint16_t* gu_bias, const uint16_t* dn_bias, int64_t T, int64_t H,
                     int64_t I, int64_t E, int top_k, int act, const float* clamps,
                     int scale_mode, uint16_t* out, float* logits_out, int32_t* topk_idx_out,
                     void* workspace, size_t workspace_bytes, void* const* stage_events,
                     void* stream);

/*
 * The decode MoE block in one call: RMSNorm (as mxmoe_rmsnorm with all_cols = 0 and a bf16
 * result) into the workspace, then mxmoe_moe_decode on the normalized rows.  Replaces the
 * RMSNorm + router + expert stages of nkilib moe_block_tkg
 * (vllm_neuron/functional/moe/moe_block_tkg.py:474-512; semantics of :134-297) for one
 * expert-parallel rank holding every expert.
 * x bf16 [T, H] (not normalized); gamma fp32 [H]; the rest as mxmoe_moe_decode.
 * stage_events: NULL, or 7 hipEvent_t: before the RMSNorm, then the 6 of
 * mxmoe_moe_decode.
 */
size_t mxmoe_moe_block_decode_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                                              int top_k);
int mxmoe_moe_block_decode(const uint16_t* x, const float* gamma, int64_t h_actual, float eps,
                           const void* router_w, int router_w_dtype, const void* router_b,
                           int router_b_dtype, int router_act, int act_before_topk, int renorm,
                           float renorm_eps, const uint8_t* gu_q, const uint8_t* gu_s,
                           const uint8_t* dn_q, const uint8_t* dn_s, const uint16_t* gu_bias,
                           const uint16_t* dn_bias, int64_t T, int64_t H, int64_t I, int64_t E,
                           int top_k, int act, const float* clamps, int scale_mode,
                           uint16_t* out, float* logits_out, int32_t* topk_idx_out,
                           void* workspace, size_t workspace_bytes, void* const* stage_events,
                           void* stream);

/*
 * mxmoe_moe_block_decode without allocation or workspace argument.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation).  The workspace
 * is a device array of MXMOE_NOALLOC_SCRATCH_BYTES in the library, one per GPU, held
 * until the process ends; shapes whose mxmoe_moe_block_decode_workspace_bytes exceed it
 * fail with MXMOE_E_WORKSPACE (GPT-OSS-120B at 64 tokens needs about 15 MiB, E=256,
 * top-8, H=7168, I=2048 at 128 tokens about 38 MiB).  The calling thread's current device must
 * be the stream's.  Calls that overlap on one GPU share the array and race: serialize
 * them (one stream, or events).  Arguments and results as mxmoe_moe_block_decode.
 */
#define MXMOE_NOALLOC_SCRATCH_BYTES (48u << 20)
int mxmoe_moe_block_decode_noalloc(const uint16_t* x, const float* gamma, int64_t h_actual,
                                   float eps, const void* router_w, int router_w_dtype,
                                   const void* router_b, int router_b_dtype, int router_act,
                                   int act_before_topk, int renorm, float renorm_eps,
                                   const uint8_t* gu_q, const uint8_t* gu_s, const uint8_t* dn_q,
                                   const uint8_t* dn_s, const uint16_t* gu_bias,
                                   const uint16_t* dn_bias, int64_t T, int64_t H, int64_t I,
                                   int64_t E, int top_k, int act, const float* clamps,
                                   int scale_mode, uint16_t* out, float* logits_out,
                                   int32_t* topk_idx_out, void* const* stage_events,
                                   void* stream);

/*
 * Diagnostics (no counterpart in the reference): they pin the hardware behaviour
 * the kernels rely on.  mxmoe_probe_hw_dequant runs the CDNA4 scaled fp4->bf16
 * conversion the GEMMs use over blocks/scales like mxmoe_dequant_bf16, and
 * mxmoe_probe_hw_dequant_fp8 the scaled fp8->bf16 one like mxmoe_dequant_mxfp8_bf16;
 * mxmoe_probe_mfma multiplies A bf16 [16, 32] by B^T (B bf16 [16, 32]) with one
 * v_mfma_f32_16x16x32_bf16 using the library's operand convention -> D fp32 [16, 16].
 */
int mxmoe_probe_hw_dequant(const uint8_t* blocks, const uint8_t* scales, uint16_t* out,
                           int64_t rows, int64_t K, void* stream);
int mxmoe_probe_hw_dequant_fp8(const uint8_t* codes, const uint8_t* scales, uint16_t* out,
                               int64_t rows, int64_t K, void* stream);
int mxmoe_probe_mfma(const uint16_t* a, const uint16_t* b, float* d, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MXFP4_MOE_H_ */
