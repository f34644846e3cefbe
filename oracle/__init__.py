"""CPU oracle for the MXFP4 mixture-of-experts expert path.

TEST INFRASTRUCTURE ONLY.  This package restates, on the CPU with PyTorch, the
reference's own CPU implementation of the MXFP4 MoE path (vllm-neuron, CPU mode):

  * MXFP4 -> bf16 dequantization and the gate/up/down loaders
    (vllm_neuron/model/gpt_oss/weight_loaders_bf16.py:264-488)       -> oracle.mxfp4
  * router: linear -> top-k -> activation -> scatter
    (vllm_neuron/functional/moe/router.py:300-598)                    -> oracle.router
  * build_blockwise_mapping, torch flow
    (vllm_neuron/functional/moe/moe_blockwise.py:24-156,294-461)      -> oracle.blockwise
  * moe_cte torch fallback `_torch_moe_impl` (prefill)
    (vllm_neuron/functional/moe/moe_cte.py:423-581)                   -> oracle.moe_cte
  * moe_block_tkg torch fallback `_torch_moe_block_tkg_impl` (decode)
    (vllm_neuron/functional/moe/moe_block_tkg.py:56-302)              -> oracle.moe_block_tkg
  * the GPT-OSS expert-layer orchestration of those calls
    (vllm_neuron/model/gpt_oss/model_bf16.py:1199-1413)               -> oracle.layer
  * the load-time transform into the Trainium kernel layout (one rank)
    (vllm_neuron/model/gpt_oss/weight_loaders_mxfp4.py:243-885)       -> oracle.neuron_layout

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the reference the GPU results
are compared with (or, for the baseline, as the timed CPU path).  The product
package never imports it; its functional API raises when the HIP extension is
missing instead of falling back to anything here.

Pinning (what each function is checked against, besides the reference text it
follows) is listed in each module's docstring; the tests under ``tests/``
named ``test_oracle_*`` hold those checks.
"""
