"""CPU oracle -- TEST INFRASTRUCTURE ONLY.

A restatement, on the CPU, of what the reference computes on its hot path:

* ``oracle.ops``               -- the fused ops in fp32 eager torch on CPU
                                  (the reference's own torch programs, restated)
* ``oracle.reference_configs`` -- the reference's candidate config grids and
                                  descriptor score adjustments (for A100 parity
                                  of the restated cost model)

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this package, and only as the checker / baseline.  The product
(``icpp_tuning_amd``) never imports it and has no CPU fallback.

Parity pins (each function is checked by tests/test_oracle.py against something
independent of its own formula):
  gemm_ref, gemm_bias_act_ref   fp64 numpy triple loop on tiny shapes; identity
                                and zero operands; torch.nn.functional
                                activations (relu, gelu(approximate="tanh"), silu)
  gemm_bias_layernorm_ref       fp64 numpy two-pass LN; constant rows -> beta;
                                torch.nn.functional.layer_norm
  conv2d_nhwc_ref               7-loop fp64 direct convolution (checks the
                                k -> (kh, kw, c) map of conv2d.py:242-250)
  fp8_gemm_bias_act_ref         exact fp8 e4m3 decode table from the OCP spec
                                (sign/exponent/mantissa bit arithmetic)
  conv2d_bn_act_ref             torch batch_norm (eval), fp64 loops, identity /
                                residual / var-clamp special cases
  layernorm_fwd_ref / _bwd_ref  F.layer_norm, autograd, constant rows
  softmax_ref, softmax_scaled_masked_ref
                                torch.softmax, row-sum / shift invariants
  qkv_split_heads_ref, merge_heads_ref
                                explicit index loops over (batch, head, seq, d)
  attention_ref                 fp64 scaled_dot_product_attention with the additive
                                causal mask, and fp64 loops per (batch, head)
  bert_layer_ref                an fp64 SDPA / layer_norm / gelu composition
  reference_configs             evaluation CSV top-1 configs and scores
                                (tests/golden/formula_scores.json)
"""
