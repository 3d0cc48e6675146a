"""CPU oracle of the DeepGenGraph attention hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only
as the checker (or the timed CPU baseline). The product (deepgengraph_amd) never imports it and has no
CPU fallback.

Each function restates the reference's PyTorch semantics on the CPU, citing the reference file:line it
follows (paths relative to the DeepGenGraph repository root):

  attention.attention      deepgengraph_exp/cases/kernels/attn.py:18-34, gemma2.py:19-38 (+ GQA roco.py:25-27,
                           + causal sliding window), LSE of the masked scaled fp32 scores
  attention.h2o            deepgengraph_exp/cases/kernels/h2o.py:18-38 (fp32 probability column sums)
  attention.decode         attn.py:18-34 with q_len == 1 (attn.py:22-23: no mask), cache layout [B, H, L, D]
  attention.decode_splitkv the split-KV + log-sum-exp merge restated in float64 (no reference counterpart;
                           pinned by equality with `decode`)
  selection.topk_indices   deepgengraph_exp/cases/models/h2o.py:51-52 (topk then index sort), ties -> lowest index
  elementwise.rms_norm     csrc/norm.cu:34-56 (twin: llama_base.py:282-285)
  elementwise.fused_add_rms_norm  csrc/norm.cu:59-83
  elementwise.silu_and_mul csrc/activation.cu:6-22
  elementwise.rotary_embedding_online  csrc/pos_encoding.cu:64-113, 180-199
  brute.*                  float64 pure-Python loops on tiny shapes: the independent pins of the above

How each function is pinned (tests/test_oracle.py): brute-force float64 loops on tiny shapes, closed forms and
invariants (rows of P sum to 1, sum_j colsum = q_len, rotary composition / norm preservation, split count
independence), and the committed golden vectors under tests/golden/.
"""
