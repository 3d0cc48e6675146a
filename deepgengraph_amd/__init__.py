"""deepgengraph_amd: the DeepGenGraph (FlashTensor) attention hot path, hand-written for MI355X (gfx950).

  deepgengraph_amd.ops        csrc-compatible rms_norm / fused_add_rms_norm / silu_and_mul / rotary_embedding_online
  deepgengraph_amd.attention  prefill attention (causal / soft-cap / window / GQA), H2O column sums + top-k,
                              split-KV decode
  deepgengraph_amd.compile    compile(model, input_names, inputs, output_names, system='mi355x') -> f(*inputs)
  deepgengraph_amd.llama      the Llama-2 attention block (config 2) and decode pre-step (config 5) on these ops
  deepgengraph_amd.configs    the five benchmark configurations as seeded input builders
  deepgengraph_amd.cases      the reference's attention case modules (Attn, Gemma2, H2O, RoCo, SnapKV, Corm, KeyFormer)
  deepgengraph_amd.run_kernel the per-case harness (run_kernel.py's CLI and perf line)
  deepgengraph_amd.run_e2e    the end-to-end harness: random-weight Llama-2-7B with each case's KV-cache selection

All GPU work runs in libdgg_hip.so (C ABI: include/dgg.h), loaded with ctypes; there is no CPU fallback.
"""
from . import _lib  # noqa: F401

_csrc = None  # set below: module alias matching the reference's `asuka_exp._csrc` (setup.py:41)

from . import ops  # noqa: E402

_csrc = ops

__all__ = ["ops", "attention", "compile", "configs", "llama"]
