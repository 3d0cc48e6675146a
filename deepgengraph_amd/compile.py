"""The reference's system dispatcher with an MI355X system.

compile(model, input_names, inputs, output_names, system) -> f(*inputs) keeps the signature and contract of the
reference's compile.py:6-296: `model` is one of the attention case modules (Attn, Gemma2, H2O, RoCo, SnapKV, Corm, KeyFormer
from deepgengraph_exp/cases/kernels/), `f` takes the same positional inputs (q, k, v in [B, S, H, D], plus
corm_mask for Corm and exp_rand for KeyFormer) and returns what the module's forward returns (out; (out, h2o_score)
for H2O; (out, roco_score, roco_sq_score) for RoCo; (out, snapkv_score) for SnapKV; (out, corm_score) for Corm;
(out, kf_score) for KeyFormer).
run_kernel.py:72 and run_e2e.py:217 call it this way.

Systems:
  'torch'           the module itself (compile.py:7-8)
  'mi355x' / 'our'  the hand-written gfx950 kernels of libdgg_hip.so ('our' is the reference's name for the
                    FlashTensor-generated kernels this path replaces, compile.py:44)
Other reference systems (tensorrt, tvm, xla, dynamo, flashinfer, flashattn) are baselines that are not part of
this build and raise NotImplementedError, as the reference does for an unknown system (compile.py:293-294).
"""
from __future__ import annotations

import math

from . import attention as _attn

SYSTEMS = ("torch", "mi355x", "our")


def _attn_f(model):
    name = model.__class__.__name__
    head_dim = int(model.head_dim)
    scale = 1.0 / math.sqrt(head_dim)
    window = int(getattr(model, "sliding_window", 0) or 0)
    if name == "Attn":  # deepgengraph_exp/cases/kernels/attn.py:18-34
        def f(q, k, v):
            return _attn.attention(q, k, v, causal=True, scale=scale, window=window)
    elif name == "Gemma2":  # gemma2.py:19-38
        cap = float(model.logit_softcapping)

        def f(q, k, v):
            return _attn.attention(q, k, v, causal=True, softcap=cap, scale=scale, window=window)
    elif name == "H2O":  # h2o.py:18-38
        def f(q, k, v):
            out, score = _attn.h2o_attention(q, k, v, ref_rounding=True)
            return out, score.view(q.shape[0], int(model.kv_head_num), k.shape[1])
    elif name == "RoCo":  # roco.py:18-48
        def f(q, k, v):
            out, s1, s2 = _attn.roco_attention(q, k, v, ref_rounding=True)
            shp = (q.shape[0], int(model.kv_head_num), k.shape[1])
            return out, s1.view(shp), s2.view(shp)
    elif name == "SnapKV":  # snapkv.py:18-40
        ks = int(getattr(model, "kernel_size", 5))

        def f(q, k, v):
            out, score = _attn.snapkv_attention(q, k, v, kernel_size=ks, ref_rounding=True)
            return out, score.view(q.shape[0], int(model.kv_head_num), k.shape[1])
    elif name == "Corm":  # corm.py:18-39
        def f(q, k, v, corm_mask):
            out, hit = _attn.corm_attention(q, k, v, corm_mask, ref_rounding=True)
            return out, hit.view(q.shape[0], int(model.kv_head_num), k.shape[1])
    elif name == "KeyFormer":  # kf.py:18-40
        tau = float(getattr(model, "tau", 1.5))

        def f(q, k, v, exp_rand):
            out, score = _attn.keyformer_attention(q, k, v, exp_rand, tau=tau, ref_rounding=True)
            return out, score.view(q.shape[0], int(model.kv_head_num), k.shape[1])
    else:
        raise NotImplementedError(f"system mi355x has no kernel for case {name!r} "
                                  "(supported: Attn, Gemma2, H2O, RoCo, SnapKV, Corm, KeyFormer)")
    return f


def compile(model, input_names, inputs, output_names, system):
    """compile.py:6 signature. Returns a callable f(*inputs)."""
    if system == "torch":
        return model
    if system in ("mi355x", "our"):
        if list(input_names)[:3] != ["q", "k", "v"]:
            raise NotImplementedError(f"expected inputs (q, k, v), got {list(input_names)}")
        return _attn_f(model)
    raise NotImplementedError(f"system {system} not implemented")
