"""CPU restatement of the Llama-2 attention block of config 2 — TEST INFRASTRUCTURE ONLY.

LlamaLayer.forward's first half (deepgengraph_exp/cases/models/attn.py:71-74) with Attention.forward
(models/attn.py:34-53): RmsNorm (csrc/norm.cu semantics, oracle.elementwise.rms_norm) -> qkv = x W_qkv^T ->
split + .contiguous() (models/attn.py:36-39) -> rotary_embedding_online on q and k (models/attn.py:40-41,
csrc/pos_encoding.cu semantics) -> causal attention (Attn.forward) -> out W_o^T (models/attn.py:52).
"""
from __future__ import annotations

import torch

from . import attention as oa
from . import elementwise as oe


def attention_block(x, w_norm, w_qkv, w_o, *, heads, kv_heads, eps=1e-6, theta=10000.0, return_parts=False):
    B, S, hidden = x.shape
    D = hidden // heads
    h = oe.rms_norm(x, w_norm, eps)
    qkv = torch.matmul(h, w_qkv.t())
    q, k, v = qkv.split([heads * D, kv_heads * D, kv_heads * D], dim=-1)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    pos = torch.arange(S, dtype=torch.int32).repeat(B)
    q2, k2 = oe.rotary_embedding_online(pos, q.reshape(B * S, -1), k.reshape(B * S, -1), D, theta)
    q2, k2 = q2.view(B, S, heads, D), k2.view(B, S, kv_heads, D)
    o = oa.attention(q2, k2, v.view(B, S, kv_heads, D), causal=True)
    out = torch.matmul(o.view(B, S, heads * D), w_o.t())
    if return_parts:
        return out, dict(h=h, q=q2, k=k2, v=v.view(B, S, kv_heads, D), o=o)
    return out
