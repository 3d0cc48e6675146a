"""Llama-2 glue around the attention kernels: the config-2 attention block and the config-5 decode step.

The attention block follows LlamaLayer.forward's first half (deepgengraph_exp/cases/models/attn.py:71-74) and
Attention.forward (models/attn.py:34-53): RMSNorm -> fused QKV projection -> rotary on q and k -> causal
attention -> output projection. The projections are plain library GEMMs (torch.matmul -> hipBLASLt); everything
else runs in libdgg_hip.so. Unlike the reference, q/k/v are not copied out of the QKV result with
.contiguous() (models/attn.py:36-39): the rotary and attention kernels take the strided views directly. With
fuse_rope (head_dim 128) the query's rotation runs inside the attention kernel from a per-position (cos, sin)
table, and the rotary kernel rotates k only: the query never makes the extra round trip through HBM.
"""
from __future__ import annotations

import torch

from . import attention as _attn
from . import ops


class LlamaAttentionBlock:
    def __init__(self, w_norm, w_qkv, w_o, *, heads: int, kv_heads: int, eps: float = 1e-6,
                 rope_theta: float = 10000.0, fuse_rope: bool = True):
        self.w_norm, self.w_qkv, self.w_o = w_norm, w_qkv, w_o
        self.heads, self.kv_heads = heads, kv_heads
        self.hidden = w_o.shape[0]
        self.head_dim = self.hidden // heads
        self.eps, self.theta = eps, rope_theta
        self.fuse_rope = fuse_rope and self.head_dim == 128 and w_qkv.dtype in (torch.float16, torch.bfloat16)
        self._pos = None
        self._cs = None

    def positions(self, B: int, S: int, device) -> torch.Tensor:
        """Token positions 0..S-1 (models/attn.py:40), repeated for each batch entry."""
        if self._pos is None or self._pos.shape != (B, S) or self._pos.device != device:
            self._pos = torch.arange(S, dtype=torch.int32, device=device).repeat(B, 1).contiguous()
            self._cs = None
        return self._pos

    def cos_sin(self, pos: torch.Tensor) -> torch.Tensor:
        """The query rotation table of the positions (computed once per positions tensor)."""
        if self._cs is None:
            self._cs = _attn.rotary_cos_sin(pos, self.head_dim, self.theta)
        return self._cs

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        B, S, _ = x.shape
        D, H, Hk = self.head_dim, self.heads, self.kv_heads
        h = torch.empty_like(x)
        ops.rms_norm(h, x, self.w_norm, self.eps)                      # LlamaLayer.input_layernorm
        qkv = torch.matmul(h, self.w_qkv.t())                          # models/attn.py:35
        q = qkv[..., : H * D]
        k = qkv[..., H * D: (H + Hk) * D]
        v = qkv[..., (H + Hk) * D:]
        pos = self.positions(B, S, x.device)
        if self.fuse_rope:
            ops.rotary_embedding_online(pos, k, None, D, self.theta)   # models/attn.py:41, key half
            cs = self.cos_sin(pos)                                     # query half: inside the attention kernel
            o = _attn.attention(q.view(B, S, H, D), k.view(B, S, Hk, D), v.view(B, S, Hk, D), causal=True,
                                rope_cos_sin=cs)
        else:
            ops.rotary_embedding_online(pos, q, k, D, self.theta)     # models/attn.py:41
            o = _attn.attention(q.view(B, S, H, D), k.view(B, S, Hk, D), v.view(B, S, Hk, D), causal=True)
        return torch.matmul(o.view(B, S, H * D), self.w_o.t())         # models/attn.py:52


def decode_prestep(x: torch.Tensor, w_norm: torch.Tensor, gate_up: torch.Tensor, eps: float = 1e-6):
    """Config 5 pre-step: RMSNorm of the query-side hidden state and SiLU-and-mul of the MLP activation pair
    (LlamaLayer's RmsNorm.forward and MLP.forward elementwise parts, llama_base.py:287-289, 305-314), both in one
    launch. Returns (normed, act)."""
    normed = torch.empty_like(x)
    act = torch.empty(*gate_up.shape[:-1], gate_up.shape[-1] // 2, dtype=gate_up.dtype, device=gate_up.device)
    ops.rms_norm_silu_and_mul(normed, x, w_norm, eps, act, gate_up)
    return normed, act
