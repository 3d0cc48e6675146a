"""CPU restatement of the csrc elementwise kernels — TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Arithmetic is fp32 with rounding to the storage dtype exactly where the CUDA kernels round: a product of two
16-bit c10 values is computed in float and rounded (c10::Half / c10::BFloat16 operator*), which is what torch's
own 16-bit elementwise multiply does on the CPU.
"""
from __future__ import annotations

import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """csrc/norm.cu:34-56 (PyTorch twin: RmsNorm.norm_torch, llama_base.py:282-285):
    s = rsqrt(sum(x^2) / hidden + eps) in fp32; out = T(T(x * s) * w)."""
    x32 = x.float()
    s = torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)
    return (x32 * s).to(x.dtype) * weight


def fused_add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """csrc/norm.cu:59-83: v = x + residual in fp32; residual <- T(v); variance from the unrounded v;
    output from the rounded residual. Returns (out, new_residual)."""
    v = x.float() + residual.float()
    res = v.to(x.dtype)
    s = torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + eps)
    return (res.float() * s).to(x.dtype) * weight, res


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """csrc/activation.cu:6-22: input [..., 2d] = [gate | up]; out = T(T(g / (1 + exp(-g))) * up)."""
    d = x.shape[-1] // 2
    g = x[..., :d].float()
    silu = (g / (1.0 + torch.exp(-g))).to(x.dtype)
    return silu * x[..., d:]


def rotary_cos_sin(positions: torch.Tensor, head_dim: int, theta: float):
    """pos_encoding.cu:83-86: angle_i = float(pos) / pow(theta, float(2i) / float(D)) in fp32, i < D/2."""
    i = torch.arange(head_dim // 2, dtype=torch.float32)
    denom = torch.pow(torch.tensor(theta, dtype=torch.float32), (2.0 * i) / float(head_dim))
    ang = positions.to(torch.float32).unsqueeze(1) / denom.unsqueeze(0)
    return torch.cos(ang), torch.sin(ang)


def rotary_embedding_online(positions, query, key, head_size: int, rope_theta: float):
    """csrc/pos_encoding.cu:64-113, 180-199, out of place. query [T, Hq*D], key [T, Hk*D] (or None).
    For each head, pairs (x_i, x_{i+D/2}) -> (x c_i - y s_i, y c_i + x s_i) in fp32, stored in the input dtype.
    Returns (query_out, key_out)."""
    c, s = rotary_cos_sin(positions.reshape(-1), head_size, rope_theta)
    half = head_size // 2

    def rot(t):
        if t is None:
            return None
        T = t.shape[0]
        x = t.reshape(T, -1, head_size).float()
        a, b = x[..., :half], x[..., half:]
        cc, ss = c.unsqueeze(1), s.unsqueeze(1)
        o = torch.cat([a * cc - b * ss, b * cc + a * ss], dim=-1)
        return o.to(t.dtype).reshape(t.shape)

    return rot(query), rot(key)


def rotary_embedding(positions, query, key, head_size: int, cos_sin_cache, is_neox: bool):
    """csrc/pos_encoding.cu:7-61, 152-178, out of place: cos_sin_cache [max_position, rot_dim] of the input dtype,
    row p = [cos (rot_dim/2) | sin (rot_dim/2)]; pairs (i, i + rot_dim/2) (is_neox) or (2i, 2i+1) for i < rot_dim/2;
    x' = x*cos - y*sin, y' = y*cos + x*sin in the reference's scalar_t arithmetic: for 16-bit types each product and
    the result rounded to the dtype (c10 Half / BFloat16 operators compute in float and round), fp32 plain. Head
    dims past rot_dim are unchanged. Returns (query_out, key_out)."""
    rot_dim = cos_sin_cache.shape[1]
    embed = rot_dim // 2
    cache = cos_sin_cache[positions.reshape(-1).long()]
    cos, sin = cache[:, :embed].unsqueeze(1), cache[:, embed:].unsqueeze(1)

    def mul(a, b):
        return (a.float() * b.float()).to(a.dtype)

    def rot(t):
        if t is None:
            return None
        T = t.shape[0]
        x = t.reshape(T, -1, head_size).clone()
        if is_neox:
            xs, ys = slice(0, embed), slice(embed, rot_dim)
        else:
            xs, ys = slice(0, rot_dim, 2), slice(1, rot_dim, 2)
        a, b = x[..., xs].clone(), x[..., ys].clone()
        x[..., xs] = (mul(a, cos).float() - mul(b, sin).float()).to(t.dtype)
        x[..., ys] = (mul(b, cos).float() + mul(a, sin).float()).to(t.dtype)
        return x.reshape(t.shape)

    return rot(query), rot(key)
