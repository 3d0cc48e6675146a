"""Drop-in replacements of the reference's `_csrc` ops (csrc/op.h:2-6, csrc/ffi.cpp:4-8).

Same argument lists and in/out semantics as the pybind11 module: the caller allocates `out`, rotary works in
place on query and key, nothing is returned. The work is enqueued on the current HIP stream of the tensors'
device; there is no host synchronisation. Unsupported dtypes, shapes or strides raise RuntimeError before any
launch (the reference raises c10::Error -> RuntimeError for a bad dtype, csrc/utils.h:8).
"""
from __future__ import annotations

import torch

from . import _lib


def _rows(t: torch.Tensor, what: str):
    """[..., n] tensor -> (rows, row_stride) for a uniformly strided row view with unit inner stride."""
    if t.dim() == 0:
        raise RuntimeError(f"{what}: expected at least one dimension")
    n = t.shape[-1]
    if t.numel() == 0:
        return 0, max(n, 1)
    if t.stride(-1) != 1 and n > 1:
        raise RuntimeError(f"{what}: innermost dimension must be contiguous (stride {t.stride(-1)})")
    if t.dim() == 1:
        return 1, n
    try:
        v = t.view(-1, n)
    except RuntimeError:
        raise RuntimeError(f"{what}: leading dimensions cannot be flattened into uniformly strided rows") from None
    return v.shape[0], v.stride(0) if v.shape[0] > 1 else n


def rms_norm(out: torch.Tensor, input: torch.Tensor, weight: torch.Tensor, epsilon: float) -> None:
    """csrc/norm.cu:85-98: out = T(T(x * rsqrt(mean(x^2) + eps)) * weight) per row of the last dimension."""
    dev = _lib.require_gpu(out, input, weight)
    if not (out.dtype == input.dtype == weight.dtype):
        raise RuntimeError(f"rms_norm: out/input/weight dtypes differ ({out.dtype}, {input.dtype}, {weight.dtype})")
    hidden = input.shape[-1]
    if out.shape != input.shape:
        raise RuntimeError(f"rms_norm: out shape {tuple(out.shape)} != input shape {tuple(input.shape)}")
    if weight.numel() != hidden or (weight.dim() > 0 and weight.stride(-1) != 1 and hidden > 1):
        raise RuntimeError(f"rms_norm: weight must be a contiguous vector of {hidden} elements")
    rows, in_rs = _rows(input, "rms_norm input")
    _, out_rs = _rows(out, "rms_norm out")
    _lib.call("dgg_rms_norm", _lib.ptr(out), _lib.ptr(input), _lib.ptr(weight), rows, hidden, in_rs, out_rs,
              _lib.dtype_code(input.dtype), float(epsilon), _lib.stream_handle(dev))


def fused_add_rms_norm(input: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, epsilon: float) -> None:
    """csrc/norm.cu:100-113 (in place): residual = T(input + residual); input = rms_norm(residual)."""
    dev = _lib.require_gpu(input, residual, weight)
    if not (input.dtype == residual.dtype == weight.dtype):
        raise RuntimeError("fused_add_rms_norm: input/residual/weight dtypes differ")
    if input.shape != residual.shape:
        raise RuntimeError("fused_add_rms_norm: input and residual shapes differ")
    hidden = input.shape[-1]
    if weight.numel() != hidden or (weight.dim() > 0 and weight.stride(-1) != 1 and hidden > 1):
        raise RuntimeError(f"fused_add_rms_norm: weight must be a contiguous vector of {hidden} elements")
    rows, in_rs = _rows(input, "fused_add_rms_norm input")
    _, res_rs = _rows(residual, "fused_add_rms_norm residual")
    _lib.call("dgg_fused_add_rms_norm", _lib.ptr(input), _lib.ptr(residual), _lib.ptr(weight), rows, hidden, in_rs,
              res_rs, _lib.dtype_code(input.dtype), float(epsilon), _lib.stream_handle(dev))


def silu_and_mul(out: torch.Tensor, input: torch.Tensor) -> None:
    """csrc/activation.cu:24-34: input [..., 2d] = [gate | up] -> out [..., d] = T(T(silu(gate)) * up)."""
    dev = _lib.require_gpu(out, input)
    if out.dtype != input.dtype:
        raise RuntimeError(f"silu_and_mul: out dtype {out.dtype} != input dtype {input.dtype}")
    if input.shape[-1] % 2:
        raise RuntimeError(f"silu_and_mul: last dimension {input.shape[-1]} must be even")
    d = input.shape[-1] // 2
    if out.shape[:-1] != input.shape[:-1] or out.shape[-1] != d:
        raise RuntimeError(f"silu_and_mul: out shape {tuple(out.shape)} does not match input {tuple(input.shape)}")
    rows, in_rs = _rows(input, "silu_and_mul input")
    _, out_rs = _rows(out, "silu_and_mul out")
    _lib.call("dgg_silu_and_mul", _lib.ptr(out), _lib.ptr(input), rows, d, in_rs, out_rs,
              _lib.dtype_code(input.dtype), _lib.stream_handle(dev))


def rms_norm_silu_and_mul(norm_out: torch.Tensor, norm_input: torch.Tensor, weight: torch.Tensor, epsilon: float,
                          act_out: torch.Tensor, act_input: torch.Tensor) -> None:
    """rms_norm(norm_out, norm_input, weight, epsilon) and silu_and_mul(act_out, act_input) in one launch (the decode
    step's RmsNorm.forward and MLP.forward elementwise parts, llama_base.py:287-289, 305-314). Same checks and results
    as the two ops; no counterpart as one op in the reference's _csrc."""
    dev = _lib.require_gpu(norm_out, norm_input, weight, act_out, act_input)
    dt = norm_input.dtype
    if not (norm_out.dtype == dt == weight.dtype == act_out.dtype == act_input.dtype):
        raise RuntimeError("rms_norm_silu_and_mul: all tensors must share one dtype")
    hidden = norm_input.shape[-1]
    if norm_out.shape != norm_input.shape:
        raise RuntimeError("rms_norm_silu_and_mul: norm_out shape differs from norm_input")
    if weight.numel() != hidden or (weight.dim() > 0 and weight.stride(-1) != 1 and hidden > 1):
        raise RuntimeError(f"rms_norm_silu_and_mul: weight must be a contiguous vector of {hidden} elements")
    if act_input.shape[-1] % 2:
        raise RuntimeError(f"rms_norm_silu_and_mul: act_input last dimension {act_input.shape[-1]} must be even")
    d = act_input.shape[-1] // 2
    if act_out.shape[:-1] != act_input.shape[:-1] or act_out.shape[-1] != d:
        raise RuntimeError("rms_norm_silu_and_mul: act_out shape does not match act_input")
    n_rows, n_in_rs = _rows(norm_input, "rms_norm_silu_and_mul norm_input")
    _, n_out_rs = _rows(norm_out, "rms_norm_silu_and_mul norm_out")
    a_rows, a_in_rs = _rows(act_input, "rms_norm_silu_and_mul act_input")
    _, a_out_rs = _rows(act_out, "rms_norm_silu_and_mul act_out")
    _lib.call("dgg_rms_norm_silu_and_mul", _lib.ptr(norm_out), _lib.ptr(norm_input), _lib.ptr(weight), n_rows, hidden,
              n_in_rs, n_out_rs, float(epsilon), _lib.ptr(act_out), _lib.ptr(act_input), a_rows, d, a_in_rs, a_out_rs,
              _lib.dtype_code(dt), _lib.stream_handle(dev))


def rotary_embedding_online(positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor | None, head_size: int,
                            rope_theta: float) -> None:
    """csrc/pos_encoding.cu:180-199: NeoX rotary of query [..., Hq*D] and key [..., Hk*D], in place.

    tokens = query.numel() / query.size(-1); row strides are query.stride(-2) / key.stride(-2) as in the
    reference. positions: int32, one per token. The reference asserts head_size == 128; this build accepts any
    multiple of 16 up to 512."""
    dev = _lib.require_gpu(positions, query, key)
    if positions.dtype != torch.int32:
        raise RuntimeError(f"rotary_embedding_online: positions must be int32 (got {positions.dtype})")
    if key is not None and key.dtype != query.dtype:
        raise RuntimeError("rotary_embedding_online: query and key dtypes differ")
    if head_size <= 0:
        raise RuntimeError(f"rotary_embedding_online: head_size {head_size} must be positive")
    width = query.shape[-1]
    if width % head_size:
        raise RuntimeError(f"rotary_embedding_online: query width {width} is not a multiple of head_size {head_size}")
    tokens = query.numel() // width if width else 0
    if positions.numel() < tokens or not positions.is_contiguous():
        raise RuntimeError(f"rotary_embedding_online: need a contiguous positions tensor with >= {tokens} entries")
    _, q_rs = _rows(query, "rotary_embedding_online query")
    hk, k_rs = 0, 0
    if key is not None:
        if key.shape[-1] % head_size:
            raise RuntimeError("rotary_embedding_online: key width is not a multiple of head_size")
        if key.numel() // max(key.shape[-1], 1) != tokens:
            raise RuntimeError("rotary_embedding_online: query and key token counts differ")
        hk = key.shape[-1] // head_size
        _, k_rs = _rows(key, "rotary_embedding_online key")
    _lib.call("dgg_rotary_embedding_online", _lib.ptr(positions), _lib.ptr(query), _lib.ptr(key), tokens,
              width // head_size, hk, head_size, q_rs, k_rs, _lib.dtype_code(query.dtype), float(rope_theta),
              _lib.stream_handle(dev))


def rotary_embedding(positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor | None, head_size: int,
                     cos_sin_cache: torch.Tensor, is_neox: bool) -> None:
    """csrc/pos_encoding.cu:152-178 (the cos/sin-cache rotary, kernel pos_encoding.cu:7-61), in place on query
    [..., Hq*head_size] and key [..., Hk*head_size]: cos_sin_cache [max_position, rot_dim] of the input dtype, row
    p = [cos | sin]; is_neox pairs (i, i + rot_dim/2), else GPT-J pairs (2i, 2i+1); dims past rot_dim unchanged.
    Products and results are rounded to the dtype as the reference's c10 Half / BFloat16 arithmetic rounds them.
    A token whose position is outside [0, max_position) is left unchanged."""
    dev = _lib.require_gpu(positions, query, key, cos_sin_cache)
    if positions.dtype != torch.int32:
        raise RuntimeError(f"rotary_embedding: positions must be int32 (got {positions.dtype})")
    if cos_sin_cache.dtype != query.dtype or (key is not None and key.dtype != query.dtype):
        raise RuntimeError("rotary_embedding: query, key and cos_sin_cache dtypes differ")
    if cos_sin_cache.dim() != 2 or not cos_sin_cache.is_contiguous():
        raise RuntimeError("rotary_embedding: cos_sin_cache must be a contiguous [max_position, rot_dim] tensor")
    rot_dim = cos_sin_cache.shape[1]
    width = query.shape[-1]
    if head_size <= 0 or width % head_size:
        raise RuntimeError(f"rotary_embedding: query width {width} is not a multiple of head_size {head_size}")
    tokens = query.numel() // width if width else 0
    if positions.numel() < tokens or not positions.is_contiguous():
        raise RuntimeError(f"rotary_embedding: need a contiguous positions tensor with >= {tokens} entries")
    _, q_rs = _rows(query, "rotary_embedding query")
    hk, k_rs = 0, 0
    if key is not None:
        if key.shape[-1] % head_size or key.numel() // max(key.shape[-1], 1) != tokens:
            raise RuntimeError("rotary_embedding: key width or token count does not match")
        hk = key.shape[-1] // head_size
        _, k_rs = _rows(key, "rotary_embedding key")
    _lib.call("dgg_rotary_embedding", _lib.ptr(positions), _lib.ptr(query), _lib.ptr(key), tokens,
              width // head_size, hk, head_size, q_rs, k_rs, _lib.ptr(cos_sin_cache), rot_dim, cos_sin_cache.shape[0],
              1 if is_neox else 0, _lib.dtype_code(query.dtype), _lib.stream_handle(dev))
