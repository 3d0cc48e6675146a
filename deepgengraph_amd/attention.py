"""Attention entry points on MI355X: prefill (causal / soft-cap / sliding window / GQA), H2O column sums,
top-k key selection, and split-KV decode. Each allocates its outputs with torch on the inputs' device (as the
callables produced by the reference's compile() do, to_triton.cpp:579-590) and launches the HIP kernels of
libdgg_hip.so on the current stream.
"""
from __future__ import annotations

import math

import torch

from . import _lib


def _check_bshd(name: str, t: torch.Tensor):
    if t.dim() != 4:
        raise RuntimeError(f"{name}: expected [B, S, H, D], got shape {tuple(t.shape)}")
    if t.stride(-1) != 1:
        raise RuntimeError(f"{name}: head dimension must be contiguous (stride {t.stride(-1)})")


def _check_qk(name: str, q: torch.Tensor, k: torch.Tensor):
    """q [B, Sq, Hq, D] and k [B, Sk, Hkv, D] as the column kernels read them: k's batch, head dim and dtype are
    taken from q."""
    _check_bshd("q", q)
    _check_bshd("k", k)
    if k.shape[0] != q.shape[0] or k.shape[3] != q.shape[3]:
        raise RuntimeError(f"{name}: incompatible shapes q {tuple(q.shape)} k {tuple(k.shape)}")
    if k.dtype != q.dtype:
        raise RuntimeError(f"{name}: q and k dtypes differ")


# Key count from which a one-row call runs on the split-KV decode kernels instead of the prefill kernel (whose
# 256-row workgroups would compute one live row per (batch, head)).
DECODE_MIN_KEYS = 256


def _decode_shaped(Sq: int, Sk: int, softcap, window, ref_rounding: bool, dtype) -> bool:
    """A call the decode kernels compute exactly as the prefill kernel would: one query row (nothing masked by the
    bottom-right causal mask), enough keys to split, no soft-cap, no window that hides keys, no reference
    rounding (the decode kernels keep fp32 scores)."""
    return (Sq == 1 and Sk >= DECODE_MIN_KEYS and not softcap and (not window or window >= Sk) and not ref_rounding
            and dtype in (torch.float16, torch.bfloat16))


# Short query blocks over long key ranges (chunked prefill, multi-row and grouped-query decode) run on the split-KV
# kernels: at most SPLITKV_MAX_QLEN query rows and SPLITKV_MAX_ROWS rows per KV head (query heads of the group x
# query rows), over at least SPLITKV_MIN_KEYS keys. The prefill kernel would give each (batch, head) one workgroup
# of 256 rows, mostly empty, and read the whole key range in it.
SPLITKV_MAX_QLEN = 64
SPLITKV_MAX_ROWS = 128
SPLITKV_MIN_KEYS = 512


def _splitkv_shaped(Sq: int, Sk: int, Hq: int, Hkv: int, ref_rounding: bool, dtype) -> bool:
    rows = (Hq // Hkv) * Sq
    return (Sq <= SPLITKV_MAX_QLEN and rows <= SPLITKV_MAX_ROWS and Sk >= SPLITKV_MIN_KEYS and Sk >= 4 * Sq
            and not ref_rounding and dtype in (torch.float16, torch.bfloat16))


def splitkv_splits(B: int, Sq: int, Hq: int, Hkv: int, span: int) -> int:
    """Key slices for a split-KV call over `span` keys: about 1024 workgroups over the chip, each slice at least 512
    keys and at least 32 keys per row it serves, so that the partials written and merged stay a few percent of the
    K / V bytes read. (Measured on MI355X at 32K keys: q_len 1-16 over 32 heads ran best with 16-32 slices, 5.0-5.2
    TB/s, against 4.2-4.7 TB/s with 256; q_len 64 with 16.)"""
    rows = (Hq // Hkv) * Sq
    rpw = 32 if rows <= 32 else 64
    groups = B * Hkv * (-(-rows // rpw))
    want = -(-1024 // max(1, groups))
    min_keys = max(512, 32 * min(rows, rpw))
    return int(max(1, min(1024, want, -(-span // min_keys))))


def decode_splits(B: int, Hq: int, L: int) -> int:
    """Split count for a decode call: enough splits for ~512 workgroups, and up to 8 splits of at least 4,096 keys
    (a split costs a partial and its share of the merge, so beyond that more of them only adds work), with at least
    128 keys per split (one unrolled block of the partial kernel). Measured on MI355X, fp16, D=128, us per call:

    ============================  ==============================================  ======
    shape (B, H, L)               splits: time                                    picked
    ============================  ==============================================  ======
    64, 32, 32768 [B, L, H, D]    1: 5,280-5,310  2: 5,121  8: 4,939  32: 5,314      8
    64, 32, 32768 [B, H, L, D]    1: 4,880  8: 4,877  32: 5,019 (flat)               8
    1, 32, 32768                  4: 128  8: 90  16: 86  64: 96  256: 148           16
    4, 32, 32768                  2: 323  8: 318  16: 320  64: 336                   8
    1, 32, 4096                   2: 36  8: 19  16: 18  32: 23                      16
    8, 8, 131072                  2: 891  4: 612  8: 618  64: 634                    8
    16, 32, 8192                  2: 316  4: 315  16: 328  64: 362                   2
    2, 8, 65536                   4: 230  16: 93  32: 90  64: 96                    32
    ============================  ==============================================  ======
    """
    want = max(-(-512 // max(1, B * Hq)), min(8, -(-L // 4096)))
    return int(max(1, min(1024, want, -(-L // 128))))


def rotary_cos_sin(positions: torch.Tensor, head_dim: int, rope_theta: float) -> torch.Tensor:
    """The (cos, sin) table of rotary_embedding_online (csrc/pos_encoding.cu:83-86) for the positions: fp32
    [n, head_dim], row t = cos of the head_dim/2 angles pos[t] / theta^(2i/head_dim), then their sines. Feeds the
    query rotation fused into attention(..., rope_cos_sin=...)."""
    dev = _lib.require_gpu(positions)
    if positions.dtype != torch.int32 or not positions.is_contiguous():
        raise RuntimeError("rotary_cos_sin: positions must be a contiguous int32 tensor")
    n = positions.numel()
    out = torch.empty(n, head_dim, dtype=torch.float32, device=positions.device)
    _lib.call("dgg_rotary_cos_sin", _lib.ptr(positions), _lib.ptr(out), n, int(head_dim), float(rope_theta),
              _lib.stream_handle(dev))
    return out


def _tag_lse(lse: torch.Tensor, ref_rounding: bool, lse_base2: bool) -> torch.Tensor:
    """Records on an lse tensor the options of the forward that wrote it, so that the column passes can take them
    from it (a copy or a slice of the tensor does not carry them)."""
    lse.dgg_ref_rounding = bool(ref_rounding)
    lse.dgg_lse_base2 = bool(lse_base2)
    return lse


def _lse_options(name: str, lse: torch.Tensor, ref_rounding, lse_base2):
    """The (ref_rounding, lse_base2) a column pass must use with `lse`: the scores must be rounded as the forward
    that wrote the lse rounded them, and the lse read in the base it was written in. Values not given are taken from
    the record attention() leaves on its lse; a given value that contradicts the record is refused, and so is a
    missing ref_rounding for an lse without a record."""
    tag_rr = getattr(lse, "dgg_ref_rounding", None)
    tag_b2 = getattr(lse, "dgg_lse_base2", None)
    if ref_rounding is None:
        if tag_rr is None:
            raise RuntimeError(f"{name}: pass ref_rounding= as given to the attention() call that wrote lse (this lse "
                               "tensor carries no record of it)")
        ref_rounding = tag_rr
    elif tag_rr is not None and bool(ref_rounding) != tag_rr:
        raise RuntimeError(f"{name}: ref_rounding={bool(ref_rounding)} but lse was written with ref_rounding={tag_rr}")
    if lse_base2 is None:
        lse_base2 = bool(tag_b2) if tag_b2 is not None else False
    elif tag_b2 is not None and bool(lse_base2) != tag_b2:
        raise RuntimeError(f"{name}: lse_base2={bool(lse_base2)} but lse was written with lse_base2={tag_b2}")
    return bool(ref_rounding), bool(lse_base2)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = True, softcap: float = 0.0,
              window: int = 0, scale: float | None = None, return_lse: bool = False, ref_rounding: bool = False,
              out: torch.Tensor | None = None, lse_base2: bool = False, rope_cos_sin: torch.Tensor | None = None):
    """Fused attention forward. q [B, Sq, Hq, D]; k, v [B, Sk, Hkv, D]; returns out [B, Sq, Hq, D] (q.dtype)
    and, with return_lse, lse [B, Hq, Sq] fp32 (natural log; base 2 with lse_base2, the form
    attention_colsum(..., lse_base2=True) reads fastest).

    Semantics of Attn.forward / Gemma2.forward (deepgengraph_exp/cases/kernels/attn.py:18-34,
    gemma2.py:19-38): scores = q.k^T * scale (default 1/sqrt(D)), optional softcap*tanh(scores/softcap),
    bottom-right aligned causal mask (attn.py:22-23), optional sliding window (key j visible iff
    i + Sk - Sq - j < window), fp32 softmax, P.V. ref_rounding rounds the scores to the input dtype at the
    reference's rounding points (slower; used for H2O selection parity). A one-row multi-head call over at least
    DECODE_MIN_KEYS keys (the reference's decode case) runs on the split-KV decode kernels; other short query blocks
    over long key ranges (_splitkv_shaped: chunked prefill, multi-row and grouped-query decode) on the split-KV
    attention kernels (splitkv_attention).

    rope_cos_sin (head_dim 128, 16-bit inputs): q is taken unrotated and each query row is rotated inside the
    kernel by its row of this table (rotary_cos_sin of the rows' positions, [B * Sq, 128], batch-major), as
    rotary_embedding_online would have rotated it in place (models/attn.py:41); q is not modified."""
    dev = _lib.require_gpu(q, k, v, out, rope_cos_sin)
    for name, t in (("q", q), ("k", k), ("v", v)):
        _check_bshd(name, t)
    B, Sq, Hq, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    if k.shape[0] != B or v.shape != k.shape or k.shape[3] != D:
        raise RuntimeError(f"attention: incompatible shapes q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise RuntimeError("attention: q, k, v dtypes differ")
    if out is None:
        out = torch.empty(B, Sq, Hq, D, dtype=q.dtype, device=q.device)
    else:
        _check_bshd("out", out)
        if out.shape != q.shape or out.dtype != q.dtype:
            raise RuntimeError("attention: out must match q in shape and dtype")
    lse = _tag_lse(torch.empty(B, Hq, Sq, dtype=torch.float32, device=q.device), ref_rounding,
                   lse_base2) if return_lse else None
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    if rope_cos_sin is not None:
        if (rope_cos_sin.dtype != torch.float32 or not rope_cos_sin.is_contiguous()
                or tuple(rope_cos_sin.shape) != (B * Sq, D)):
            raise RuntimeError(f"attention: rope_cos_sin must be a contiguous fp32 [{B * Sq}, {D}] tensor")
        flags = ((_lib.ATTN_CAUSAL if causal else 0) | (_lib.ATTN_REF_ROUNDING if ref_rounding else 0)
                 | (_lib.ATTN_LSE_BASE2 if lse_base2 else 0))
        strides = _lib.int64_array([*q.stride()[:3], *k.stride()[:3], *v.stride()[:3], *out.stride()[:3]])
        _lib.call("dgg_attn_prefill_rope", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(lse), B, Sq,
                  Sk, Hq, Hkv, D, strides, scale, float(softcap or 0.0), int(window or 0), flags,
                  _lib.dtype_code(q.dtype), _lib.ptr(rope_cos_sin), _lib.stream_handle(dev))
        return (out, lse) if return_lse else out
    if Hq == Hkv and _decode_shaped(Sq, Sk, softcap, window, ref_rounding, q.dtype):
        # One query row (attn.py:22-23: the bottom-right causal mask hides nothing): the split-KV decode kernels,
        # reading the case layout [B, L, H, D] through its strides.
        splits = decode_splits(B, Hq, Sk)
        ws = torch.empty(max(decode_workspace_bytes(B, Hq, D, splits), 16), dtype=torch.uint8, device=q.device)
        lse1 = torch.empty(B, Hq, dtype=torch.float32, device=q.device) if return_lse else None
        strides = _lib.int64_array([q.stride(0), q.stride(2), k.stride(0), k.stride(2), k.stride(1), v.stride(0),
                                    v.stride(2), v.stride(1), out.stride(0), out.stride(2)])
        _lib.call("dgg_attn_decode", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(lse1),
                  _lib.ptr(ws), ws.numel(), B, Hq, Hkv, Sk, D, strides, splits, scale, _lib.dtype_code(q.dtype),
                  _lib.stream_handle(dev))
        if return_lse:
            lse.copy_(lse1.view(B, Hq, 1) * (math.log2(math.e) if lse_base2 else 1.0))
        return (out, lse) if return_lse else out
    if _splitkv_shaped(Sq, Sk, Hq, Hkv, ref_rounding, q.dtype):
        _splitkv(q, k, v, out, lse, causal, softcap, window, scale, lse_base2, None, dev)
        return (out, lse) if return_lse else out
    flags = ((_lib.ATTN_CAUSAL if causal else 0) | (_lib.ATTN_REF_ROUNDING if ref_rounding else 0)
             | (_lib.ATTN_LSE_BASE2 if lse_base2 else 0))
    strides = _lib.int64_array([*q.stride()[:3], *k.stride()[:3], *v.stride()[:3], *out.stride()[:3]])
    _lib.call("dgg_attn_prefill", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(lse), B, Sq, Sk,
              Hq, Hkv, D, strides, scale, float(softcap or 0.0), int(window or 0), flags, _lib.dtype_code(q.dtype),
              _lib.stream_handle(dev))
    return (out, lse) if return_lse else out


def _splitkv(q, k, v, out, lse, causal, softcap, window, scale, lse_base2, splits, dev):
    B, Sq, Hq, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    if splits is None:
        first = max(0, Sk - Sq - window + 1) if window else 0
        splits = splitkv_splits(B, Sq, Hq, Hkv, Sk - first)
    need = int(_lib.load().dgg_attn_splitkv_workspace_bytes(B, Sq, Hq, D, splits))
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=q.device)
    flags = (_lib.ATTN_CAUSAL if causal else 0) | (_lib.ATTN_LSE_BASE2 if lse_base2 else 0)
    strides = _lib.int64_array([*q.stride()[:3], *k.stride()[:3], *v.stride()[:3], *out.stride()[:3]])
    _lib.call("dgg_attn_splitkv", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(ws),
              ws.numel(), B, Sq, Sk, Hq, Hkv, D, strides, int(splits), float(scale), float(softcap or 0.0),
              int(window or 0), flags, _lib.dtype_code(q.dtype), _lib.stream_handle(dev))


def splitkv_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = True,
                      softcap: float = 0.0, window: int = 0, scale: float | None = None, return_lse: bool = False,
                      lse_base2: bool = False, splits: int | None = None, out: torch.Tensor | None = None):
    """attention() on the split-KV kernels, whatever the shape (attention() picks them by itself for short query
    blocks over long key ranges): the keys any row sees are cut into `splits` slices (default splitkv_splits),
    each workgroup takes one slice and up to 64 rows of a KV head (its query heads times the query rows), and a merge
    combines the slices. Same arguments, semantics and results as attention() without reference rounding."""
    dev = _lib.require_gpu(q, k, v, out)
    for name, t in (("q", q), ("k", k), ("v", v)):
        _check_bshd(name, t)
    B, Sq, Hq, D = q.shape
    if k.shape[0] != B or v.shape != k.shape or k.shape[3] != D:
        raise RuntimeError(f"splitkv_attention: incompatible shapes q {tuple(q.shape)} k {tuple(k.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise RuntimeError("splitkv_attention: q, k, v dtypes differ")
    if out is None:
        out = torch.empty(B, Sq, Hq, D, dtype=q.dtype, device=q.device)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(-1) != 1:
        raise RuntimeError("splitkv_attention: out must match q")
    lse = _tag_lse(torch.empty(B, Hq, Sq, dtype=torch.float32, device=q.device), False,
                   lse_base2) if return_lse else None
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    _splitkv(q, k, v, out, lse, causal, softcap, window, scale, lse_base2, splits, dev)
    return (out, lse) if return_lse else out


def attention_colsum(q: torch.Tensor, k: torch.Tensor, lse: torch.Tensor, *, causal: bool = True,
                     softcap: float = 0.0, window: int = 0, scale: float | None = None,
                     ref_rounding: bool | None = None, lse_base2: bool | None = None) -> torch.Tensor:
    """Column sums of the softmax probabilities over the query axis, per query head: [B, Hq, Sk] fp32, recomputed
    from q, k and the lse written by attention(..., return_lse=True) with the same options. ref_rounding and
    lse_base2 must be those of that call: left as None they are read from the record attention() keeps on its lse,
    and a value that contradicts the record raises (for an lse without the record, ref_rounding must be given).
    ref_rounding=True rounds the 16-bit scores where the reference's eager module rounds them (attn.py:29,
    gemma2.py:29-33), which the selection cases' 1e-3 contract on the sums needs; False keeps fp32 scores (faster,
    but up to ~1% off the reference's sums in 16-bit)."""
    dev = _lib.require_gpu(q, k, lse)
    _check_qk("attention_colsum", q, k)
    ref_rounding, lse_base2 = _lse_options("attention_colsum", lse, ref_rounding, lse_base2)
    B, Sq, Hq, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    if lse.shape != (B, Hq, Sq) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise RuntimeError(f"attention_colsum: lse must be contiguous fp32 [{B}, {Hq}, {Sq}]")
    colsum = torch.empty(B, Hq, Sk, dtype=torch.float32, device=q.device)
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    flags = ((_lib.ATTN_CAUSAL if causal else 0) | (_lib.ATTN_REF_ROUNDING if ref_rounding else 0)
             | (_lib.ATTN_LSE_BASE2 if lse_base2 else 0))
    strides = _lib.int64_array([*q.stride()[:3], *k.stride()[:3]])
    _lib.call("dgg_attn_colsum", _lib.ptr(q), _lib.ptr(k), _lib.ptr(lse), _lib.ptr(colsum), B, Sq, Sk, Hq, Hkv, D,
              strides, scale, float(softcap or 0.0), int(window or 0), flags, _lib.dtype_code(q.dtype),
              _lib.stream_handle(dev))
    return colsum


def h2o_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, ref_rounding: bool = True):
    """H2O.forward (deepgengraph_exp/cases/kernels/h2o.py:18-38): causal attention output [B, S, H, D] and the fp32
    probability column sums h2o_score [B, Hkv, Sk]. Two launches: the forward kernel (which also writes the row
    lse) and the column-sum kernel. With GQA the per-query-head sums are averaged over each KV group (the
    convention of roco.py:40-41)."""
    out, lse = attention(q, k, v, causal=True, return_lse=True, ref_rounding=ref_rounding, lse_base2=True)
    colsum = attention_colsum(q, k, lse, causal=True, ref_rounding=ref_rounding, lse_base2=True)
    Hq, Hkv = q.shape[2], k.shape[2]
    if Hq != Hkv:
        colsum = colsum.view(q.shape[0], Hkv, Hq // Hkv, -1).mean(dim=2)
    return out, colsum


def attention_colscore(q: torch.Tensor, k: torch.Tensor, lse: torch.Tensor, *, epilogue: int,
                       thr: torch.Tensor | None = None, causal: bool = True, window: int = 0,
                       scale: float | None = None, ref_rounding: bool | None = None,
                       lse_base2: bool | None = None):
    """Column scores over the query axis from q, k and the forward's lse (same options; ref_rounding and lse_base2
    as in attention_colsum), per query head [B, Hq, Sk]:
    epilogue COL_SUM -> sum_i p; COL_SUM_SQ -> (sum_i p, sum_i p^2) (roco.py:43-47); COL_ANY_GE -> bool
    any_i p[i, j] >= thr[i, j] with thr fp32 [Sq, Sk] (corm.py:35-37)."""
    dev = _lib.require_gpu(q, k, lse, thr)
    _check_qk("attention_colscore", q, k)
    ref_rounding, lse_base2 = _lse_options("attention_colscore", lse, ref_rounding, lse_base2)
    B, Sq, Hq, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    if lse.shape != (B, Hq, Sq) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise RuntimeError(f"attention_colscore: lse must be contiguous fp32 [{B}, {Hq}, {Sq}]")
    out0 = out1 = anyo = None
    thr_rs = 0
    if epilogue == _lib.COL_ANY_GE:
        if thr is None or thr.dim() != 2 or thr.shape != (Sq, Sk) or thr.dtype != torch.float32 or thr.stride(-1) != 1:
            raise RuntimeError(f"attention_colscore: thr must be fp32 [{Sq}, {Sk}] with unit column stride")
        thr_rs = thr.stride(0)
        anyo = torch.empty(B, Hq, Sk, dtype=torch.uint8, device=q.device)
    else:
        out0 = torch.empty(B, Hq, Sk, dtype=torch.float32, device=q.device)
        if epilogue == _lib.COL_SUM_SQ:
            out1 = torch.empty(B, Hq, Sk, dtype=torch.float32, device=q.device)
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    flags = ((_lib.ATTN_CAUSAL if causal else 0) | (_lib.ATTN_REF_ROUNDING if ref_rounding else 0)
             | (_lib.ATTN_LSE_BASE2 if lse_base2 else 0))
    strides = _lib.int64_array([*q.stride()[:3], *k.stride()[:3]])
    _lib.call("dgg_attn_colscore", _lib.ptr(q), _lib.ptr(k), _lib.ptr(lse), int(epilogue), _lib.ptr(out0),
              _lib.ptr(out1), _lib.ptr(anyo), _lib.ptr(thr), thr_rs, B, Sq, Sk, Hq, Hkv, D, strides, scale, 0.0,
              int(window or 0), flags, _lib.dtype_code(q.dtype), _lib.stream_handle(dev))
    if epilogue == _lib.COL_ANY_GE:
        return anyo.view(torch.bool)
    return (out0, out1) if epilogue == _lib.COL_SUM_SQ else out0


def _require_mha(name: str, q: torch.Tensor, k: torch.Tensor):
    if q.shape[2] != k.shape[2]:
        raise RuntimeError(f"{name}: the reference case is multi-head attention (head_num == kv_head_num)")


def roco_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, ref_rounding: bool = True):
    """RoCo.forward (deepgengraph_exp/cases/kernels/roco.py:18-48): causal attention, roco_score = sum_i p and
    roco_sq_score = sum_i p^2 per key, fp32 [B, H, Sk]. MHA, as roco.py:16 asserts."""
    _require_mha("roco_attention", q, k)
    out, lse = attention(q, k, v, causal=True, return_lse=True, ref_rounding=ref_rounding, lse_base2=True)
    s1, s2 = attention_colscore(q, k, lse, epilogue=_lib.COL_SUM_SQ, causal=True, ref_rounding=ref_rounding,
                                lse_base2=True)
    return out, s1, s2


def avg_pool1d(x: torch.Tensor, kernel_size: int) -> torch.Tensor:
    """F.avg_pool1d(x, kernel_size, padding=kernel_size // 2, stride=1) over the last axis of a contiguous fp32
    [..., n] tensor (snapkv.py:38); kernel_size odd."""
    dev = _lib.require_gpu(x)
    if x.dtype != torch.float32 or not x.is_contiguous():
        raise RuntimeError("avg_pool1d: x must be a contiguous fp32 tensor")
    n = x.shape[-1]
    out = torch.empty_like(x)
    _lib.call("dgg_avg_pool1d", _lib.ptr(x), _lib.ptr(out), x.numel() // n if n else 0, n, int(kernel_size),
              _lib.stream_handle(dev))
    return out


def snapkv_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, kernel_size: int = 5,
                     ref_rounding: bool = True):
    """SnapKV.forward (deepgengraph_exp/cases/kernels/snapkv.py:18-40): causal attention, then the column sums of
    p pooled by avg_pool1d(kernel_size) along the keys: snapkv_score fp32 [B, Hkv, Sk]. With GQA the per-head sums
    are averaged over each KV group before the pooling, as h2o_attention does."""
    out, cs = h2o_attention(q, k, v, ref_rounding=ref_rounding)
    return out, avg_pool1d(cs.contiguous(), kernel_size)


def corm_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, corm_mask: torch.Tensor, *,
                   ref_rounding: bool = True):
    """Corm.forward (deepgengraph_exp/cases/kernels/corm.py:18-39): causal attention and
    corm_score[b, h, j] = any_i p[b, h, i, j] >= corm_mask[i, j] (bool [B, H, Sk]); corm_mask fp32 [Sq, Sk].
    MHA, as corm.py:16 asserts."""
    _require_mha("corm_attention", q, k)
    out, lse = attention(q, k, v, causal=True, return_lse=True, ref_rounding=ref_rounding, lse_base2=True)
    hit = attention_colscore(q, k, lse, epilogue=_lib.COL_ANY_GE, thr=corm_mask, causal=True,
                             ref_rounding=ref_rounding, lse_base2=True)
    return out, hit


def keyformer_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, exp_rand: torch.Tensor, *,
                        tau: float = 1.5, ref_rounding: bool = True):
    """KeyFormer.forward (deepgengraph_exp/cases/kernels/kf.py:18-40): causal attention `out` [B, S, H, D] and
    kf_score [B, H, Sk] fp32, the column sums over the queries of softmax((scores + gumbels) / tau) with
    gumbels = -log(exp_rand) (kf.py:36-40); exp_rand fp32 [B, H, Sq, Sk] (unit key stride). MHA, as kf.py:16
    asserts. Three launches: the forward, the perturbed row lse, the column pass."""
    dev = _lib.require_gpu(q, k, v, exp_rand)
    _check_qk("keyformer_attention", q, k)
    _require_mha("keyformer_attention", q, k)
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    if (exp_rand.dtype != torch.float32 or exp_rand.dim() != 4 or tuple(exp_rand.shape) != (B, H, Sq, Sk)
            or exp_rand.stride(-1) != 1):
        raise RuntimeError(f"keyformer_attention: exp_rand must be fp32 [{B}, {H}, {Sq}, {Sk}] with unit key stride")
    out = attention(q, k, v, causal=True, ref_rounding=ref_rounding)
    scale = 1.0 / math.sqrt(D)
    flags = _lib.ATTN_CAUSAL | (_lib.ATTN_REF_ROUNDING if ref_rounding else 0)
    strides = _lib.int64_array([*q.stride()[:3], *k.stride()[:3]])
    er_strides = _lib.int64_array(list(exp_rand.stride()[:3]))
    lse2 = torch.empty(B, H, Sq, dtype=torch.float32, device=q.device)
    _lib.call("dgg_attn_kf_rowlse", _lib.ptr(q), _lib.ptr(k), _lib.ptr(exp_rand), er_strides, _lib.ptr(lse2), B, Sq,
              Sk, H, H, D, strides, scale, float(tau), 0, flags, _lib.dtype_code(q.dtype), _lib.stream_handle(dev))
    score = torch.empty(B, H, Sk, dtype=torch.float32, device=q.device)
    _lib.call("dgg_attn_kf_colsum", _lib.ptr(q), _lib.ptr(k), _lib.ptr(exp_rand), er_strides, _lib.ptr(lse2),
              _lib.ptr(score), B, Sq, Sk, H, H, D, strides, scale, float(tau), 0, flags, _lib.dtype_code(q.dtype),
              _lib.stream_handle(dev))
    return out, score


def kv_gather(k: torch.Tensor, v: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """KV-cache compaction after the selection (models/h2o.py:53-57): k / v [B, S, Hkv, D], indices int64
    [B, Hkv, n] -> kv_cache [B, 2, n, Hkv, D] with kv_cache[b, 0, i, h] = k[b, indices[b, h, i], h] (1: v).
    Indices outside [0, S) give zero rows."""
    dev = _lib.require_gpu(k, v, indices)
    for name, t in (("k", k), ("v", v)):
        _check_bshd(name, t)
    if v.shape != k.shape or v.dtype != k.dtype:
        raise RuntimeError("kv_gather: k and v must match")
    B, S, Hkv, D = k.shape
    if indices.dtype != torch.int64 or indices.dim() != 3 or indices.shape[:2] != (B, Hkv) or not indices.is_contiguous():
        raise RuntimeError(f"kv_gather: indices must be contiguous int64 [{B}, {Hkv}, n]")
    n = indices.shape[2]
    out = torch.empty(B, 2, n, Hkv, D, dtype=k.dtype, device=k.device)
    _lib.call("dgg_kv_gather", _lib.ptr(k), _lib.ptr(v), _lib.ptr(indices), _lib.ptr(out), B, S, Hkv, D, n,
              _lib.int64_array([*k.stride()[:3], *v.stride()[:3]]), _lib.dtype_code(k.dtype), _lib.stream_handle(dev))
    return out


def nonzero(x: torch.Tensor) -> torch.Tensor:
    """torch.nonzero of a bool / uint8 tensor (Corm's key selection, deepgengraph_exp/cases/models/corm.py:53):
    int64 [count, x.dim()] coordinates of the nonzero elements in row-major order. Reads the count back to the
    host (as torch.nonzero does) to size the result."""
    dev = _lib.require_gpu(x)
    if x.dtype not in (torch.bool, torch.uint8) or not x.is_contiguous() or x.dim() < 1:
        raise RuntimeError("nonzero: x must be a contiguous bool / uint8 tensor with at least one dimension")
    numel = x.numel()
    n = x.shape[-1]
    rows = numel // n if n else 0
    ws = torch.empty(max(int(_lib.load().dgg_nonzero_workspace_bytes(rows)), 8), dtype=torch.uint8, device=x.device)
    coords = torch.empty(max(numel, 1), x.dim(), dtype=torch.int64, device=x.device)
    total = torch.empty(1, dtype=torch.int64, device=x.device)
    _lib.call("dgg_nonzero", _lib.ptr(x), x.dim(), _lib.int64_array(list(x.shape)), _lib.ptr(coords), numel,
              _lib.ptr(total), _lib.ptr(ws), ws.numel(), _lib.stream_handle(dev))
    return coords[: int(total.item())]


def topk_indices(scores: torch.Tensor, k: int, largest: bool = True) -> torch.Tensor:
    """deepgengraph_exp/cases/models/h2o.py:51-52 (torch.topk then sort of the indices) with a defined tie
    order: the k largest (largest=False: smallest, models/roco.py:55) of each row of scores [..., n] (fp32), ties
    broken by the lowest index, NaN ranked above +inf as torch.topk ranks it, returned as int64 indices [..., k] in
    ascending order."""
    dev = _lib.require_gpu(scores)
    if scores.dtype != torch.float32 or not scores.is_contiguous():
        raise RuntimeError("topk_indices: scores must be a contiguous fp32 tensor")
    n = scores.shape[-1]
    rows = scores.numel() // n if n else 0
    out = torch.empty(*scores.shape[:-1], k, dtype=torch.int64, device=scores.device)
    ws = _select_workspace(rows, n, scores.device)
    _lib.call("dgg_topk_select_ws", _lib.ptr(scores), rows, n, int(k), 1 if largest else 0, _lib.ptr(out),
              _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.stream_handle(dev))
    return out


def _select_workspace(rows: int, n: int, device) -> torch.Tensor | None:
    """Scratch of the selections over rows of more than 65536 keys (several workgroups per row); None below."""
    need = int(_lib.load().dgg_select_workspace_bytes(rows, n))
    if need <= 0:
        return None
    return torch.empty(need, dtype=torch.uint8, device=device)


def roco_select(score: torch.Tensor, sq_score: torch.Tensor, q_len: int, recent: int, budget: int) -> torch.Tensor:
    """RoCo's KV selection, deepgengraph_exp/cases/models/roco.py:54-61, in one kernel: std of each key's
    probabilities from roco_score / roco_sq_score [..., n] (fp32, rounded as torch rounds it on the GPU), the
    `recent` keys of largest std plus the `budget` keys of largest roco_score among the n - recent of smallest std,
    as int64 indices [..., budget + recent] in ascending order (ties: lowest index first)."""
    dev = _lib.require_gpu(score)
    for t in (score, sq_score):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise RuntimeError("roco_select: scores must be contiguous fp32 tensors")
    if sq_score.shape != score.shape or sq_score.device != score.device:
        raise RuntimeError(f"roco_select: score {tuple(score.shape)} and sq_score {tuple(sq_score.shape)} differ")
    n = score.shape[-1]
    rows = score.numel() // n if n else 0
    out = torch.empty(*score.shape[:-1], budget + recent, dtype=torch.int64, device=score.device)
    ws = _select_workspace(rows, n, score.device)
    _lib.call("dgg_roco_select_ws", _lib.ptr(score), _lib.ptr(sq_score), rows, n, int(q_len), int(recent),
              int(budget), _lib.ptr(out), _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.stream_handle(dev))
    return out


def decode_workspace_bytes(B: int, Hq: int, D: int, splits: int) -> int:
    return int(_lib.load().dgg_attn_decode_workspace_bytes(B, Hq, D, splits))


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, *, splits: int = 64,
                     scale: float | None = None, return_lse: bool = False, out: torch.Tensor | None = None,
                     workspace: torch.Tensor | None = None):
    """Attn.forward with q_len == 1 (attn.py:22-23: nothing masked) over a [B, Hkv, L, D] KV cache, computed as a
    split-KV pass (`splits` slices of the cache) followed by a log-sum-exp merge. q [B, Hq, D] -> out
    [B, Hq, D] (+ lse [B, Hq] fp32). `workspace` (uint8/any, >= decode_workspace_bytes bytes) may be passed to
    avoid an allocation per call."""
    dev = _lib.require_gpu(q, k_cache, v_cache, out, workspace)
    if q.dim() != 3 or k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise RuntimeError("decode_attention: expected q [B, Hq, D] and k/v caches [B, Hkv, L, D]")
    B, Hq, D = q.shape
    Hkv, L = k_cache.shape[1], k_cache.shape[2]
    if k_cache.shape[0] != B or k_cache.shape[3] != D:
        raise RuntimeError("decode_attention: cache shape does not match q")
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        if t.stride(-1) != 1:
            raise RuntimeError(f"decode_attention: {name} head dimension must be contiguous")
    if not (q.dtype == k_cache.dtype == v_cache.dtype):
        raise RuntimeError("decode_attention: dtypes differ")
    if out is None:
        out = torch.empty(B, Hq, D, dtype=q.dtype, device=q.device)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(-1) != 1:
        raise RuntimeError("decode_attention: out must match q")
    need = decode_workspace_bytes(B, Hq, D, splits)
    if need < 0:
        raise RuntimeError("decode_attention: invalid sizes")
    if workspace is None:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=q.device)
    elif not workspace.is_contiguous():
        raise RuntimeError("decode_attention: workspace must be contiguous")
    ws_bytes = workspace.numel() * workspace.element_size()
    lse = torch.empty(B, Hq, dtype=torch.float32, device=q.device) if return_lse else None
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    strides = _lib.int64_array([*q.stride()[:2], *k_cache.stride()[:3], *v_cache.stride()[:3], *out.stride()[:2]])
    _lib.call("dgg_attn_decode", _lib.ptr(q), _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.ptr(out), _lib.ptr(lse),
              _lib.ptr(workspace), ws_bytes, B, Hq, Hkv, L, D, strides, int(splits), scale,
              _lib.dtype_code(q.dtype), _lib.stream_handle(dev))
    return (out, lse) if return_lse else out
