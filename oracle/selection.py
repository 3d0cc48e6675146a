"""CPU restatement of the KV-cache selection (top-k, SnapKV pooling, compaction gather, Corm's nonzero) — TEST
INFRASTRUCTURE ONLY (see oracle/__init__.py)."""
from __future__ import annotations

import numpy as np
import torch


def topk_indices(scores: np.ndarray, k: int, largest: bool = True) -> np.ndarray:
    """deepgengraph_exp/cases/models/h2o.py:51-52: torch.topk(h2o_score, k) then sort of the indices (largest=False:
    torch.topk(..., largest=False), models/roco.py:55).

    torch.topk leaves the order among equal values unspecified; this build defines it: a stable sort by value
    (descending, or ascending when largest=False), so that among equal values the lowest index comes first, the
    first k, then ascending index order. Values are ordered as torch orders them: -0.0 equals +0.0 and NaN (either
    sign) ranks above +inf. Returns int64 [..., k]."""
    s = np.asarray(scores, dtype=np.float32)
    nan = np.isnan(s)
    v = np.where(nan, np.float32(0), s)
    idx = np.broadcast_to(np.arange(s.shape[-1]), s.shape)
    # np.lexsort sorts by its last key first: NaN class, then value, then index
    if largest:
        order = np.lexsort((idx, -v, ~nan), axis=-1)
    else:
        order = np.lexsort((idx, v, nan), axis=-1)
    return np.sort(order[..., :k], axis=-1).astype(np.int64)


def roco_select(score: np.ndarray, sq_score: np.ndarray, q_len: int, recent: int, budget: int) -> np.ndarray:
    """deepgengraph_exp/cases/models/roco.py:54-61 on fp32 roco_score / roco_sq_score [..., n]:

        std = sqrt(roco_sq_score / q_len - (roco_score / q_len) ** 2)                  roco.py:54
        other = topk(std, largest=False, k=n - recent); recent = topk(std, k=recent)   roco.py:55-56
        pick = topk(roco_score.gather(other) / q_len, k=budget)                          roco.py:57-58
        sort(cat(other.gather(pick), recent))                                            roco.py:59-61

    rounded as torch computes it on the GPU: the division of a tensor by the Python number q_len is a multiplication
    by the fp32 reciprocal RN(1 / q_len), ** 2 one fp32 multiply, sqrt correctly rounded (NaN where the variance
    cancels below zero). Ties follow topk_indices (lowest index first); `other` is kept in ascending index order, so
    ties in the last top-k also go to the lowest key index. Returns int64 [..., budget + recent]."""
    s1 = np.asarray(score, dtype=np.float32)
    s2 = np.asarray(sq_score, dtype=np.float32)
    n = s1.shape[-1]
    rcp = np.float32(1) / np.float32(q_len)
    mean = s1 * rcp
    with np.errstate(invalid="ignore"):
        std = np.sqrt(s2 * rcp - mean * mean)
    other = topk_indices(std, n - recent, largest=False)
    rec = topk_indices(std, recent, largest=True)
    pick = topk_indices(np.take_along_axis(s1, other, axis=-1) * rcp, budget)
    sel = np.take_along_axis(other, pick, axis=-1)
    return np.sort(np.concatenate([sel, rec], axis=-1), axis=-1).astype(np.int64)


def avg_pool1d(x: torch.Tensor, kernel_size: int) -> torch.Tensor:
    """snapkv.py:38: F.avg_pool1d(x, kernel_size, padding=kernel_size // 2, stride=1) over the last axis of a
    fp32 [..., n] tensor (zero padding counted in the mean)."""
    shp = x.shape
    y = torch.nn.functional.avg_pool1d(x.reshape(-1, 1, shp[-1]), kernel_size=kernel_size, padding=kernel_size // 2,
                                       stride=1)
    return y.reshape(*shp[:-1], y.shape[-1])


def kv_gather(k: torch.Tensor, v: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """models/h2o.py:53-57: k/v [B, S, Hkv, D], indices [B, Hkv, n] (sorted top-k positions) ->
    kv_cache [B, 2, n, Hkv, D] = cat(gather(k), gather(v)) along a new axis 1."""
    B, S, Hkv, D = k.shape
    n = indices.shape[-1]
    idx = indices.transpose(1, 2)[:, :, :, None].expand(B, n, Hkv, D)  # models/h2o.py:53
    kc = torch.gather(k, dim=1, index=idx).view(B, 1, n, Hkv, D)     # models/h2o.py:54
    vc = torch.gather(v, dim=1, index=idx).view(B, 1, n, Hkv, D)     # models/h2o.py:55
    return torch.cat([kc, vc], dim=1)                                # models/h2o.py:56


def nonzero(x: torch.Tensor) -> torch.Tensor:
    """deepgengraph_exp/cases/models/corm.py:53 (torch.nonzero(corm_score)): int64 [count, x.dim()] coordinates of
    the nonzero elements in row-major order (the library routine the reference calls, on the CPU)."""
    return torch.nonzero(x)
