"""CPU restatement of the KV-cache selection (top-k, SnapKV pooling, compaction gather, Corm's nonzero) — TEST
INFRASTRUCTURE ONLY (see oracle/__init__.py)."""
from __future__ import annotations

import numpy as np
import torch


def topk_indices(scores: np.ndarray, k: int) -> np.ndarray:
    """deepgengraph_exp/cases/models/h2o.py:51-52: torch.topk(h2o_score, k) then sort of the indices.

    torch.topk leaves the order among equal values unspecified; this build defines it: a stable descending
    sort by value (so among equal values the lowest index comes first), the first k, then ascending index
    order. -0.0 equals +0.0. Returns int64 [..., k]."""
    s = np.asarray(scores, dtype=np.float32)
    order = np.argsort(-s, axis=-1, kind="stable")[..., :k]
    return np.sort(order, axis=-1).astype(np.int64)


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
