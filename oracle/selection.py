"""CPU restatement of the H2O key selection — TEST INFRASTRUCTURE ONLY (see oracle/__init__.py)."""
from __future__ import annotations

import numpy as np


def topk_indices(scores: np.ndarray, k: int) -> np.ndarray:
    """deepgengraph_exp/cases/models/h2o.py:51-52: torch.topk(h2o_score, k) then sort of the indices.

    torch.topk leaves the order among equal values unspecified; this build defines it: a stable descending
    sort by value (so among equal values the lowest index comes first), the first k, then ascending index
    order. -0.0 equals +0.0. Returns int64 [..., k]."""
    s = np.asarray(scores, dtype=np.float32)
    order = np.argsort(-s, axis=-1, kind="stable")[..., :k]
    return np.sort(order, axis=-1).astype(np.int64)
