"""Float64 pure-Python loops over tiny inputs: the independent pins of the oracle — TEST INFRASTRUCTURE ONLY.

These follow the mathematical definitions (no intermediate rounding, math.exp / math.sin / math.cos in float64),
written without torch so that a mistake in the vectorised oracle (a wrong mask diagonal, a transposed operand,
a wrong GQA head, a dropped scale) shows up as a mismatch. Inputs are nested lists or numpy arrays.
"""
from __future__ import annotations

import math


def attention(q, k, v, *, causal=True, softcap=None, window=None, scale=None):
    """q [B][Sq][Hq][D], k/v [B][Sk][Hkv][D] -> (out [B][Sq][Hq][D], lse [B][Hq][Sq]).
    Key j visible to query i iff (not causal or j <= i + Sk - Sq) and (not window or i + Sk - Sq - j < window);
    query head h reads KV head h // (Hq // Hkv)."""
    B, Sq, Hq, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    Sk, Hkv = len(k[0]), len(k[0][0])
    group = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    off = Sk - Sq
    out = [[[[0.0] * D for _ in range(Hq)] for _ in range(Sq)] for _ in range(B)]
    lse = [[[0.0] * Sq for _ in range(Hq)] for _ in range(B)]
    for b in range(B):
        for h in range(Hq):
            hk = h // group
            for i in range(Sq):
                xs = []
                for j in range(Sk):
                    if causal and j > i + off:
                        continue
                    if window and i + off - j >= window:
                        continue
                    s = sum(float(q[b][i][h][d]) * float(k[b][j][hk][d]) for d in range(D)) * scale
                    if softcap:
                        s = softcap * math.tanh(s / softcap)
                    xs.append((j, s))
                if not xs:
                    out[b][i][h] = [float("nan")] * D
                    lse[b][h][i] = float("-inf")
                    continue
                m = max(s for _, s in xs)
                den = sum(math.exp(s - m) for _, s in xs)
                lse[b][h][i] = m + math.log(den)
                for d in range(D):
                    out[b][i][h][d] = sum(math.exp(s - m) * float(v[b][j][hk][d]) for j, s in xs) / den
    return out, lse


def colsum(q, k, *, causal=True, scale=None):
    """H2O column sums: colsum[b][h][j] = sum_i softmax_j(scores_i)[j] (h2o.py:35-36), float64."""
    B, Sq, Hq, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    Sk, Hkv = len(k[0]), len(k[0][0])
    group = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    off = Sk - Sq
    cs = [[[0.0] * Sk for _ in range(Hq)] for _ in range(B)]
    for b in range(B):
        for h in range(Hq):
            for i in range(Sq):
                xs = [(j, sum(float(q[b][i][h][d]) * float(k[b][j][h // group][d]) for d in range(D)) * scale)
                      for j in range(Sk) if not (causal and j > i + off)]
                if not xs:
                    continue
                m = max(s for _, s in xs)
                den = sum(math.exp(s - m) for _, s in xs)
                for j, s in xs:
                    cs[b][h][j] += math.exp(s - m) / den
    return cs


def colscores(q, k, *, thr=None):
    """Causal MHA column scores in float64 loops: (sum_i p, sum_i p^2, any_i p >= thr[i][j]) per (b, h, j)
    (roco.py:43-47, corm.py:35-37; masked pairs have p = 0)."""
    B, Sq, H, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    Sk = len(k[0])
    scale = 1.0 / math.sqrt(D)
    off = Sk - Sq
    s1 = [[[0.0] * Sk for _ in range(H)] for _ in range(B)]
    s2 = [[[0.0] * Sk for _ in range(H)] for _ in range(B)]
    hit = [[[False] * Sk for _ in range(H)] for _ in range(B)]
    for b in range(B):
        for h in range(H):
            for i in range(Sq):
                xs = {j: sum(float(q[b][i][h][d]) * float(k[b][j][h][d]) for d in range(D)) * scale
                      for j in range(Sk) if j <= i + off}
                if not xs:
                    continue
                m = max(xs.values())
                den = sum(math.exp(s - m) for s in xs.values())
                for j in range(Sk):
                    pr = math.exp(xs[j] - m) / den if j in xs else 0.0
                    s1[b][h][j] += pr
                    s2[b][h][j] += pr * pr
                    if thr is not None and pr >= float(thr[i][j]):
                        hit[b][h][j] = True
    return s1, s2, hit


def keyformer_colsum(q, k, exp_rand, *, tau):
    """KeyFormer column sums in float64 loops: sum_i softmax_j((s_ij - ln e_ij) / tau) over the causal keys
    (kf.py:36-40), with s_ij = q_i . k_j / sqrt(D) unrounded."""
    B, Sq, H, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    Sk = len(k[0])
    scale = 1.0 / math.sqrt(D)
    off = Sk - Sq
    cs = [[[0.0] * Sk for _ in range(H)] for _ in range(B)]
    for b in range(B):
        for h in range(H):
            for i in range(Sq):
                ys = {}
                for j in range(Sk):
                    if j > i + off:
                        continue
                    s = sum(float(q[b][i][h][d]) * float(k[b][j][h][d]) for d in range(D)) * scale
                    ys[j] = (s - math.log(float(exp_rand[b][h][i][j]))) / tau
                if not ys:
                    continue
                m = max(ys.values())
                den = sum(math.exp(y - m) for y in ys.values())
                for j, y in ys.items():
                    cs[b][h][j] += math.exp(y - m) / den
    return cs


def avg_pool(row, ks):
    """Mean over the window [j - ks//2, j + ks//2] of a list, zeros outside, divided by ks."""
    n, h = len(row), ks // 2
    return [sum(row[t] for t in range(j - h, j + h + 1) if 0 <= t < n) / ks for j in range(n)]


def rms_norm(x, w, eps):
    """Rows of x: y_i = x_i / sqrt(mean(x^2) + eps) * w_i (csrc/norm.cu:34-56 without rounding)."""
    out = []
    for row in x:
        ms = sum(float(a) * float(a) for a in row) / len(row)
        s = 1.0 / math.sqrt(ms + eps)
        out.append([float(a) * s * float(wi) for a, wi in zip(row, w)])
    return out


def silu_and_mul(x):
    """Rows [g | u]: g / (1 + e^-g) * u (csrc/activation.cu:6-22 without rounding)."""
    out = []
    for row in x:
        d = len(row) // 2
        out.append([float(row[i]) / (1.0 + math.exp(-float(row[i]))) * float(row[d + i]) for i in range(d)])
    return out


def rotary(pos, x, head_dim, theta):
    """Rows of x ([T][H*D]) rotated per head: pairs (i, i + D/2), angle pos / theta^(2i/D) (float64)."""
    half = head_dim // 2
    out = []
    for p, row in zip(pos, x):
        o = list(map(float, row))
        for h in range(len(row) // head_dim):
            base = h * head_dim
            for i in range(half):
                a = float(p) / theta ** (2.0 * i / head_dim)
                c, s = math.cos(a), math.sin(a)
                xa, ya = float(row[base + i]), float(row[base + half + i])
                o[base + i] = xa * c - ya * s
                o[base + half + i] = ya * c + xa * s
        out.append(o)
    return out


def topk_indices(row, k, largest=True):
    """Definition by exhaustive ranking: with NaN ranked above every number and all NaN equal, element i outranks
    j iff it comes first in the direction (larger when largest, else smaller) or they are equal and i < j; the k
    elements outranked by fewer than k others, in ascending index order."""
    def first(a, b):  # a strictly before b in the direction
        if math.isnan(a) or math.isnan(b):
            return math.isnan(a) and not math.isnan(b) if largest else math.isnan(b) and not math.isnan(a)
        return a > b if largest else a < b

    def equal(a, b):
        return (math.isnan(a) and math.isnan(b)) or a == b

    n = len(row)
    sel = []
    for i in range(n):
        rank = sum(1 for j in range(n) if first(row[j], row[i]) or (equal(row[j], row[i]) and j < i))
        if rank < k:
            sel.append(i)
    return sel
