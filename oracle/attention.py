"""CPU restatement of the reference attention cases — TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

All functions take CPU tensors in the case layout [B, S, H, D] (decode: q [B, H, D], cache [B, H, L, D]) and
evaluate the reference's eager PyTorch formula with its rounding points:

  scores = (q @ k^T) / sqrt(D)          in the input dtype (matmul result rounded, then the division rounded)
  soft-cap: scores /= c; tanh; *= c     each step in the input dtype (gemma2.py:31-33)

Each division by a Python float is evaluated as torch evaluates it on the GPU the reference runs on: an fp32
multiply by the fp32 reciprocal of the fp32 divisor, rounded to the tensor dtype (div_scalar). torch's CPU kernel
divides instead; the two differ in the last bit of some 16-bit quotients (52 of the finite fp16 values at
d = sqrt(128)), which can move a key across the H2O top-k boundary.
  scores += mask                        -inf / 0 in the input dtype; adding 0 is exact, so masked_fill is used
  probs = softmax(scores.float())       fp32
  out = probs.to(dtype) @ v             input dtype

Query rows are processed in chunks: softmax is per row, so chunking changes nothing but peak memory.
"""
from __future__ import annotations

import math

import numpy as np
import torch


def _mm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a @ b in a's dtype with fp32 accumulation and one rounding at the end, as the GPU's 16-bit GEMM computes the
    reference's matmuls. fp16 goes through fp32 products explicitly: CPUs without native fp16 arithmetic otherwise
    take minutes per config-4 head, and on CPUs with it (AVX512-FP16) torch's fp16 matmul gives the same bits."""
    if a.dtype == torch.float16:
        return torch.matmul(a.float(), b.float()).to(torch.float16)
    return torch.matmul(a, b)


def div_scalar(x: torch.Tensor, d: float) -> torch.Tensor:
    """x / d for a tensor x and a Python float d, as torch computes it on the GPU (the reference's
    `torch.matmul(q, k^T) / math.sqrt(D)`, attn.py:29, and `scores /= softcap`, gemma2.py:31): the divisor is
    taken to fp32, its reciprocal rounded to fp32, and x (in fp32) multiplied by it; the product is rounded to
    x's dtype."""
    inv = np.float32(1.0) / np.float32(d)
    return (x.float() * float(inv)).to(x.dtype)


def _scores(qt: torch.Tensor, kT: torch.Tensor, D: int, softcap=None) -> torch.Tensor:
    """attn.py:29 / gemma2.py:29-33 in the input dtype: the matmul result rounded, divided by sqrt(D) (rounded),
    and with a soft-cap: divided by it, tanh, multiplied by it, each rounded."""
    scores = div_scalar(_mm(qt, kT), math.sqrt(D))
    if softcap:
        scores = div_scalar(scores, softcap)
        scores = torch.tanh(scores)
        scores = scores * softcap
    return scores


def _mask(i0: int, n: int, Sq: int, Sk: int, causal: bool, window: int | None) -> torch.Tensor | None:
    """Boolean [n, Sk] mask of *hidden* pairs for query rows i0..i0+n.

    causal: attn.py:22-23 builds triu(full(-inf), diagonal = Sk - Sq + 1), i.e. key j is hidden from query i
    iff j > i + (Sk - Sq) (bottom-right aligned; q_len == 1 hides nothing).
    window (extension for the Gemma-2-style config): key j is also hidden iff i + (Sk - Sq) - j >= window.
    """
    if not causal and not window:
        return None
    i = torch.arange(i0, i0 + n).unsqueeze(1) + (Sk - Sq)
    j = torch.arange(Sk).unsqueeze(0)
    hidden = torch.zeros(n, Sk, dtype=torch.bool)
    if causal:
        hidden |= j > i
    if window:
        hidden |= (i - j) >= window
    return hidden


def attention(q, k, v, *, causal=True, softcap=None, window=None, return_lse=False, q_chunk=256):
    """Attn.forward (deepgengraph_exp/cases/kernels/attn.py:18-34) and Gemma2.forward (gemma2.py:19-38).

    Extensions used by the BASELINE configs: GQA with query head h reading KV head h // (Hq // Hkv) (the
    expand/reshape convention of roco.py:25-27) and an optional causal sliding window.
    Returns out [B, Sq, Hq, D] in q.dtype, and with return_lse the natural-log log-sum-exp [B, Hq, Sq] (fp32)
    of the masked fp32 scores that the softmax sees (-inf for a row with no visible key).
    """
    B, Sq, Hq, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    assert Hq % Hkv == 0
    group = Hq // Hkv
    dt = q.dtype
    qt = q.transpose(1, 2)  # attn.py:25-27
    kt = k.transpose(1, 2)
    vt = v.transpose(1, 2)
    if group > 1:
        kt = kt.repeat_interleave(group, dim=1)
        vt = vt.repeat_interleave(group, dim=1)
    kT = kt.transpose(-2, -1)
    out = torch.empty(B, Hq, Sq, D, dtype=dt)
    lse = torch.empty(B, Hq, Sq, dtype=torch.float32) if return_lse else None
    for i0 in range(0, Sq, q_chunk):
        n = min(q_chunk, Sq - i0)
        scores = _scores(qt[:, :, i0:i0 + n], kT, D, softcap)  # attn.py:29, gemma2.py:29-33
        hidden = _mask(i0, n, Sq, Sk, causal, window)
        if hidden is not None:
            scores = scores.masked_fill(hidden, float("-inf"))  # attn.py:30 (`scores += mask`)
        sf = scores.float()
        probs = torch.softmax(sf, dim=-1)  # attn.py:31
        out[:, :, i0:i0 + n] = _mm(probs.to(dt), vt)  # attn.py:32
        if return_lse:
            lse[:, :, i0:i0 + n] = torch.logsumexp(sf, dim=-1)
    out = out.transpose(1, 2).contiguous()  # attn.py:32-34
    return (out, lse) if return_lse else out


def h2o(q, k, v, *, q_chunk=256):
    """H2O.forward (deepgengraph_exp/cases/kernels/h2o.py:18-38): causal attention plus the fp32 column sums of
    the fp32 probabilities over the query axis, h2o_score [B, H, Sk] (h2o.py:35-36; MHA, as h2o.py:16 asserts).
    Returns (out, h2o_score, lse)."""
    B, Sq, Hq, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    assert Hq == Hkv, "H2O is multi-head attention (h2o.py:16)"
    dt = q.dtype
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    kT = kt.transpose(-2, -1)
    out = torch.empty(B, Hq, Sq, D, dtype=dt)
    lse = torch.empty(B, Hq, Sq, dtype=torch.float32)
    colsum = torch.zeros(B, Hq, Sk, dtype=torch.float32)
    for i0 in range(0, Sq, q_chunk):
        n = min(q_chunk, Sq - i0)
        scores = _scores(qt[:, :, i0:i0 + n], kT, D)  # h2o.py:29
        scores = scores.masked_fill(_mask(i0, n, Sq, Sk, True, None), float("-inf"))  # h2o.py:30
        sf = scores.float()
        probs = torch.softmax(sf, dim=-1)  # h2o.py:31
        out[:, :, i0:i0 + n] = _mm(probs.to(dt), vt)  # h2o.py:32
        colsum += probs.sum(dim=2)  # h2o.py:35-36
        lse[:, :, i0:i0 + n] = torch.logsumexp(sf, dim=-1)
    return out.transpose(1, 2).contiguous(), colsum, lse


def _causal_probs(q, k, v, q_chunk):
    """Shared body of the KV-selection cases (roco.py / snapkv.py / corm.py: MHA, causal, `scores += mask`,
    fp32 softmax, out = probs.to(dtype) @ v). Yields (i0, n, probs [B, H, n, Sk] fp32) per query chunk and fills
    out [B, H, Sq, D] and lse [B, H, Sq] in place; returns (out, lse) holders."""
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    assert k.shape[2] == H, "the reference's selection cases are multi-head attention (roco.py:16 etc.)"
    dt = q.dtype
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    kT = kt.transpose(-2, -1)
    out = torch.empty(B, H, Sq, D, dtype=dt)
    lse = torch.empty(B, H, Sq, dtype=torch.float32)

    def gen():
        for i0 in range(0, Sq, q_chunk):
            n = min(q_chunk, Sq - i0)
            scores = _scores(qt[:, :, i0:i0 + n], kT, D)  # roco.py:37 / snapkv.py:31 / corm.py:30
            scores = scores.masked_fill(_mask(i0, n, Sq, Sk, True, None), float("-inf"))
            sf = scores.float()
            probs = torch.softmax(sf, dim=-1)
            out[:, :, i0:i0 + n] = _mm(probs.to(dt), vt)
            lse[:, :, i0:i0 + n] = torch.logsumexp(sf, dim=-1)
            yield i0, n, probs

    return gen(), out, lse


def roco(q, k, v, *, q_chunk=256):
    """RoCo.forward (deepgengraph_exp/cases/kernels/roco.py:18-48): causal attention plus the fp32 column sums of
    p and of p^2 over the query axis (roco.py:43-47). Returns (out, roco_score, roco_sq_score, lse)."""
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    rows, out, lse = _causal_probs(q, k, v, q_chunk)
    s1 = torch.zeros(B, H, Sk, dtype=torch.float32)
    s2 = torch.zeros(B, H, Sk, dtype=torch.float32)
    for _, _, probs in rows:
        s1 += probs.sum(dim=2)           # roco.py:43, 46
        s2 += (probs ** 2).sum(dim=2)    # roco.py:44, 47
    return out.transpose(1, 2).contiguous(), s1, s2, lse


def snapkv(q, k, v, *, kernel_size=5, q_chunk=256):
    """SnapKV.forward (deepgengraph_exp/cases/kernels/snapkv.py:18-40): causal attention plus the column sums
    (snapkv.py:36-37) smoothed by F.avg_pool1d(kernel_size, padding=kernel_size // 2, stride=1) (snapkv.py:38).
    Returns (out, snapkv_score, lse)."""
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    rows, out, lse = _causal_probs(q, k, v, q_chunk)
    cs = torch.zeros(B, H, Sk, dtype=torch.float32)
    for _, _, probs in rows:
        cs += probs.sum(dim=2)
    pooled = torch.nn.functional.avg_pool1d(cs, kernel_size=kernel_size, padding=kernel_size // 2, stride=1)
    return out.transpose(1, 2).contiguous(), pooled, lse


def corm(q, k, v, corm_mask, *, q_chunk=256):
    """Corm.forward (deepgengraph_exp/cases/kernels/corm.py:18-39): causal attention plus
    corm_score[b, h, j] = any_i (probs[b, h, i, j] >= corm_mask[i, j]) (corm.py:35-37), a bool [B, H, Sk].
    corm_mask is fp32 [Sq, Sk] (corm.py:47-49 builds 1 / (i + 1)). Returns (out, corm_score, lse)."""
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    rows, out, lse = _causal_probs(q, k, v, q_chunk)
    hit = torch.zeros(B, H, Sk, dtype=torch.bool)
    for i0, n, probs in rows:
        hit |= (probs >= corm_mask[i0:i0 + n]).any(dim=2)
    return out.transpose(1, 2).contiguous(), hit, lse


def keyformer(q, k, v, exp_rand, *, tau=1.5, q_chunk=256):
    """KeyFormer.forward (deepgengraph_exp/cases/kernels/kf.py:18-40): causal attention plus
    kf_score[b, h, j] = sum_i softmax_j((scores + gumbels) / tau)[i, j] with gumbels = -log(exp_rand) (kf.py:36-40),
    where `scores` are the dtype-rounded, masked scores (kf.py:29-30) taken to fp32; exp_rand fp32 [B, H, Sq, Sk].
    Returns (out, kf_score, lse2p) with lse2p the base-2 log-sum-exp of the perturbed rows [B, H, Sq]."""
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    assert k.shape[2] == H, "KeyFormer is multi-head attention (kf.py:16)"
    dt = q.dtype
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    kT = kt.transpose(-2, -1)
    out = torch.empty(B, H, Sq, D, dtype=dt)
    score = torch.zeros(B, H, Sk, dtype=torch.float32)
    lse2p = torch.empty(B, H, Sq, dtype=torch.float32)
    for i0 in range(0, Sq, q_chunk):
        n = min(q_chunk, Sq - i0)
        scores = _scores(qt[:, :, i0:i0 + n], kT, D)  # kf.py:29
        scores = scores.masked_fill(_mask(i0, n, Sq, Sk, True, None), float("-inf"))  # kf.py:30
        probs = torch.softmax(scores.float(), dim=-1)  # kf.py:31
        out[:, :, i0:i0 + n] = _mm(probs.to(dt), vt)  # kf.py:32
        gumbels = -exp_rand[:, :, i0:i0 + n].log()  # kf.py:36-37
        pert = (scores.float() + gumbels) / tau  # kf.py:38
        score += torch.softmax(pert, dim=-1).sum(dim=2)  # kf.py:39-40
        lse2p[:, :, i0:i0 + n] = torch.logsumexp(pert, dim=-1) / math.log(2.0)
    return out.transpose(1, 2).contiguous(), score, lse2p


def exp_rand(B: int, H: int, Sq: int, Sk: int, generator: torch.Generator | None = None) -> torch.Tensor:
    """KeyFormer.prepare's exp_rand (kf.py:48): 1 + |N(0, 1)|, fp32 [B, H, Sq, Sk]."""
    return 1 + torch.randn(B, H, Sq, Sk, generator=generator, dtype=torch.float32).abs()


def corm_mask(q_len: int, kv_len: int) -> torch.Tensor:
    """Corm.prepare's threshold (corm.py:47-49): row i of ones divided by i + 1, fp32 [q_len, kv_len]."""
    m = torch.ones(q_len, kv_len, dtype=torch.float32)
    for i in range(q_len):
        m[i] /= i + 1
    return m


def decode(q, k_cache, v_cache):
    """Attn.forward with q_len == 1 (attn.py:18-34): the mask triu(diagonal = L) hides nothing (attn.py:22-23).

    q [B, Hq, D]; k_cache / v_cache [B, Hkv, L, D] (the module's post-transpose layout); out [B, Hq, D].
    Also returns the natural-log LSE [B, Hq] of the fp32 scores. Processed one batch entry at a time."""
    B, Hq, D = q.shape
    Hkv = k_cache.shape[1]
    group = Hq // Hkv
    dt = q.dtype
    out = torch.empty(B, Hq, D, dtype=dt)
    lse = torch.empty(B, Hq, dtype=torch.float32)
    for b in range(B):
        kb, vb = k_cache[b], v_cache[b]
        if group > 1:
            kb = kb.repeat_interleave(group, dim=0)
            vb = vb.repeat_interleave(group, dim=0)
        scores = _scores(q[b].unsqueeze(1), kb.transpose(-2, -1), D)  # [Hq, 1, L], attn.py:29
        sf = scores.float()
        probs = torch.softmax(sf, dim=-1)
        out[b] = _mm(probs.to(dt), vb).squeeze(1)
        lse[b] = torch.logsumexp(sf, dim=-1).squeeze(1)
    return out, lse


def decode_splitkv(q, k_cache, v_cache, splits: int, scale: float | None = None):
    """Split-KV decode + log-sum-exp merge in float64 (numpy). No reference counterpart: it is pinned by being
    equal to the unsplit softmax for every split count. Per split s over keys [s*c, (s+1)*c), c = ceil(L/splits):
    m_s = max x, l_s = sum exp(x - m_s), O_s = sum exp(x - m_s) v; merge: M = max m_s,
    o = sum e^(m_s - M) O_s / sum e^(m_s - M) l_s, lse = M + log(sum e^(m_s - M) l_s)."""
    qn = q.double().numpy()
    kn = k_cache.double().numpy()
    vn = v_cache.double().numpy()
    B, Hq, D = qn.shape
    Hkv, L = kn.shape[1], kn.shape[2]
    group = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    c = -(-L // splits)
    out = np.zeros((B, Hq, D))
    lse = np.zeros((B, Hq))
    for b in range(B):
        for h in range(Hq):
            x = kn[b, h // group] @ qn[b, h] * scale
            ms, ls, os_ = [], [], []
            for s in range(splits):
                xs = x[s * c:(s + 1) * c]
                if xs.size == 0:
                    continue
                m = xs.max()
                p = np.exp(xs - m)
                ms.append(m)
                ls.append(p.sum())
                os_.append(p @ vn[b, h // group, s * c:(s + 1) * c])
            M = max(ms)
            wts = np.exp(np.array(ms) - M)
            lt = float((wts * np.array(ls)).sum())
            out[b, h] = (wts[:, None] * np.array(os_)).sum(0) / lt
            lse[b, h] = M + math.log(lt)
    return out, lse
