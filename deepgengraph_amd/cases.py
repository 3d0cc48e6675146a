"""The reference's attention case modules (deepgengraph_exp/cases/kernels/__init__.py: KERNEL_ZOO) as the 'torch'
system of the harness: same class names, constructor arguments, attributes, prepare() and output names, with the
eager PyTorch forward the reference times and checks against (compile.py:7-8 returns the module itself for
system='torch'). They run on whatever device their inputs are on, in query-row chunks (exact: the softmax is per
row) so that the [S, S] intermediates stay bounded. The MI355X system never calls them: compile(system='mi355x')
maps each class to the HIP kernels of libdgg_hip.so.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

_CHUNK = 512


class _Case(nn.Module):
    OUTPUTS = ("out",)

    def __init__(self, kv_head_num=32, head_num=32, head_dim=128):
        super().__init__()
        self.kv_head_num = kv_head_num
        self.head_num = head_num
        self.head_dim = head_dim
        self.hidden_size = head_num * head_dim
        self.kv_hidden_size = kv_head_num * head_dim
        self.group_size = self.head_num // self.kv_head_num
        assert self.group_size == 1  # attn.py:16 and the other cases

    def _inputs(self, batch_size, q_len, kv_len, dtype, device, seed, uniform=False):
        g = torch.Generator().manual_seed(seed)
        draw = torch.rand if uniform else torch.randn  # attn.py:38 (rand) vs gemma2.py:42 etc. (randn)
        shape_q = (batch_size, q_len, self.head_num, self.head_dim)
        shape_k = (batch_size, kv_len, self.kv_head_num, self.head_dim)
        return [draw(*s, generator=g).to(dtype).to(device) for s in (shape_q, shape_k, shape_k)]

    def prepare(self, batch_size=1, q_len=4096, kv_len=4096, dtype=torch.float16, device="cuda", seed=0):
        q, k, v = self._inputs(batch_size, q_len, kv_len, dtype, device, seed, uniform=isinstance(self, Attn))
        return {"input": {"q": q, "k": k, "v": v}, "output": list(self.OUTPUTS)}

    def _rows(self, q, k, v, softcap=None):
        """Yields (i0, n, scores [B, H, n, Sk] masked, probs fp32) per query chunk and the output holder:
        scores = (q @ k^T) / sqrt(D) in the input dtype (attn.py:29), optional soft-cap (gemma2.py:31-33),
        bottom-right causal mask (attn.py:22-23), fp32 softmax (attn.py:31); out = probs.to(dtype) @ v."""
        B, Sq, H, D = q.shape
        Sk = k.shape[1]
        qt, vt = q.transpose(1, 2), v.transpose(1, 2).contiguous()
        kT = k.transpose(1, 2).transpose(-2, -1).contiguous()
        out = torch.empty(B, H, Sq, D, dtype=q.dtype, device=q.device)

        def gen():
            for i0 in range(0, Sq, _CHUNK):
                n = min(_CHUNK, Sq - i0)
                scores = torch.matmul(qt[:, :, i0:i0 + n].contiguous(), kT) / math.sqrt(D)
                if softcap:
                    scores /= softcap
                    scores = torch.tanh(scores)
                    scores *= softcap
                i = torch.arange(i0, i0 + n, device=q.device).unsqueeze(1) + (Sk - Sq)
                hidden = torch.arange(Sk, device=q.device).unsqueeze(0) > i
                scores = scores.masked_fill(hidden, float("-inf"))
                probs = torch.softmax(scores.float(), dim=-1)
                out[:, :, i0:i0 + n] = torch.matmul(probs.to(q.dtype), vt)
                yield i0, n, scores, probs

        return gen(), out

    @staticmethod
    def _finish(out):
        return out.transpose(1, 2).contiguous()


class Attn(_Case):
    """deepgengraph_exp/cases/kernels/attn.py:7-50."""

    def forward(self, q, k, v):
        rows, out = self._rows(q, k, v)
        for _ in rows:
            pass
        return self._finish(out)


class Gemma2(_Case):
    """deepgengraph_exp/cases/kernels/gemma2.py:7-54."""

    def __init__(self, logit_softcapping=50.0, kv_head_num=32, head_num=32, head_dim=128):
        super().__init__(kv_head_num, head_num, head_dim)
        self.logit_softcapping = logit_softcapping

    def forward(self, q, k, v):
        rows, out = self._rows(q, k, v, softcap=self.logit_softcapping)
        for _ in rows:
            pass
        return self._finish(out)


class H2O(_Case):
    """deepgengraph_exp/cases/kernels/h2o.py:7-55."""
    OUTPUTS = ("out", "h2o_score")

    def forward(self, q, k, v):
        rows, out = self._rows(q, k, v)
        score = torch.zeros(q.shape[0], self.head_num, k.shape[1], dtype=torch.float32, device=q.device)
        for _, _, _, probs in rows:
            score += probs.sum(dim=2)  # h2o.py:35-36
        return self._finish(out), score.view(q.shape[0], self.kv_head_num, k.shape[1])


class RoCo(_Case):
    """deepgengraph_exp/cases/kernels/roco.py:7-48."""
    OUTPUTS = ("out", "roco_score", "roco_sq_score")

    def forward(self, q, k, v):
        rows, out = self._rows(q, k, v)
        s1 = torch.zeros(q.shape[0], self.head_num, k.shape[1], dtype=torch.float32, device=q.device)
        s2 = torch.zeros_like(s1)
        for _, _, _, probs in rows:
            s1 += probs.sum(dim=2)          # roco.py:43, 46
            s2 += (probs * probs).sum(dim=2)  # roco.py:44, 47
        return self._finish(out), s1, s2


class SnapKV(_Case):
    """deepgengraph_exp/cases/kernels/snapkv.py:7-40."""
    OUTPUTS = ("out", "snapkv_score")

    def __init__(self, kernel_size=5, kv_head_num=32, head_num=32, head_dim=128):
        super().__init__(kv_head_num, head_num, head_dim)
        self.kernel_size = kernel_size

    def forward(self, q, k, v):
        rows, out = self._rows(q, k, v)
        cs = torch.zeros(q.shape[0], self.head_num, k.shape[1], dtype=torch.float32, device=q.device)
        for _, _, _, probs in rows:
            cs += probs.sum(dim=2)  # snapkv.py:36-37
        pooled = torch.nn.functional.avg_pool1d(cs, kernel_size=self.kernel_size, padding=self.kernel_size // 2,
                                                stride=1)  # snapkv.py:38
        return self._finish(out), pooled


class Corm(_Case):
    """deepgengraph_exp/cases/kernels/corm.py:7-58."""
    OUTPUTS = ("out", "corm_score")

    def prepare(self, batch_size=1, q_len=4096, kv_len=4096, dtype=torch.float16, device="cuda", seed=0):
        spec = super().prepare(batch_size, q_len, kv_len, dtype, device, seed)
        spec["input"]["corm_mask"] = (1.0 / torch.arange(1, q_len + 1, dtype=torch.float32)).unsqueeze(1).expand(
            q_len, kv_len).contiguous().to(device)  # corm.py:47-49: row i of ones / (i + 1)
        return spec

    def forward(self, q, k, v, corm_mask):
        rows, out = self._rows(q, k, v)
        hit = torch.zeros(q.shape[0], self.head_num, k.shape[1], dtype=torch.bool, device=q.device)
        for i0, n, _, probs in rows:
            hit |= (probs >= corm_mask[i0:i0 + n]).any(dim=2)  # corm.py:35-37
        return self._finish(out), hit


class KeyFormer(_Case):
    """deepgengraph_exp/cases/kernels/kf.py:7-60."""
    OUTPUTS = ("out", "kf_score")

    def __init__(self, tau=1.5, kv_head_num=32, head_num=32, head_dim=128):
        super().__init__(kv_head_num, head_num, head_dim)
        self.tau = tau

    def prepare(self, batch_size=1, q_len=4096, kv_len=4096, dtype=torch.float16, device="cuda", seed=0):
        spec = super().prepare(batch_size, q_len, kv_len, dtype, device, seed)
        g = torch.Generator().manual_seed(seed + 1)
        spec["input"]["exp_rand"] = (1 + torch.randn(batch_size, self.head_num, q_len, kv_len, generator=g).abs()
                                     ).to(device)  # kf.py:48
        return spec

    def forward(self, q, k, v, exp_rand):
        rows, out = self._rows(q, k, v)
        score = torch.zeros(q.shape[0], self.head_num, k.shape[1], dtype=torch.float32, device=q.device)
        for i0, n, scores, _ in rows:
            pert = (scores.float() - exp_rand[:, :, i0:i0 + n].log()) / self.tau  # kf.py:36-38
            score += torch.softmax(pert, dim=-1).sum(dim=2)  # kf.py:39-40
        return self._finish(out), score.view(q.shape[0], self.kv_head_num, k.shape[1])


KERNEL_ZOO = {
    "attn": Attn,
    "corm": Corm,
    "gemma2": Gemma2,
    "h2o": H2O,
    "kf": KeyFormer,
    "roco": RoCo,
    "snapkv": SnapKV,
}
