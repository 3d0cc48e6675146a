"""The reference's attention case modules restated on the CPU oracle — TEST INFRASTRUCTURE ONLY.

Same class names, constructor arguments and attributes as deepgengraph_exp/cases/kernels/{attn,gemma2,h2o,roco,
snapkv,corm,kf}.py,
so that tests can hand them to deepgengraph_amd.compile.compile() exactly as run_kernel.py:44-78 does. forward()
evaluates the oracle (oracle/attention.py) on CPU copies of the inputs and returns CPU tensors.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import attention as _oa


class _Case(nn.Module):
    def __init__(self, kv_head_num=32, head_num=32, head_dim=128):
        super().__init__()
        self.kv_head_num = kv_head_num
        self.head_num = head_num
        self.head_dim = head_dim
        self.hidden_size = head_num * head_dim
        self.kv_hidden_size = kv_head_num * head_dim
        self.group_size = self.head_num // self.kv_head_num

    def prepare(self, batch_size=1, q_len=4096, kv_len=4096, dtype=torch.float16, device="cpu", seed=0):
        """attn.py:36-50 / gemma2.py:41-54 / h2o.py:41-55 from a seeded CPU generator: Attn draws uniform [0, 1)
        inputs (torch.rand, attn.py:38), the other cases N(0, 1) (torch.randn, gemma2.py:42)."""
        g = torch.Generator().manual_seed(seed)
        draw = torch.rand if isinstance(self, Attn) else torch.randn
        q = draw(batch_size, q_len, self.head_num, self.head_dim, generator=g).to(dtype).to(device)
        k = draw(batch_size, kv_len, self.kv_head_num, self.head_dim, generator=g).to(dtype).to(device)
        v = draw(batch_size, kv_len, self.kv_head_num, self.head_dim, generator=g).to(dtype).to(device)
        return {"input": {"q": q, "k": k, "v": v}, "output": list(self.OUTPUTS)}


class Attn(_Case):
    """deepgengraph_exp/cases/kernels/attn.py:7-34."""
    OUTPUTS = ("out",)

    def forward(self, q, k, v):
        return _oa.attention(q.cpu(), k.cpu(), v.cpu(), causal=True)


class Gemma2(_Case):
    """deepgengraph_exp/cases/kernels/gemma2.py:7-38 (+ optional `sliding_window`, + GQA)."""
    OUTPUTS = ("out",)

    def __init__(self, logit_softcapping=50.0, kv_head_num=32, head_num=32, head_dim=128, sliding_window=0):
        super().__init__(kv_head_num, head_num, head_dim)
        self.logit_softcapping = logit_softcapping
        self.sliding_window = sliding_window

    def forward(self, q, k, v):
        return _oa.attention(q.cpu(), k.cpu(), v.cpu(), causal=True, softcap=self.logit_softcapping,
                             window=self.sliding_window or None)


class H2O(_Case):
    """deepgengraph_exp/cases/kernels/h2o.py:7-38."""
    OUTPUTS = ("out", "h2o_score")

    def forward(self, q, k, v):
        out, colsum, _ = _oa.h2o(q.cpu(), k.cpu(), v.cpu())
        return out, colsum.view(q.shape[0], self.kv_head_num, k.shape[1])


class RoCo(_Case):
    """deepgengraph_exp/cases/kernels/roco.py:7-48."""
    OUTPUTS = ("out", "roco_score", "roco_sq_score")

    def forward(self, q, k, v):
        out, s1, s2, _ = _oa.roco(q.cpu(), k.cpu(), v.cpu())
        return out, s1, s2


class SnapKV(_Case):
    """deepgengraph_exp/cases/kernels/snapkv.py:7-40."""
    OUTPUTS = ("out", "snapkv_score")

    def __init__(self, kernel_size=5, kv_head_num=32, head_num=32, head_dim=128):
        super().__init__(kv_head_num, head_num, head_dim)
        self.kernel_size = kernel_size

    def forward(self, q, k, v):
        out, score, _ = _oa.snapkv(q.cpu(), k.cpu(), v.cpu(), kernel_size=self.kernel_size)
        return out, score


class Corm(_Case):
    """deepgengraph_exp/cases/kernels/corm.py:7-58 (prepare adds corm_mask = 1 / (i + 1), corm.py:47-49)."""
    OUTPUTS = ("out", "corm_score")

    def prepare(self, batch_size=1, q_len=4096, kv_len=4096, dtype=torch.float16, device="cpu", seed=0):
        spec = super().prepare(batch_size, q_len, kv_len, dtype, device, seed)
        spec["input"]["corm_mask"] = _oa.corm_mask(q_len, kv_len).to(device)
        return spec

    def forward(self, q, k, v, corm_mask):
        out, hit, _ = _oa.corm(q.cpu(), k.cpu(), v.cpu(), corm_mask.cpu())
        return out, hit


class KeyFormer(_Case):
    """deepgengraph_exp/cases/kernels/kf.py:7-60 (prepare adds exp_rand = 1 + |N(0, 1)|, kf.py:48)."""
    OUTPUTS = ("out", "kf_score")

    def __init__(self, tau=1.5, kv_head_num=32, head_num=32, head_dim=128):
        super().__init__(kv_head_num, head_num, head_dim)
        self.tau = tau

    def prepare(self, batch_size=1, q_len=4096, kv_len=4096, dtype=torch.float16, device="cpu", seed=0):
        spec = super().prepare(batch_size, q_len, kv_len, dtype, device, seed)
        g = torch.Generator().manual_seed(seed + 1)
        spec["input"]["exp_rand"] = _oa.exp_rand(batch_size, self.head_num, q_len, kv_len, g).to(device)
        return spec

    def forward(self, q, k, v, exp_rand):
        out, score, _ = _oa.keyformer(q.cpu(), k.cpu(), v.cpu(), exp_rand.cpu(), tau=self.tau)
        return out, score.view(q.shape[0], self.kv_head_num, k.shape[1])
