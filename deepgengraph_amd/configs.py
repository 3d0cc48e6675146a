"""The five benchmark configurations as concrete, seeded input builders.

Inputs are drawn from N(0, 1) in fp32 with a dedicated torch.Generator per configuration (seed 1000 + config
number), in the order documented per builder, then cast to the configuration's dtype. Builders take size
overrides so that tests can run the same recipe at reduced sizes. Large tensors (the decode cache) are drawn
with a generator on the target device, one batch entry at a time, so no fp32 copy of the whole cache exists.
"""
from __future__ import annotations

import dataclasses
import math

import torch


@dataclasses.dataclass(frozen=True)
class AttnConfig:
    name: str
    B: int
    Sq: int
    Sk: int
    Hq: int
    Hkv: int
    D: int
    dtype: torch.dtype
    causal: bool = True
    softcap: float = 0.0
    window: int = 0
    sinks: int = 0       # number of key rows scaled x4 (H2O heavy hitters)
    topk: int = 0        # H2O selection size
    seed: int = 0

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.D)

    def pairs_per_head(self) -> int:
        """Number of visible (query, key) pairs of one head."""
        off = self.Sk - self.Sq
        total = 0
        for i in range(self.Sq):
            hi = min(self.Sk, i + off + 1) if self.causal else self.Sk
            lo = max(0, i + off - self.window + 1) if self.window else 0
            total += max(0, hi - lo)
        return total

    def flops(self) -> float:
        """Algorithmic FLOPs: 4*D per visible pair (Q.K^T and P.V), summed over heads and batch."""
        return 4.0 * self.D * self.Hq * self.B * self.pairs_per_head()

    def reference_flops(self) -> float:
        """run_kernel.py:24 FLOP model: 4*B*H*S^2*D/2 (causal half)."""
        return 4.0 * self.B * self.Hq * self.Sq * self.Sq * self.D / 2


@dataclasses.dataclass(frozen=True)
class DecodeConfig:
    name: str
    B: int
    Hq: int
    Hkv: int
    L: int
    D: int
    dtype: torch.dtype
    splits: int
    hidden: int          # RMSNorm width of the pre-step
    intermediate: int    # SiLU-and-mul output width of the pre-step (input is 2x)
    seed: int = 0

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.D)

    def bytes(self) -> int:
        """Algorithmic HBM bytes of one decode call: K + V + q + o."""
        e = torch.tensor([], dtype=self.dtype).element_size()
        return e * (2 * self.B * self.Hkv * self.L * self.D + 2 * self.B * self.Hq * self.D)


CFG1 = AttnConfig("cfg1_cpu_plumbing_fp32", 1, 512, 512, 8, 8, 64, torch.float32, seed=1001)
CFG2 = AttnConfig("cfg2_llama2_7b_prefill_bf16", 1, 4096, 4096, 32, 32, 128, torch.bfloat16, seed=1002)
CFG3 = AttnConfig("cfg3_gemma2_gqa_softcap_window_bf16", 2, 8192, 8192, 16, 8, 256, torch.bfloat16,
                  softcap=50.0, window=4096, seed=1003)
CFG4 = AttnConfig("cfg4_h2o_fp16", 1, 4096, 4096, 32, 32, 128, torch.float16, sinks=16, topk=256, seed=1004)
CFG5 = DecodeConfig("cfg5_decode_fp16", 64, 32, 32, 32768, 128, torch.float16, splits=64, hidden=4096,
                    intermediate=11008, seed=1005)

# Llama-2-7B block of config 2.
LLAMA_HIDDEN = 4096
LLAMA_EPS = 1e-6
LLAMA_THETA = 10000.0


def _randn(shape, gen, dtype, device="cpu"):
    return torch.randn(*shape, generator=gen, dtype=torch.float32, device=gen.device).to(dtype).to(device)


def attn_inputs(cfg: AttnConfig, device="cpu", **overrides):
    """q [B, Sq, Hq, D], k, v [B, Sk, Hkv, D] ~ N(0, 1) (draw order q, k, v). With cfg.sinks, then
    `sinks` key positions drawn without replacement (randperm) have k scaled by 4 in every head.
    Returns (q, k, v, sink_positions or None)."""
    cfg = dataclasses.replace(cfg, **overrides) if overrides else cfg
    g = torch.Generator().manual_seed(cfg.seed)
    q = _randn((cfg.B, cfg.Sq, cfg.Hq, cfg.D), g, torch.float32)
    k = _randn((cfg.B, cfg.Sk, cfg.Hkv, cfg.D), g, torch.float32)
    v = _randn((cfg.B, cfg.Sk, cfg.Hkv, cfg.D), g, torch.float32)
    sinks = None
    if cfg.sinks:
        sinks = torch.randperm(cfg.Sk, generator=g)[: cfg.sinks]
        k[:, sinks] *= 4.0
    return q.to(cfg.dtype).to(device), k.to(cfg.dtype).to(device), v.to(cfg.dtype).to(device), sinks


def llama_block_inputs(seed: int = CFG2.seed, S: int = CFG2.Sq, hidden: int = LLAMA_HIDDEN, heads: int = CFG2.Hq,
                       kv_heads: int = CFG2.Hkv, dtype=torch.bfloat16, device="cpu"):
    """Config 2's attention block: x [1, S, hidden] ~ N(0,1); RMSNorm weight 1 + N(0, 0.02);
    W_qkv [hidden + 2*kv_hidden, hidden] ~ N(0, 0.02); W_o [hidden, hidden] ~ N(0, 0.02) (draw order as listed).
    Returns dict(x, w_norm, w_qkv, w_o)."""
    D = hidden // heads
    g = torch.Generator().manual_seed(seed + 100)
    x = _randn((1, S, hidden), g, dtype)
    w_norm = (1.0 + 0.02 * torch.randn(hidden, generator=g)).to(dtype)
    w_qkv = (0.02 * torch.randn(hidden + 2 * kv_heads * D, hidden, generator=g)).to(dtype)
    w_o = (0.02 * torch.randn(hidden, hidden, generator=g)).to(dtype)
    return {k: v.to(device) for k, v in dict(x=x, w_norm=w_norm, w_qkv=w_qkv, w_o=w_o).items()}


def decode_inputs(cfg: DecodeConfig, device="cpu", **overrides):
    """q [B, Hq, D], k_cache / v_cache [B, Hkv, L, D] ~ N(0, 1). Drawn with a generator on `device`: q first,
    then for each batch entry b its K slice then its V slice. Returns (q, k_cache, v_cache)."""
    cfg = dataclasses.replace(cfg, **overrides) if overrides else cfg
    g = torch.Generator(device=device).manual_seed(cfg.seed)
    q = torch.randn(cfg.B, cfg.Hq, cfg.D, generator=g, device=device, dtype=torch.float32).to(cfg.dtype)
    k = torch.empty(cfg.B, cfg.Hkv, cfg.L, cfg.D, dtype=cfg.dtype, device=device)
    v = torch.empty_like(k)
    for b in range(cfg.B):
        k[b] = torch.randn(cfg.Hkv, cfg.L, cfg.D, generator=g, device=device, dtype=torch.float32).to(cfg.dtype)
        v[b] = torch.randn(cfg.Hkv, cfg.L, cfg.D, generator=g, device=device, dtype=torch.float32).to(cfg.dtype)
    return q, k, v


def decode_prestep_inputs(cfg: DecodeConfig, device="cpu"):
    """Config 5 pre-step: x [B, hidden] ~ N(0,1), RMSNorm weight 1 + N(0, 0.02), gate_up [B, 2*intermediate]
    ~ N(0,1) (draw order as listed, CPU generator seed + 200). Returns dict(x, w_norm, gate_up)."""
    g = torch.Generator().manual_seed(cfg.seed + 200)
    x = _randn((cfg.B, cfg.hidden), g, cfg.dtype)
    w_norm = (1.0 + 0.02 * torch.randn(cfg.hidden, generator=g)).to(cfg.dtype)
    gate_up = _randn((cfg.B, 2 * cfg.intermediate), g, cfg.dtype)
    return {k: v.to(device) for k, v in dict(x=x, w_norm=w_norm, gate_up=gate_up).items()}
