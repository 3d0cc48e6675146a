"""End-to-end harness over a random-weight Llama-2-7B, the counterpart of the reference's run_e2e.py:190-251.

    python -m deepgengraph_amd.run_e2e -m attn -s mi355x --seqlen 4096 --layer_num 32

Builds the model of deepgengraph_exp/cases/models/<model>.py (embedding, `layer_num` decoder layers, final
RMSNorm; Llama-2-7B sizes of run_e2e.py:22-43: hidden 4096, 32 heads of 128, MLP 11008, fp16) with random weights
and random token ids (run_e2e.py:46-90), plugs in the attention callable compile(...) returns for the case
(run_e2e.py:206-230) and times the forward with the reference's perf() report line (deepgengraph_exp/utils.py:
50-82; run = warmup = 50, run_e2e.py:241-249). RMSNorm, rotary and SiLU-and-mul run on this library's kernels
(the csrc ops of llama_base.py:257-314), each residual add inside the next RMSNorm (fused_add_rms_norm); the
projections are torch matmuls. After the attention each model
compacts its KV cache as its reference model does (top-k of the case's key scores, RoCo's std rule, Corm's
nonzero); with system 'mi355x' those steps run on this library's kernels (topk_indices, kv_gather, nonzero),
with 'torch' on torch's. Every model here uses random weights: in the reference only `attn` (and `h2o`) skip
load_param, the others read checkpoint files, which this build does not restate.
"""
from __future__ import annotations

import argparse
import math
import random
import time

import numpy as np
import torch
import torch.nn as nn

from . import attention as A
from . import ops
from .cases import KERNEL_ZOO
from .compile import compile as dgg_compile

SCORED = {"h2o", "snapkv", "kf"}  # attention returns (out, score); keep the top cache_budget keys


class E2EConfig:
    """run_e2e.py:22-43 (SimpleConfig) plus the selection parameters of llm_setup_random (run_e2e.py:60-77)."""

    def __init__(self, seqlen, layer_num, vocab_size=32000, hidden_size=4096, dtype=torch.float16, device="cuda"):
        self.vocab_size = vocab_size
        self.hidden_size = hidden_size
        self.num_hidden_layers = layer_num
        self.max_position_embeddings = seqlen
        self.rms_norm_eps = 1e-6
        self.torch_dtype = dtype
        self.rope_theta = self.rotary_base = 10000.0
        self.num_attention_heads = 32
        self.num_key_value_heads = 32
        self.intermediate_size = 11008
        self.hidden_act = "silu"
        self.cache_budget = 512
        assert self.cache_budget < seqlen, "cache_budget (512) must be below seqlen (run_e2e.py:63)"
        self.roco_recent = 256
        self.tau = 1.5
        rows = torch.arange(1, seqlen + 1, dtype=torch.float32, device=device)[:, None]
        self.corm_mask = torch.ones(seqlen, seqlen, dtype=torch.float32, device=device) / rows  # run_e2e.py:67-70


class RmsNorm(nn.Module):
    """llama_base.py:276-289 on dgg_rms_norm."""

    def __init__(self, dim, eps, dtype):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, dtype=dtype))

    def forward(self, x):
        out = torch.empty_like(x)
        ops.rms_norm(out, x, self.weight, self.eps)
        return out


class MLP(nn.Module):
    """llama_base.py:293-314: gate_up projection, SiLU-and-mul (dgg_silu_and_mul), down projection."""

    def __init__(self, hidden_size, intermediate_size, dtype):
        super().__init__()
        self.gate_up_proj = nn.Linear(hidden_size, 2 * intermediate_size, bias=False, dtype=dtype)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False, dtype=dtype)

    def forward(self, x):
        gate_up = self.gate_up_proj(x)
        out = torch.empty(*gate_up.shape[:-1], gate_up.shape[-1] // 2, dtype=gate_up.dtype, device=gate_up.device)
        ops.silu_and_mul(out, gate_up)
        return self.down_proj(out)


class Attention(nn.Module):
    """models/attn.py:11-56 and the selection tails of models/{h2o,snapkv,kf,roco,corm}.py."""

    def __init__(self, cfg: E2EConfig, attn_f, model: str, system: str):
        super().__init__()
        self.cfg, self.attn_f, self.model, self.system = cfg, attn_f, model, system
        self.hidden_size = cfg.hidden_size
        self.head_num = cfg.num_attention_heads
        self.kv_head_num = cfg.num_key_value_heads
        self.head_dim = self.hidden_size // self.head_num
        self.kv_hidden_size = self.kv_head_num * self.head_dim
        self.qkv_proj = nn.Linear(self.hidden_size, self.hidden_size + 2 * self.kv_hidden_size, bias=False,
                                  dtype=cfg.torch_dtype)
        self.out_proj = nn.Linear(self.hidden_size, self.hidden_size, bias=False, dtype=cfg.torch_dtype)

    def _select(self, idx, k4, v4):
        """KV-cache compaction of the selected keys idx [B, Hkv, n] (ascending): [B, 2, n, Hkv, D]
        (models/h2o.py:53-57)."""
        if self.system == "torch":
            B, S, H, D = k4.shape
            g = idx.transpose(1, 2)[:, :, :, None].expand(B, idx.shape[-1], H, D)
            kc = torch.gather(k4, dim=1, index=g).view(B, 1, -1, H, D)
            vc = torch.gather(v4, dim=1, index=g).view(B, 1, -1, H, D)
            return torch.cat([kc, vc], dim=1)
        return A.kv_gather(k4, v4, idx.contiguous())

    def _topk(self, score, k):
        if self.system == "torch":
            return torch.topk(score, k=k, dim=-1, sorted=True)[1].sort(dim=-1)[0]
        return A.topk_indices(score.contiguous(), k)

    def forward(self, x, kv_caches):
        cfg = self.cfg
        qkv = self.qkv_proj(x)
        q, k, v = qkv.split([self.hidden_size, self.kv_hidden_size, self.kv_hidden_size], dim=-1)
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        pos = torch.arange(0, q.shape[1], dtype=torch.int32, device=x.device)
        ops.rotary_embedding_online(pos, q, k, self.head_dim, cfg.rotary_base)
        B, S = q.shape[0], q.shape[1]
        q4 = q.view(B, S, self.head_num, self.head_dim)
        k4 = k.view(B, S, self.kv_head_num, self.head_dim)
        v4 = v.view(B, S, self.kv_head_num, self.head_dim)
        if self.model in ("attn", "gemma2"):
            out = self.attn_f(q4, k4, v4)
            kv_caches.append(torch.cat([k, v], dim=1))
        elif self.model in SCORED:
            if self.model == "kf":  # models/kf.py: a fresh exp_rand per layer
                er = torch.empty(B, self.head_num, S, S, dtype=torch.float32, device=x.device).uniform_(1e-8, 1.0)
                out, score = self.attn_f(q4, k4, v4, er)
            else:
                out, score = self.attn_f(q4, k4, v4)
            kv_caches.append((score, self._select(self._topk(score, cfg.cache_budget), k4, v4)))
        elif self.model == "roco":  # models/roco.py: std of the probabilities, recent window plus top budget
            out, s1, s2 = self.attn_f(q4, k4, v4)
            if self.system == "torch":
                std = torch.sqrt(s2 / S - (s1 / S) ** 2)
                other = torch.topk(std, largest=False, k=S - cfg.roco_recent, dim=-1)[1]
                recent = torch.topk(std, largest=True, k=cfg.roco_recent, dim=-1)[1]
                pick = torch.topk(s1.gather(dim=-1, index=other) / S, dim=-1, k=cfg.cache_budget)[1]
                idx = torch.cat([other.gather(dim=-1, index=pick), recent], dim=-1).sort(dim=-1)[0]
            else:
                idx = A.roco_select(s1.contiguous(), s2.contiguous(), S, cfg.roco_recent, cfg.cache_budget)
            kv_caches.append((s1, s2, self._select(idx, k4, v4)))
        elif self.model == "corm":  # models/corm.py: the flagged (head, key) pairs, as torch.nonzero lists them
            out, score = self.attn_f(q4, k4, v4, cfg.corm_mask[:S, :S].contiguous())
            sel = torch.nonzero(score) if self.system == "torch" else A.nonzero(score)
            kv_caches.append((score, sel, torch.cat([k, v], dim=1)))
        else:
            raise NotImplementedError(self.model)
        return self.out_proj(out.reshape(B, S, -1)), kv_caches


class Layer(nn.Module):
    """models/attn.py:58-83: pre-norm attention and MLP, each with a residual add."""

    def __init__(self, cfg, attn_f, model, system):
        super().__init__()
        self.input_layernorm = RmsNorm(cfg.hidden_size, cfg.rms_norm_eps, cfg.torch_dtype)
        self.attention = Attention(cfg, attn_f, model, system)
        self.mlp = MLP(cfg.hidden_size, cfg.intermediate_size, cfg.torch_dtype)
        self.post_layernorm = RmsNorm(cfg.hidden_size, cfg.rms_norm_eps, cfg.torch_dtype)

    def forward(self, x, kv_caches):
        a, kv_caches = self.attention(self.input_layernorm(x), kv_caches)
        x = x + a
        x = x + self.mlp(self.post_layernorm(x))
        return x, kv_caches


class Llama(nn.Module):
    """models/attn.py:85-109 (forward: embedding, the layers, final RMSNorm; returns (x, kv_caches)).

    With fuse_residual (the default for the 'mi355x' system) each residual add runs inside the RMSNorm that reads
    its result, as the unexported fused_add_rms_norm of csrc/norm.cu:59-83 / 100-113 does: the add after the
    attention with the layer's post_layernorm, the add after the MLP with the next layer's input_layernorm (the
    model's final rms_norm after the last layer). That saves one read and one write of the [S, hidden] residual
    stream per add. The variance is taken from the fp32 sum before it is rounded to the stored residual
    (norm.cu:59-83), where the unfused path (models/attn.py:71-80) takes it from the rounded sum."""

    def __init__(self, cfg, attn_f, model, system, fuse_residual=None):
        super().__init__()
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size, dtype=cfg.torch_dtype)
        self.layers = nn.ModuleList(Layer(cfg, attn_f, model, system) for _ in range(cfg.num_hidden_layers))
        self.rms_norm = RmsNorm(cfg.hidden_size, cfg.rms_norm_eps, cfg.torch_dtype)
        self.eps = cfg.rms_norm_eps
        self.fuse_residual = system != "torch" if fuse_residual is None else bool(fuse_residual)

    def forward(self, token_ids):
        kv_caches = []
        x = self.embed_tokens(token_ids)
        if not self.fuse_residual:
            for layer in self.layers:
                x, kv_caches = layer(x, kv_caches)
            return self.rms_norm(x), kv_caches
        res = x  # the residual stream, updated in place
        h = self.layers[0].input_layernorm(res) if self.layers else self.rms_norm(res)
        for i, layer in enumerate(self.layers):
            a, kv_caches = layer.attention(h, kv_caches)
            ops.fused_add_rms_norm(a, res, layer.post_layernorm.weight, self.eps)  # res += a; a = norm(res)
            m = layer.mlp(a)
            nxt = self.layers[i + 1].input_layernorm if i + 1 < len(self.layers) else self.rms_norm
            ops.fused_add_rms_norm(m, res, nxt.weight, self.eps)  # res += m; m = norm(res)
            h = m
        return h, kv_caches


def perf(label, f, args, run=4, warmup=4):
    """deepgengraph_exp/utils.py:50-82: synchronised wall-clock runs and the same report line."""
    print("warmup start", flush=True)
    for _ in range(warmup):
        torch.cuda.synchronize()
        f(*args)
        torch.cuda.synchronize()
    print("warmup done", flush=True)
    ms = []
    for _ in range(run):
        torch.cuda.synchronize()
        t0 = time.time()
        f(*args)
        torch.cuda.synchronize()
        ms.append((time.time() - t0) * 1000.0)
    print(f"[{label}] avg {np.mean(ms):.4f} ms, min {np.min(ms):.4f} ms, max {np.max(ms):.4f} ms "
          f"({run} runs, {warmup} warmups)", flush=True)
    return float(np.mean(ms))


def build(model: str, system: str, seqlen: int, layer_num: int, seed: int = 0, fuse_residual=None):
    """run_e2e.py:197-238: the case module, its compiled attention callable, the random-weight model and the
    random token ids."""
    if model not in KERNEL_ZOO:
        raise SystemExit(f"model {model} not found in KERNEL_ZOO {list(KERNEL_ZOO)}")
    torch.manual_seed(seed)
    random.seed(seed)
    np.random.seed(seed)
    kernel = KERNEL_ZOO[model]().eval()
    specs = kernel.prepare(q_len=min(seqlen, 1024), kv_len=min(seqlen, 1024), device="cuda")
    names = list(specs["input"].keys())
    attn_f = dgg_compile(model=kernel, input_names=names, inputs=[specs["input"][n] for n in names],
                         output_names=specs["output"], system=system)
    cfg = E2EConfig(seqlen, layer_num)
    with torch.device("cuda"):
        net = Llama(cfg, attn_f, model, system, fuse_residual)
    for p in net.parameters():
        p.requires_grad = False
    token_ids = torch.randint(0, cfg.vocab_size, (1, seqlen), dtype=torch.int64, device="cuda").contiguous()
    return net.eval(), token_ids


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--model", "-m", default="attn", help="Model name")
    ap.add_argument("--system", "-s", default="mi355x", help="System name")
    ap.add_argument("--seqlen", type=int, default=4096, help="seqlen")
    ap.add_argument("--layer_num", type=int, default=32, help="layer_num")
    ap.add_argument("--platform", "-p", default="yes", help="accepted for compatibility (it chose checkpoint paths)")
    ap.add_argument("--run", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-fuse-residual", action="store_true",
                    help="residual adds as separate torch adds (models/attn.py:71-80) instead of fused_add_rms_norm")
    a = ap.parse_args(argv)
    print(f"model={a.model!r} system={a.system!r} seqlen={a.seqlen} layer_num={a.layer_num}")
    net, token_ids = build(a.model, a.system, a.seqlen, a.layer_num,
                           fuse_residual=False if a.no_fuse_residual else None)
    print(f"token_ids.shape={tuple(token_ids.shape)}")
    with torch.no_grad():
        return perf(a.system, net, (token_ids,), run=a.run, warmup=a.warmup)


if __name__ == "__main__":
    main()
