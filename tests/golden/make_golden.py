"""Writes the golden vectors under tests/golden/ from the float64 brute-force definitions in oracle/brute.py.

    python tests/golden/make_golden.py

The reference ships no golden vectors for this path (no .npy/.pt fixtures; its ONNX case graphs are missing
blobs), so these fixtures come from the mathematical definitions evaluated in float64 with pure-Python loops,
independent of torch. Inputs are drawn from N(0, 1) with numpy's PCG64 and rounded to the precision of the
dtype they are meant for (stored as float32 values that are exactly representable in that dtype).
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import brute  # noqa: E402

OUT = Path(__file__).resolve().parent


def _rounded(rng, shape, dtype):
    x = rng.standard_normal(shape).astype(np.float32)
    return torch.from_numpy(x).to(dtype).float().numpy()


def attn_case(name, rng, B, Sq, Sk, Hq, Hkv, D, dtype, causal=True, softcap=None, window=None, sinks=0):
    q = _rounded(rng, (B, Sq, Hq, D), dtype)
    k = _rounded(rng, (B, Sk, Hkv, D), dtype)
    v = _rounded(rng, (B, Sk, Hkv, D), dtype)
    if sinks:
        k[:, rng.choice(Sk, sinks, replace=False)] *= 4.0
    out, lse = brute.attention(q.tolist(), k.tolist(), v.tolist(), causal=causal, softcap=softcap, window=window)
    arrays = dict(q=q, k=k, v=v, out=np.array(out), lse=np.array(lse))
    if causal and not softcap and not window and Hq == Hkv:
        arrays["colsum"] = np.array(brute.colsum(q.tolist(), k.tolist(), causal=True))
    meta = dict(kind="attention", dtype=str(dtype).replace("torch.", ""), causal=causal, softcap=softcap or 0.0,
                window=window or 0)
    return name, arrays, meta


def main():
    rng = np.random.Generator(np.random.PCG64(20250101))
    cases = [
        # tiny: for the CPU oracle pins (D = 8)
        attn_case("attn_tiny_causal_f32", rng, 1, 16, 16, 2, 2, 8, torch.float32),
        attn_case("attn_tiny_gqa_softcap_window_f32", rng, 1, 12, 16, 4, 2, 8, torch.float32, softcap=5.0, window=5),
        attn_case("attn_tiny_noncausal_f32", rng, 2, 5, 9, 2, 1, 8, torch.float32, causal=False),
        attn_case("attn_tiny_causal_sq_gt_sk_f32", rng, 1, 9, 5, 1, 1, 8, torch.float32),
        # kernel-sized (D = 64): also run by the GPU parity tests
        attn_case("attn_d64_causal_bf16", rng, 1, 80, 80, 2, 2, 64, torch.bfloat16),
        attn_case("attn_d64_gqa_softcap_window_bf16", rng, 1, 70, 100, 4, 2, 64, torch.bfloat16, softcap=5.0,
                  window=33),
        attn_case("attn_d64_h2o_sinks_f16", rng, 1, 72, 72, 2, 2, 64, torch.float16, sinks=3),
    ]

    # elementwise
    x = _rounded(rng, (3, 64), torch.bfloat16)
    w = (1.0 + 0.02 * _rounded(rng, (64,), torch.float32)).astype(np.float32)
    w = torch.from_numpy(w).to(torch.bfloat16).float().numpy()
    cases.append(("rms_norm_bf16", dict(x=x, w=w, out=np.array(brute.rms_norm(x.tolist(), w.tolist(), 1e-6))),
                  dict(kind="rms_norm", dtype="bfloat16", eps=1e-6)))
    g = _rounded(rng, (4, 2 * 40), torch.float16)
    cases.append(("silu_and_mul_f16", dict(x=g, out=np.array(brute.silu_and_mul(g.tolist()))),
                  dict(kind="silu_and_mul", dtype="float16")))
    pos = np.array([0, 1, 7, 100, 4095, 31], dtype=np.int32)
    xr = _rounded(rng, (6, 3 * 32), torch.float32)
    cases.append(("rotary_d32_f32", dict(pos=pos, x=xr, out=np.array(brute.rotary(pos.tolist(), xr.tolist(), 32,
                                                                                     10000.0))),
                  dict(kind="rotary", dtype="float32", head_dim=32, theta=10000.0)))
    # top-k with ties (values from a small set so that many are equal), including -0.0 / +0.0
    vals = rng.integers(0, 6, size=(4, 50)).astype(np.float32) * 0.25
    vals[0, :10] = 0.0
    vals[0, 10:20] = -0.0
    idx = np.array([brute.topk_indices(row.tolist(), 17) for row in vals], dtype=np.int64)
    cases.append(("topk_ties", dict(x=vals, out=idx), dict(kind="topk", k=17)))

    index = {}
    for name, arrays, meta in cases:
        np.savez_compressed(OUT / f"{name}.npz", **arrays)
        index[name] = meta
    (OUT / "index.json").write_text(json.dumps(index, indent=1, sort_keys=True) + "\n")
    print(f"wrote {len(cases)} fixtures to {OUT}")


if __name__ == "__main__":
    main()
