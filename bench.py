"""Benchmark of the DeepGenGraph attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--sections prefill,decode,...] [--no-cpu-baseline]

Prints ONE JSON line. The headline `value` is config 2: bf16 causal prefill attention at Llama-2-7B shape
(B=1, H=32, S=4096, D=128) in TFLOP/s under the reference's FLOP model 4*B*H*S^2*D/2 (run_kernel.py:24),
one step = one attention forward over inputs already resident in HBM. The decode section reports config 5
(split-KV decode over a 64 x 32 x 32768 x 128 fp16 cache) in GB/s of algorithmic K+V+q+o bytes; the other
sections report configs 3 and 4, the config-2 block and the elementwise kernels. Kernel durations come from
HIP events recorded on the stream the kernels are launched on (torch's current stream). The CPU baseline is
the oracle (reference formula in PyTorch eager on the host cores) on a bounded sample of config 2.

Clock: under a sustained load the part raises its shader clock over the first few hundred launches of this kernel,
so a short warm-up times the kernel at a lower clock than a long one. The line records the shader clock measured
right before and right after the timed region (`clock_mhz`, a one-lane probe reading the cycle counter against the
100 MHz real-time counter), and, apart from `value`, a `steady` figure: the same kernel timed again after the
launches so far are topped up to STEADY_WARMUP, with its own clock reading.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

import torch

METRIC = "attention TFLOP/s (% bf16 MFMA peak) + decode HBM GB/s, Llama-2-7B shapes"
STEADY_WARMUP = 600  # launches before the `steady` figure is timed
STEADY_STEPS = 200
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16/fp16 MFMA
PEAK_HBM_GBPS = 8000.0      # MI355X HBM3E


_COVER = {}  # device -> buffer of the fill that _events_time queues its timed calls behind


def _events_time(fn, iters: int, warmup: int) -> float:
    """Runs fn warmup + iters times; returns the mean GPU time of one call (ms) over iters back-to-back calls,
    from one HIP event pair on the current stream around them.

    The timed calls are queued behind a device fill (512 MiB, repeated) that keeps the GPU busy while the host
    enqueues them, so the host's launch cost (~12 us per call through the Python wrappers) cannot starve the GPU
    between short kernels. A run counts when the start event was still pending after the last call had been
    enqueued, or when a call takes the GPU more than twice as long as the host takes to enqueue it (then the host
    stays ahead); otherwise the cover is made 4x longer and the run repeated. An event pair around each call would
    instead count ~3 us of marker handling inside every bracket (12.6 us kernels read 16 us)."""
    dev = torch.cuda.current_device()
    if dev not in _COVER:
        _COVER[dev] = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    cover = _COVER[dev]
    for _ in range(warmup):
        fn()
    reps = 2
    for _ in range(5):
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(reps):
            cover.fill_(0)
        start.record()
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
        host_s = time.perf_counter() - t0
        covered = not start.query()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / iters
        if covered or ms * 1e-3 > 2.0 * host_s / iters:
            break
        reps *= 4
    return ms


def _variant(fn, iters: int, warm_ms: float = 60.0):
    """A secondary workload's GPU time per call (ms) by _events_time, after a warm-up of about warm_ms of its own
    work (at least 3 calls): each section first builds its inputs on the host, which leaves the GPU idle, and the
    part lowers and then raises its clock over the first tens of milliseconds of load that follow. Returns
    (ms, info) with the warm-up call count and the shader clock just before and after the timed calls."""
    dev = torch.cuda.current_device()
    clk = torch.zeros(2, 2, dtype=torch.int64, device=dev)
    fn()  # the first call carries one-time host work (allocations, lazy set-up); the second sizes the warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize()
    one_ms = (time.perf_counter() - t0) * 1e3
    warm = int(min(2000, max(3, warm_ms / max(one_ms, 1e-3))))
    for _ in range(warm):
        fn()
    _clock_probe(dev, clk, 0)
    ms = _events_time(fn, iters, 0)
    _clock_probe(dev, clk, 1)
    torch.cuda.synchronize()
    return ms, dict(warmup=warm + 2, clock_mhz=[_clock_mhz(clk, 0), _clock_mhz(clk, 1)])


def _clock_probe(dev, buf, slot):
    """Enqueues the shader-clock probe (20 us spin) on the current stream; its result lands in buf[slot]."""
    from deepgengraph_amd import _lib

    _lib.call("dgg_clock_probe", _lib.ptr(buf[slot]), 2000, _lib.stream_handle(dev))


def _clock_mhz(buf, slot):
    cyc, ticks = buf[slot].tolist()
    return round(cyc / ticks * 100.0, 1) if ticks > 0 else None


def bench_prefill(args, dev):
    from deepgengraph_amd import attention as A
    from deepgengraph_amd import configs as C

    cfg = C.CFG2
    q, k, v, _ = C.attn_inputs(cfg, device=dev)
    out = torch.empty_like(q)
    fn = lambda: A.attention(q, k, v, causal=True, out=out)  # noqa: E731
    clk = torch.zeros(4, 2, dtype=torch.int64, device=dev)
    for _ in range(args.warmup):
        fn()
    _clock_probe(dev, clk, 0)
    # Timed region: K back-to-back steps between two synchronisations. One HIP event pair on the launch stream
    # brackets the same K launches; nothing else runs on the GPU in between, so its elapsed time / K is the
    # kernel's average launch duration (the roofline figure; it also counts whatever gap the GPU leaves between
    # two launches). An event pair around every launch would add ~7 us of its own to each step.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    kern_ms = start.elapsed_time(end) / args.steps
    _clock_probe(dev, clk, 1)
    flops = cfg.reference_flops()
    if args.no_steady:
        return dict(cfg=cfg, wall_ms=wall_ms, kern_ms=kern_ms, flops=flops, exact_flops=cfg.flops(),
                    tflops_wall=flops / (wall_ms * 1e-3) / 1e12, tflops_kern=flops / (kern_ms * 1e-3) / 1e12,
                    clock_mhz=[_clock_mhz(clk, 0), _clock_mhz(clk, 1)], steady=None)
    # steady figure (not `value`): top the launches up to STEADY_WARMUP, then time STEADY_STEPS more
    for _ in range(max(0, STEADY_WARMUP - args.warmup - args.steps)):
        fn()
    _clock_probe(dev, clk, 2)
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record()
    for _ in range(STEADY_STEPS):
        fn()
    s1.record()
    _clock_probe(dev, clk, 3)
    torch.cuda.synchronize()
    steady_ms = s0.elapsed_time(s1) / STEADY_STEPS
    steady = dict(warmup_launches=max(STEADY_WARMUP, args.warmup + args.steps), steps=STEADY_STEPS,
                  kernel_ms=round(steady_ms, 5), tflops=round(flops / (steady_ms * 1e-3) / 1e12, 2),
                  frac=round(flops / (steady_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                  clock_mhz=[_clock_mhz(clk, 2), _clock_mhz(clk, 3)])
    return dict(cfg=cfg, wall_ms=wall_ms, kern_ms=kern_ms, flops=flops, exact_flops=cfg.flops(),
                tflops_wall=flops / (wall_ms * 1e-3) / 1e12, tflops_kern=flops / (kern_ms * 1e-3) / 1e12,
                clock_mhz=[_clock_mhz(clk, 0), _clock_mhz(clk, 1)], steady=steady)


def bench_decode(args, dev):
    from deepgengraph_amd import attention as A
    from deepgengraph_amd import configs as C

    cfg = C.CFG5
    q, kc, vc = C.decode_inputs(cfg, device=dev)
    ws = torch.empty(A.decode_workspace_bytes(cfg.B, cfg.Hq, cfg.D, cfg.splits), dtype=torch.uint8, device=dev)
    out = torch.empty_like(q)
    fn = lambda: A.decode_attention(q, kc, vc, splits=cfg.splits, out=out, workspace=ws)  # noqa: E731
    ms = _events_time(fn, max(5, args.steps // 2), 2)
    nbytes = cfg.bytes()
    del kc, vc, ws
    torch.cuda.empty_cache()
    gbps = nbytes / (ms * 1e-3) / 1e9
    res = dict(workload=cfg.name, ms=round(ms, 4), bytes=nbytes, gbps=round(gbps, 1),
               frac=round(gbps / PEAK_HBM_GBPS, 4), splits=cfg.splits)
    # The same decode through the drop-in compile(Attn) callable: q [B, 1, H, D] and the cache in the case layout
    # [B, L, H, D] (attn.py:18-34 with q_len == 1), routed to the split-KV kernels by attention().
    from deepgengraph_amd import cases as tcases
    from deepgengraph_amd.compile import compile as dgg_compile

    qc = torch.randn(cfg.B, 1, cfg.Hq, cfg.D, device=dev).to(cfg.dtype)
    kcl = torch.randn(cfg.B, cfg.L, cfg.Hkv, cfg.D, device=dev, dtype=cfg.dtype)
    vcl = torch.randn(cfg.B, cfg.L, cfg.Hkv, cfg.D, device=dev, dtype=cfg.dtype)
    model = tcases.Attn(kv_head_num=cfg.Hkv, head_num=cfg.Hq, head_dim=cfg.D)
    f = dgg_compile(model, ["q", "k", "v"], [qc, kcl, vcl], ["out"], "mi355x")
    ms = _events_time(lambda: f(qc, kcl, vcl), max(5, args.steps // 2), 2)
    del kcl, vcl
    torch.cuda.empty_cache()
    gbps = nbytes / (ms * 1e-3) / 1e9
    res["compile_attn_case_layout"] = dict(ms=round(ms, 4), gbps=round(gbps, 1), frac=round(gbps / PEAK_HBM_GBPS, 4),
                                           splits=A.decode_splits(cfg.B, cfg.Hq, cfg.L))
    return res


def bench_prestep(args, dev):
    from deepgengraph_amd import configs as C
    from deepgengraph_amd import ops

    cfg = C.CFG5
    pre = C.decode_prestep_inputs(cfg, device=dev)
    normed = torch.empty_like(pre["x"])
    act = torch.empty(cfg.B, cfg.intermediate, dtype=cfg.dtype, device=dev)
    e = pre["x"].element_size()
    res = {}
    ms = _events_time(lambda: ops.rms_norm(normed, pre["x"], pre["w_norm"], C.LLAMA_EPS), 20, 3)
    nb = e * (2 * pre["x"].numel() + pre["w_norm"].numel())
    res["rms_norm_64x4096_f16"] = dict(us=round(ms * 1e3, 2), gbps=round(nb / (ms * 1e-3) / 1e9, 1))
    ms = _events_time(lambda: ops.silu_and_mul(act, pre["gate_up"]), 20, 3)
    nb2 = e * (pre["gate_up"].numel() + act.numel())
    res["silu_and_mul_64x11008_f16"] = dict(us=round(ms * 1e3, 2), gbps=round(nb2 / (ms * 1e-3) / 1e9, 1))
    # the pre-step as it runs (llama.decode_prestep): both ops in one launch
    ms = _events_time(lambda: ops.rms_norm_silu_and_mul(normed, pre["x"], pre["w_norm"], C.LLAMA_EPS, act,
                                                        pre["gate_up"]), 20, 3)
    res["prestep_one_launch_f16"] = dict(us=round(ms * 1e3, 2), gbps=round((nb + nb2) / (ms * 1e-3) / 1e9, 1))
    # config-2 sized elementwise kernels (bandwidth-meaningful sizes)
    x = torch.randn(4096, 4096, device=dev).bfloat16()
    w = torch.ones(4096, device=dev).bfloat16()
    y = torch.empty_like(x)
    ms = _events_time(lambda: ops.rms_norm(y, x, w, 1e-6), 20, 3)
    nb = 2 * (2 * x.numel() + w.numel())
    res["rms_norm_4096x4096_bf16"] = dict(us=round(ms * 1e3, 2), gbps=round(nb / (ms * 1e-3) / 1e9, 1),
                                          frac=round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4))
    qkv = torch.randn(4096, 3 * 4096, device=dev).bfloat16()
    pos = torch.arange(4096, dtype=torch.int32, device=dev)
    ms = _events_time(
        lambda: ops.rotary_embedding_online(pos, qkv[:, :4096], qkv[:, 4096:8192], 128, 1e4), 20, 3)
    nb = 2 * 2 * (2 * 4096 * 4096) + 4 * 4096
    res["rotary_4096tok_32+32heads_bf16"] = dict(us=round(ms * 1e3, 2), gbps=round(nb / (ms * 1e-3) / 1e9, 1),
                                                 frac=round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4))
    gu = torch.randn(4096, 2 * 11008, device=dev).bfloat16()
    a = torch.empty(4096, 11008, device=dev, dtype=torch.bfloat16)
    ms = _events_time(lambda: ops.silu_and_mul(a, gu), 20, 3)
    nb = 2 * (gu.numel() + a.numel())
    res["silu_and_mul_4096x11008_bf16"] = dict(us=round(ms * 1e3, 2), gbps=round(nb / (ms * 1e-3) / 1e9, 1),
                                               frac=round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4))
    return res


def bench_variants(args, dev):
    from deepgengraph_amd import attention as A
    from deepgengraph_amd import configs as C

    res = {}
    cfg = C.CFG3
    q, k, v, _ = C.attn_inputs(cfg, device=dev)
    ms, info = _variant(lambda: A.attention(q, k, v, causal=True, softcap=cfg.softcap, window=cfg.window), 10)
    res["cfg3_gemma2"] = dict(ms=round(ms, 4), tflops=round(cfg.flops() / (ms * 1e-3) / 1e12, 1),
                              frac=round(cfg.flops() / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4), **info)
    del q, k, v
    cfg = C.CFG4
    q, k, v, _ = C.attn_inputs(cfg, device=dev)
    ms, info = _variant(lambda: A.topk_indices(A.h2o_attention(q, k, v)[1], cfg.topk), 5)
    res["cfg4_h2o_fwd_colsum_topk"] = dict(ms=round(ms, 4),
                                           tflops=round(cfg.reference_flops() / (ms * 1e-3) / 1e12, 1),
                                           frac=round(cfg.reference_flops() / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                                           **info)
    cs = A.h2o_attention(q, k, v)[1]
    ms, info = _variant(lambda: A.topk_indices(cs, cfg.topk), 20)
    ms_t, _ = _variant(lambda: torch.topk(cs, k=cfg.topk, dim=-1, sorted=True)[1].sort(dim=-1)[0], 20)
    res["cfg4_topk256"] = dict(us=round(ms * 1e3, 2), torch_us=round(ms_t * 1e3, 2), **info)
    del cs
    # the other selection cases of the reference at config-4 shapes (same inputs; Corm's threshold 1/(i+1))
    thr = torch.ones(cfg.Sq, cfg.Sk, device=dev) / torch.arange(1, cfg.Sq + 1, device=dev, dtype=torch.float32)[:, None]
    for name, fn in (("cfg4_roco", lambda: A.roco_attention(q, k, v)),
                     ("cfg4_snapkv", lambda: A.snapkv_attention(q, k, v)),
                     ("cfg4_corm", lambda: A.corm_attention(q, k, v, thr))):
        ms, info = _variant(fn, 5)
        res[name] = dict(ms=round(ms, 4), tflops=round(cfg.reference_flops() / (ms * 1e-3) / 1e12, 1), **info)
    # KeyFormer (kf.py): exp_rand [1, 32, 4096, 4096] fp32 (1 + |N(0,1)|, kf.py:48); its causal half is read twice
    # (row lse pass, column pass)
    er = 1 + torch.randn(cfg.B, cfg.Hq, cfg.Sq, cfg.Sk, device=dev).abs()
    ms, info = _variant(lambda: A.keyformer_attention(q, k, v, er), 5)
    er_bytes = 2 * cfg.B * cfg.Hq * (cfg.Sq * (cfg.Sq + 1) // 2) * 4
    res["cfg4_keyformer"] = dict(ms=round(ms, 4), tflops=round(cfg.reference_flops() / (ms * 1e-3) / 1e12, 1),
                                 exp_rand_gbps=round(er_bytes / (ms * 1e-3) / 1e9, 1), **info)
    del er
    # RoCo's selection (models/roco.py:54-61) over the config-4 column sums with the e2e model's budget (512) and
    # recent window (256): the fused kernel against the reference's torch lines on the same GPU
    _, s1, s2 = A.roco_attention(q, k, v)
    S = cfg.Sk

    def roco_torch():
        std = torch.sqrt(s2 / S - (s1 / S) ** 2)
        other = torch.topk(std, largest=False, k=S - 256, dim=-1)[1]
        recent = torch.topk(std, largest=True, k=256, dim=-1)[1]
        pick = torch.topk(s1.gather(dim=-1, index=other) / S, dim=-1, k=512)[1]
        return torch.cat([other.gather(dim=-1, index=pick), recent], dim=-1).sort(dim=-1)[0]

    ms, info = _variant(lambda: A.roco_select(s1, s2, S, 256, 512), 20)
    ms_t, _ = _variant(roco_torch, 20)
    nb = 2 * s1.numel() * 4 + s1.numel() // S * 768 * 8  # both sums read once, 768 indices written per row
    res["cfg4_roco_select"] = dict(us=round(ms * 1e3, 2), gbps=round(nb / (ms * 1e-3) / 1e9, 1),
                                   torch_us=round(ms_t * 1e3, 2), **info)
    del s1, s2
    idx = A.topk_indices(A.h2o_attention(q, k, v)[1], cfg.topk)
    ms, info = _variant(lambda: A.kv_gather(k, v, idx), 20)
    nb = 2 * 2 * idx.numel() * cfg.D * k.element_size()  # K and V rows read once and written once
    res["cfg4_kv_gather_top256"] = dict(us=round(ms * 1e3, 2), gbps=round(nb / (ms * 1e-3) / 1e9, 1), **info)
    return res


def bench_splitkv(args, dev):
    """Short query blocks over a long cache (attn.py:18-34 with q_len 4 / 16 over 32K keys, as in chunked prefill
    and speculative decode) and grouped-query decode (16 query heads over 8 KV heads, roco.py:25-27): each call runs
    the split-KV kernels. Rate = algorithmic bytes (K and V read once, q and o) per call."""
    from deepgengraph_amd import attention as A

    res = {}
    H, D, L = 32, 128, 32768
    for Sq, dt in ((4, torch.float16), (16, torch.bfloat16)):
        g = torch.Generator(device=dev).manual_seed(Sq)
        q = torch.randn(1, Sq, H, D, generator=g, device=dev).to(dt)
        k = torch.randn(1, L, H, D, generator=g, device=dev).to(dt)
        v = torch.randn(1, L, H, D, generator=g, device=dev).to(dt)
        out = torch.empty_like(q)
        ms, info = _variant(lambda: A.attention(q, k, v, causal=True, out=out), 20)
        nb = 2 * (2 * k.numel() + 2 * q.numel())
        gbps = nb / (ms * 1e-3) / 1e9
        res[f"qlen{Sq}_kv{L}_h{H}_d{D}"] = dict(us=round(ms * 1e3, 2), gbps=round(gbps, 1),
                                                 frac=round(gbps / PEAK_HBM_GBPS, 4),
                                                 splits=A.splitkv_splits(1, Sq, H, H, L), **info)
        del q, k, v, out
    B, Hq, Hkv = 64, 16, 8
    g = torch.Generator(device=dev).manual_seed(7)
    q = torch.randn(B, Hq, D, generator=g, device=dev).half()
    kc = torch.randn(B, Hkv, L, D, generator=g, device=dev).half()
    vc = torch.randn(B, Hkv, L, D, generator=g, device=dev).half()
    splits = 8  # best of 8 .. 128 in a sweep on MI355X (6.13 vs 5.80 TB/s at 64)
    ws = torch.empty(A.decode_workspace_bytes(B, Hq, D, splits), dtype=torch.uint8, device=dev)
    out = torch.empty_like(q)
    ms, info = _variant(lambda: A.decode_attention(q, kc, vc, splits=splits, out=out, workspace=ws), 10)
    nb = 2 * (2 * kc.numel() + 2 * q.numel())
    gbps = nb / (ms * 1e-3) / 1e9
    res[f"gqa_decode_b{B}_h{Hq}/{Hkv}_kv{L}_d{D}_f16"] = dict(ms=round(ms, 4), gbps=round(gbps, 1),
                                                             frac=round(gbps / PEAK_HBM_GBPS, 4), splits=splits,
                                                             **info)
    del q, kc, vc, ws, out
    torch.cuda.empty_cache()
    return res


def bench_longsel(args, dev):
    """H2O / SnapKV top-256 (models/h2o.py:51-52) and RoCo's selection (models/roco.py:54-61) over rows longer than
    65536 keys (32 heads, long-context KV caches): the multi-workgroup radix select, against torch.topk + sort on the
    same GPU."""
    from deepgengraph_amd import attention as A

    res = {}
    for n in (131072, 1048576):
        g = torch.Generator(device=dev).manual_seed(n)
        cs = torch.rand(32, n, generator=g, device=dev)
        ms, info = _variant(lambda: A.topk_indices(cs, 256), 10)
        ms_t, _ = _variant(lambda: torch.topk(cs, k=256, dim=-1, sorted=True)[1].sort(dim=-1)[0], 10)
        res[f"topk256_32x{n}"] = dict(us=round(ms * 1e3, 2), gbps=round(cs.numel() * 4 / (ms * 1e-3) / 1e9, 1),
                                      torch_us=round(ms_t * 1e3, 2), **info)
    n = 131072
    s1 = torch.rand(32, n, device=dev) * 64
    s2 = s1 * s1 / 4096 + torch.rand(32, n, device=dev)
    ms, info = _variant(lambda: A.roco_select(s1, s2, 4096, 256, 512), 10)
    res[f"roco_select_32x{n}"] = dict(us=round(ms * 1e3, 2), **info)
    return res


def bench_block(args, dev):
    from deepgengraph_amd import configs as C
    from deepgengraph_amd.llama import LlamaAttentionBlock

    inp = C.llama_block_inputs(device=dev)
    # query rotary inside the attention kernel (the default) or the rotary kernel on q and k: timed in alternation
    # (medians of 6 runs each) so that clock drift does not favour either
    blks = {fuse: LlamaAttentionBlock(inp["w_norm"], inp["w_qkv"], inp["w_o"], heads=32, kv_heads=32,
                                      eps=C.LLAMA_EPS, rope_theta=C.LLAMA_THETA, fuse_rope=fuse)
            for fuse in (True, False)}
    times = {True: [], False: []}
    for i in range(6):
        for fuse in ((True, False) if i % 2 == 0 else (False, True)):
            times[fuse].append(_events_time(lambda: blks[fuse](inp["x"]), 10, 2))
    return dict(ms=round(statistics.median(times[True]), 4), unfused_rope_ms=round(statistics.median(times[False]), 4))


def bench_copycal(args, dev):
    """A plain device copy of known size (256 MiB read + 256 MiB written): the reference point that scales the
    FETCH_SIZE / WRITE_SIZE counters of the profiled kernels to bytes."""
    n = 256 * 1024 * 1024
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    ms = _events_time(lambda: dst.copy_(src), 5, 1)
    return dict(bytes_read=n, bytes_written=n, ms=round(ms, 4), gbps=round(2 * n / (ms * 1e-3) / 1e9, 1))


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter summary (profiles/traffic.json):
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of the kernel, each divided by the same counter's reading for
    the calibration copy and multiplied by the copy's known byte count. None if not measured."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        k, cal = t["kernels"][kernel], t["copy_calibration"]
        rd = k["FETCH_SIZE_KiB"] / cal["FETCH_SIZE_KiB"] * cal["bytes_read"]
        wr = k["WRITE_SIZE_KiB"] / cal["WRITE_SIZE_KiB"] * cal["bytes_written"]
        return int(rd + wr)
    except (OSError, KeyError, ValueError, ZeroDivisionError):
        return None


def cpu_baseline(target_s: float = 10.0):
    """Oracle (reference formula, PyTorch eager on the host CPU) on config 2's attention (all 32 heads, full
    sequence), repeated until ~target_s seconds of CPU work; the median run is reported."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from deepgengraph_amd import configs as C
    from oracle import attention as oa

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    heads = 32
    q, k, v, _ = C.attn_inputs(C.CFG2)
    oa.attention(q[:, :256], k[:, :256], v[:, :256])  # warm-up
    times, t_start = [], time.perf_counter()
    while (time.perf_counter() - t_start < target_s and len(times) < 200) or len(times) < 1:
        t0 = time.perf_counter()
        oa.attention(q, k, v, causal=True)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    flops = 4.0 * 1 * heads * 4096 * 4096 * 128 / 2
    return {"value": round(flops / t / 1e12, 5), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"config 2 attention (B=1, H={heads}, S=4096, D=128, bf16, causal), median of "
                                      f"{len(times)} runs ({t:.3f} s each), same FLOP model",
            "cpu": platform.processor() or platform.machine()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--sections", default="prefill,decode,splitkv,prestep,variants,longsel,block")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-steady", action="store_true", help="skip the steady-clock figure (short profiled runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this build measures one GPU only (the attention hot path runs on a single GPU; multi-GPU "
              f"sharding is not built); --gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    sections = set(args.sections.split(","))
    extra = {}
    pre = bench_prefill(args, dev)
    cfg = pre["cfg"]
    if "decode" in sections:
        extra["decode"] = bench_decode(args, dev)
    if "splitkv" in sections:
        extra["splitkv"] = bench_splitkv(args, dev)
    if "prestep" in sections:
        extra["elementwise"] = bench_prestep(args, dev)
    if "variants" in sections:
        extra["variants"] = bench_variants(args, dev)
    if "longsel" in sections:
        extra["long_selection"] = bench_longsel(args, dev)
    if "block" in sections:
        blk = bench_block(args, dev)
        extra["cfg2_block_ms"] = blk["ms"]
        extra["cfg2_block_unfused_rope_ms"] = blk["unfused_rope_ms"]
    if "copycal" in sections:
        extra["copy_calibration"] = bench_copycal(args, dev)
    line = {
        "metric": METRIC,
        "value": round(pre["tflops_wall"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["wall_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "cfg2_llama2_7b_prefill_attention", "B": cfg.B, "S": cfg.Sq, "H": cfg.Hq,
                   "D": cfg.D, "causal": True, "flop_model": "4*B*H*S^2*D/2 (run_kernel.py:24)",
                   "flops_per_step": pre["flops"], "exact_pair_flops": pre["exact_flops"]},
        "roofline": {"bound": "mfma", "achieved": round(pre["tflops_kern"], 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(pre["tflops_kern"] / PEAK_BF16_TFLOPS, 4),
                     "traffic": measured_traffic("attn_fwd_dma_kernel<BF16, 128"), "kernel_ms": round(pre["kern_ms"], 5)},
        "clock_mhz": pre["clock_mhz"],
        "steady": pre["steady"],
    }
    line.update(extra)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
