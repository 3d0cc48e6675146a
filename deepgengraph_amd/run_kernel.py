"""Kernel harness with the reference's CLI (run_kernel.py:29-119):

    python -m deepgengraph_amd.run_kernel -m attn -s mi355x --seqlen 4096 [--check/--no-check] [--show_result]

Builds the case of KERNEL_ZOO (deepgengraph_amd.cases), its seeded inputs (prepare(), fp16 by default) and the
callable of compile(model, input_names, inputs, output_names, system); prints the same report lines as the
reference: gflops (4*B*H*S^2*D/2, run_kernel.py:24) and peak MiB of one call, then with --check the median
speedup over the 'torch' system (7 timed pairs) and per-output losses (utils.py:85-133: allclose(1e-2) flag,
abs / rel / nz-rel max and mean, mse, rmse; error counts for integer and bool outputs). Systems: 'mi355x'
(alias 'our', the HIP kernels of this build) and 'torch' (the eager modules).
"""
from __future__ import annotations

import argparse
import math
import random

import numpy as np
import torch

from .cases import KERNEL_ZOO
from .compile import compile as dgg_compile


def gflops_and_mib(seqlen, f, *args):
    torch.cuda.reset_peak_memory_stats()
    torch.cuda.empty_cache()
    start = torch.cuda.max_memory_allocated() / 1024 / 1024
    print(f"start_peak_mem_mib={start}", flush=True)
    f(*args)
    end = torch.cuda.max_memory_allocated() / 1024 / 1024
    print(f"end_peak_mem_mib={end}", flush=True)
    return 4 * 1 * 32 * seqlen * seqlen * 128 * 1e-9 / 2, end


def loss(out, ref) -> dict:
    if out.dtype != ref.dtype or out.shape != ref.shape:
        raise AssertionError(f"output mismatch: {out.dtype} {tuple(out.shape)} vs {ref.dtype} {tuple(ref.shape)}")
    out, ref = out.cpu(), ref.cpu()
    if out.dtype in (torch.int32, torch.int64, torch.bool):
        err = torch.sum(out != ref).item()
        return {"err_num": err, "err": err / max(out.numel(), 1)}
    d = out.double() - ref.double()
    rel = (d / ref.double()).abs()
    nz = ref != 0
    nzrel = (d[nz] / ref.double()[nz]).abs()
    mse = torch.mean(d * d).item()
    return {"abs_max": d.abs().max().item(), "abs_mean": d.abs().mean().item(), "rel_max": rel.max().item(),
            "rel_mean": rel.mean().item(), "nz_rel_max": nzrel.max().item() if nzrel.numel() else 0.0,
            "nz_rel_mean": nzrel.mean().item() if nzrel.numel() else 0.0, "mse": mse, "rmse": math.sqrt(mse)}


def compare(outs, refs, names):
    if not isinstance(outs, (list, tuple)):
        outs, refs = [outs], [refs]
    for out, ref, name in zip(outs, refs, names):
        ok = torch.equal(out.cpu(), ref.cpu()) if out.dtype == torch.bool else torch.allclose(
            out.float(), ref.float(), rtol=1e-2, atol=1e-2, equal_nan=True)
        print(f"[D] ---- isCorrect : {ok}", flush=True)
        print(f"{name} loss: {loss(out, ref)}", flush=True)


def display(outs, refs, names):
    if not isinstance(outs, (list, tuple)):
        outs, refs = [outs], [refs]
    for out, ref, name in zip(outs, refs, names):
        print(f"{name}:\n out {out}\n ref {ref}", flush=True)


def _time(f) -> float:
    st, et = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    f()
    et.record()
    torch.cuda.synchronize()
    return st.elapsed_time(et)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--model", "-m", default="attn", help="Model name")
    ap.add_argument("--system", "-s", default="mi355x", help="System name")
    ap.add_argument("--seqlen", type=int, default=4096, help="seqlen")
    ap.add_argument("--show_result", action="store_true", help="show result")
    ap.add_argument("--check", dest="check", action="store_true", default=True, help="check result with torch")
    ap.add_argument("--no-check", dest="check", action="store_false")
    a = ap.parse_args(argv)
    print(f"model={a.model!r} system={a.system!r} seqlen={a.seqlen}")
    if a.model not in KERNEL_ZOO:
        raise SystemExit(f"model {a.model} not found in KERNEL_ZOO {list(KERNEL_ZOO)}")
    torch.manual_seed(0)
    random.seed(0)
    np.random.seed(0)
    model = KERNEL_ZOO[a.model]().eval()
    specs = model.prepare(q_len=a.seqlen, kv_len=a.seqlen, device="cuda")
    input_names = list(specs["input"].keys())
    inputs = [specs["input"][n] for n in input_names]
    output_names = specs["output"]
    print(f"input_names={input_names}")
    print(f"output_names={output_names}")
    print(f"check={a.check}")
    f = dgg_compile(model=model, input_names=input_names, inputs=inputs, output_names=output_names, system=a.system)
    gflops, mib = gflops_and_mib(a.seqlen, f, *inputs)
    print(f"gflops={gflops}", flush=True)
    print(f"mib={mib}", flush=True)
    if a.check:
        print(f"checking {a.system}...")
        t_ours, t_base = [], []
        for _ in range(7):
            t_base.append(_time(lambda: model(*inputs)))
            t_ours.append(_time(lambda: f(*inputs)))
        print(f"[D] --- speedup = {np.median(t_base) / np.median(t_ours)}", flush=True)
        print(f"[D] --- {a.system} median {np.median(t_ours):.4f} ms, torch median {np.median(t_base):.4f} ms",
              flush=True)
        refs = model(*inputs)
        outs = f(*inputs)
        torch.cuda.synchronize()
        compare(outs, refs, output_names)
        if a.show_result:
            display(outs, refs, output_names)


if __name__ == "__main__":
    main()
