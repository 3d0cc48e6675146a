import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")
    config.addinivalue_line("markers", "slow: full-size configuration checks")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from deepgengraph_amd import _lib

    _lib.load()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")


def progress(msg):
    """Progress line for long tests (visible with pytest -s)."""
    print(f"[progress] {msg}", flush=True)


def load_golden(name):
    import numpy as np

    with np.load(GOLDEN / f"{name}.npz") as z:
        return {k: z[k] for k in z.files}


def assert_close(out, ref, atol, rtol, what=""):
    """allclose-style check |out - ref| <= atol + rtol * |ref| with a readable failure report (max errors and
    the worst element), in the spirit of the reference's loss() report (deepgengraph_exp/utils.py:85-118).
    NaN must match NaN."""
    import torch

    out = torch.as_tensor(out).double().cpu()
    ref = torch.as_tensor(ref).double().cpu()
    assert out.shape == ref.shape, f"{what}: shape {tuple(out.shape)} != {tuple(ref.shape)}"
    nan_o, nan_r = torch.isnan(out), torch.isnan(ref)
    assert torch.equal(nan_o, nan_r), f"{what}: NaN pattern differs ({int(nan_o.sum())} vs {int(nan_r.sum())})"
    o, r = out[~nan_r], ref[~nan_r]
    err = (o - r).abs()
    bound = atol + rtol * r.abs()
    bad = err > bound
    if bad.any():
        i = int(torch.argmax(err - bound))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{o.numel()} elements out of tolerance (atol={atol}, rtol={rtol}); "
            f"max abs err {float(err.max()):.3e}, worst: out={float(o[i]):.6g} ref={float(r[i]):.6g}")
