"""The run_kernel.py-style harness end to end on the GPU: every case of KERNEL_ZOO compiled for the mi355x system,
checked against the torch system with the reference's report lines."""
import contextlib
import io

import pytest

from conftest import progress
from deepgengraph_amd import cases
from deepgengraph_amd.run_kernel import main

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", sorted(cases.KERNEL_ZOO))
def test_run_kernel_cli(gpu, name):
    progress(f"run_kernel -m {name}")
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        main(["-m", name, "-s", "mi355x", "--seqlen", "384"])
    text = buf.getvalue()
    assert "gflops=" in text and "speedup = " in text, text
    flags = [line for line in text.splitlines() if "isCorrect" in line]
    n_out = len(cases.KERNEL_ZOO[name].OUTPUTS)
    assert len(flags) == n_out and all(line.endswith("True") for line in flags), text
