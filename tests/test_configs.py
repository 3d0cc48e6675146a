"""Algorithmic work figures of the benchmark configurations (no GPU)."""
import math

from deepgengraph_amd import configs as C


def test_config_work_figures():
    # the algorithmic work each benchmark line divides by
    assert C.CFG2.reference_flops() == 4 * 32 * 4096 * 4096 * 128 / 2
    assert C.CFG3.pairs_per_head() == 25_167_872
    assert abs(C.CFG3.flops() - 824.70e9) < 0.01e9
    assert C.CFG5.bytes() == 34_360_786_944
    assert math.isclose(C.CFG2.scale, 1 / math.sqrt(128))
