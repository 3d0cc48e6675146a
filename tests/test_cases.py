"""The harness's 'torch' system (deepgengraph_amd.cases: the reference's eager case modules) against the oracle
on the CPU, and the harness report helpers."""
import pytest
import torch

from conftest import assert_close
from deepgengraph_amd import cases
from deepgengraph_amd.run_kernel import loss
from oracle import cases as ocases


@pytest.mark.parametrize("name", sorted(cases.KERNEL_ZOO))
def test_torch_system_matches_oracle_cases(name):
    kw = dict(kv_head_num=2, head_num=2, head_dim=16)
    model = cases.KERNEL_ZOO[name](**kw)
    ref_model = getattr(ocases, model.__class__.__name__)(**kw)
    spec = model.prepare(q_len=70, kv_len=70, dtype=torch.float16, device="cpu", seed=3)
    assert spec["output"] == list(ref_model.OUTPUTS)
    ins = list(spec["input"].values())
    outs, refs = model(*ins), ref_model(*ins)
    outs = outs if isinstance(outs, tuple) else (outs,)
    refs = refs if isinstance(refs, tuple) else (refs,)
    for o, r in zip(outs, refs):
        assert o.shape == r.shape and o.dtype == r.dtype
        if o.dtype == torch.bool:
            assert torch.equal(o, r)
        else:
            assert_close(o.float(), r.float(), 1e-3, 1e-3, f"{name} torch system vs oracle")


def test_loss_report_fields():
    a = torch.tensor([1.0, 2.0, 4.0])
    r = loss(a, torch.tensor([1.0, 2.0, 5.0]))
    assert set(r) == {"abs_max", "abs_mean", "rel_max", "rel_mean", "nz_rel_max", "nz_rel_mean", "mse", "rmse"}
    assert r["abs_max"] == 1.0 and abs(r["rel_max"] - 0.2) < 1e-12
    assert loss(torch.tensor([True, False]), torch.tensor([True, True])) == {"err_num": 1, "err": 0.5}
