"""GPU parity of split-KV decode + LSE merge against the CPU oracle (Attn.forward with q_len == 1) and against the
float64 split/merge restatement, including empty splits and GQA."""
import pytest
import torch

from conftest import assert_close
from deepgengraph_amd import attention as A
from oracle import attention as oa

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (1e-2, 5e-3)}


@pytest.mark.parametrize("B,H,Hkv,L,D,splits,dtype", [
    (2, 4, 4, 1000, 128, 7, torch.float16),
    (3, 8, 2, 4096, 128, 64, torch.float16),
    (1, 2, 2, 513, 64, 3, torch.bfloat16),
    (2, 4, 1, 300, 256, 5, torch.bfloat16),
    (1, 2, 2, 5, 128, 16, torch.float16),     # more splits than keys: empty splits
    (1, 1, 1, 1, 128, 1, torch.float16),      # a single key
])
def test_decode_matches_oracle(gpu, B, H, Hkv, L, D, splits, dtype):
    g = torch.Generator().manual_seed(L + D)
    q = torch.randn(B, H, D, generator=g).to(dtype)
    kc = torch.randn(B, Hkv, L, D, generator=g).to(dtype)
    vc = torch.randn(B, Hkv, L, D, generator=g).to(dtype)
    ref, ref_lse = oa.decode(q, kc, vc)
    out, lse = A.decode_attention(q.to(gpu), kc.to(gpu), vc.to(gpu), splits=splits, return_lse=True)
    what = f"decode B{B} H{H}/{Hkv} L{L} D{D} splits{splits} {dtype}"
    assert_close(out.cpu().float(), ref.float(), *TOL[dtype], what)
    assert_close(lse.cpu(), ref_lse, 2e-2, 1e-3, what + " lse")
    o64, l64 = oa.decode_splitkv(q.float(), kc.float(), vc.float(), splits)
    assert_close(out.cpu().float(), torch.from_numpy(o64), *TOL[dtype], what + " vs float64 split-kv")


def test_decode_split_count_independent(gpu):
    g = torch.Generator().manual_seed(9)
    q = torch.randn(2, 4, 128, generator=g).half().to(gpu)
    kc = torch.randn(2, 4, 2048, 128, generator=g).half().to(gpu)
    vc = torch.randn(2, 4, 2048, 128, generator=g).half().to(gpu)
    base = A.decode_attention(q, kc, vc, splits=1).float()
    for s in (2, 16, 64, 1000):
        assert_close(A.decode_attention(q, kc, vc, splits=s).float().cpu(), base.cpu(), 2e-3, 2e-3, f"splits={s}")


def test_decode_strided_cache_and_workspace_reuse(gpu):
    # cache slices of a larger allocation (max length 1024, first 700 used) and a reused workspace
    g = torch.Generator().manual_seed(10)
    full_k = torch.randn(2, 4, 1024, 128, generator=g).half()
    full_v = torch.randn(2, 4, 1024, 128, generator=g).half()
    q = torch.randn(2, 4, 128, generator=g).half()
    ref, _ = oa.decode(q, full_k[:, :, :700], full_v[:, :, :700])
    ws = torch.empty(A.decode_workspace_bytes(2, 4, 128, 8), dtype=torch.uint8, device=gpu)
    kg, vg = full_k.to(gpu), full_v.to(gpu)
    for _ in range(2):
        out = A.decode_attention(q.to(gpu), kg[:, :, :700], vg[:, :, :700], splits=8, workspace=ws)
        assert_close(out.cpu().float(), ref.float(), 1e-2, 5e-3, "strided cache")
    with pytest.raises(RuntimeError, match="workspace"):
        A.decode_attention(q.to(gpu), kg, vg, splits=8, workspace=ws[:100])
