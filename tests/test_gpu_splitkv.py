"""GPU parity of the split-KV attention kernels (short query blocks over long key ranges, and grouped-query decode)
against the CPU oracle: Attn.forward / Gemma2.forward with 1 <= q_len << kv_len under the bottom-right causal mask
(attn.py:18-34, gemma2.py:19-38), the GQA convention of roco.py:25-27, a sliding window and the soft-cap; through
splitkv_attention with explicit split counts, through attention() (which routes these shapes to the split-KV kernels),
through compile(Attn) and through decode_attention for grouped query heads."""
import pytest
import torch

from conftest import assert_close, progress
from deepgengraph_amd import attention as A
from deepgengraph_amd import cases
from deepgengraph_amd.compile import compile as dgg_compile
from oracle import attention as oa

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (1e-2, 5e-3)}


def _qkv(B, Sq, Sk, Hq, Hkv, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Sq, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, Sk, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, Sk, Hkv, D, generator=g).to(dtype)
    return q, k, v


@pytest.mark.parametrize("B,Sq,Sk,Hq,Hkv,D,causal,window,softcap,dtype,splits", [
    (1, 4, 2048, 4, 4, 128, True, 0, 0.0, torch.float16, None),
    (2, 16, 1500, 4, 4, 128, True, 0, 0.0, torch.bfloat16, 7),       # ragged slices
    (1, 2, 700, 8, 2, 128, True, 0, 0.0, torch.float16, 3),          # GQA, 8 rows per KV head
    (1, 5, 1000, 16, 2, 64, True, 0, 0.0, torch.bfloat16, 5),        # 40 rows: two waves
    (1, 64, 3000, 2, 1, 128, True, 0, 0.0, torch.float16, 11),       # 128 rows: two row groups
    (2, 3, 1200, 4, 2, 256, True, 0, 0.0, torch.bfloat16, 4),
    (1, 8, 2000, 4, 4, 128, True, 300, 0.0, torch.float16, 6),       # sliding window
    (1, 8, 2000, 8, 4, 256, True, 900, 30.0, torch.bfloat16, 9),     # window + soft-cap + GQA
    (1, 16, 1024, 4, 4, 64, False, 0, 0.0, torch.float16, 8),        # no mask
    (1, 33, 500, 2, 2, 128, True, 0, 0.0, torch.bfloat16, 1),        # one slice
    (1, 4, 100, 2, 2, 128, True, 0, 0.0, torch.float16, 64),         # more slices than keys: empty slices
    (1, 40, 32, 2, 2, 128, True, 0, 0.0, torch.float16, 2),          # Sq > Sk: the first rows see no key (NaN)
])
def test_splitkv_matches_oracle(gpu, B, Sq, Sk, Hq, Hkv, D, causal, window, softcap, dtype, splits):
    q, k, v = _qkv(B, Sq, Sk, Hq, Hkv, D, dtype, 11 + Sq + Sk + D)
    what = f"splitkv B{B} Sq{Sq} Sk{Sk} H{Hq}/{Hkv} D{D} causal{causal} w{window} sc{softcap} {dtype} splits{splits}"
    progress(what)
    ref, ref_lse = oa.attention(q, k, v, causal=causal, window=window or None, softcap=softcap or None,
                                return_lse=True)
    out, lse = A.splitkv_attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal, window=window, softcap=softcap,
                                   return_lse=True, splits=splits)
    assert_close(out.cpu().float(), ref.float(), *TOL[dtype], what)
    assert_close(lse.cpu(), ref_lse, 2e-2, 1e-3, what + " lse")
    _, lse2 = A.splitkv_attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal, window=window, softcap=softcap,
                                  return_lse=True, lse_base2=True, splits=splits)
    assert_close(lse2.cpu(), ref_lse * 1.4426950408889634, 3e-2, 1e-3, what + " lse base 2")


def test_splitkv_slice_count_independent(gpu):
    q, k, v = _qkv(1, 12, 4000, 4, 2, 128, torch.bfloat16, 5)
    q, k, v = q.to(gpu), k.to(gpu), v.to(gpu)
    base, base_lse = A.splitkv_attention(q, k, v, splits=1, return_lse=True)
    for s in (2, 13, 125, 1024):
        out, lse = A.splitkv_attention(q, k, v, splits=s, return_lse=True)
        assert_close(out.float().cpu(), base.float().cpu(), 1e-2, 1e-2, f"splits={s}")
        assert_close(lse.cpu(), base_lse.cpu(), 1e-4, 1e-5, f"splits={s} lse")


@pytest.mark.parametrize("Sq,dtype", [(4, torch.float16), (16, torch.bfloat16)])
def test_attn_case_short_query_long_cache(gpu, Sq, dtype):
    # compile(Attn) with q_len 4 / 16 over 32K keys (chunked prefill / speculative decode shapes): attention() routes
    # them to the split-KV kernels; every head against the oracle
    Sk, H, D = 32768, 32, 128
    model = cases.Attn(kv_head_num=H, head_num=H, head_dim=D)
    inp = model.prepare(batch_size=1, q_len=Sq, kv_len=Sk, dtype=dtype, device="cpu", seed=3)["input"]
    q, k, v = inp["q"], inp["k"], inp["v"]
    assert A._splitkv_shaped(Sq, Sk, H, H, False, dtype)
    f = dgg_compile(model, ["q", "k", "v"], [q, k, v], ["out"], "mi355x")
    out = f(q.to(gpu), k.to(gpu), v.to(gpu)).cpu()
    progress(f"Attn q_len {Sq} over {Sk} keys: GPU done")
    ref = oa.attention(q, k, v, causal=True)
    assert_close(out.float(), ref.float(), *TOL[dtype], f"Attn q_len {Sq} kv_len {Sk}")


@pytest.mark.parametrize("B,Hq,Hkv,L,D,dtype,splits", [
    (4, 16, 8, 32768, 128, torch.float16, 64),    # the GQA shape of the Gemma-2 config, one query token
    (2, 32, 4, 5000, 128, torch.bfloat16, 37),    # group 8
    (3, 12, 3, 999, 64, torch.float16, 8),        # group 4, ragged slices
])
def test_gqa_decode(gpu, B, Hq, Hkv, L, D, dtype, splits):
    g = torch.Generator().manual_seed(L + Hq)
    q = torch.randn(B, Hq, D, generator=g).to(dtype)
    kc = torch.randn(B, Hkv, L, D, generator=g).to(dtype)
    vc = torch.randn(B, Hkv, L, D, generator=g).to(dtype)
    ref, ref_lse = oa.decode(q, kc, vc)
    out, lse = A.decode_attention(q.to(gpu), kc.to(gpu), vc.to(gpu), splits=splits, return_lse=True)
    what = f"GQA decode B{B} H{Hq}/{Hkv} L{L} D{D} {dtype} splits{splits}"
    assert_close(out.cpu().float(), ref.float(), *TOL[dtype], what)
    assert_close(lse.cpu(), ref_lse, 2e-2, 1e-3, what + " lse")
    # the case layout [B, L, Hkv, D] through attention() with one query row
    out2 = A.attention(q.to(gpu).unsqueeze(1), kc.to(gpu).transpose(1, 2), vc.to(gpu).transpose(1, 2), causal=True)
    assert_close(out2.squeeze(1).cpu().float(), ref.float(), *TOL[dtype], what + " via attention()")


def test_splitkv_rejects_reference_rounding_and_small_workspace(gpu):
    from deepgengraph_amd import _lib

    q, k, v = _qkv(1, 4, 512, 2, 2, 128, torch.float16, 1)
    q, k, v = q.to(gpu), k.to(gpu), v.to(gpu)
    o = torch.empty_like(q)
    st = _lib.int64_array([*q.stride()[:3], *k.stride()[:3], *v.stride()[:3], *o.stride()[:3]])
    need = int(_lib.load().dgg_attn_splitkv_workspace_bytes(1, 4, 2, 128, 4))
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    args = lambda wsb, flags: (_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), None, _lib.ptr(ws), wsb, 1, 4, 512,
                               2, 2, 128, st, 4, 0.088, 0.0, 0, flags, _lib.DGG_F16, _lib.stream_handle(gpu))
    with pytest.raises(RuntimeError, match="reference rounding"):
        _lib.call("dgg_attn_splitkv", *args(need, _lib.ATTN_CAUSAL | _lib.ATTN_REF_ROUNDING))
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.call("dgg_attn_splitkv", *args(need - 4, _lib.ATTN_CAUSAL))
    _lib.call("dgg_attn_splitkv", *args(need, _lib.ATTN_CAUSAL))
    torch.cuda.synchronize()
    assert_close(o.cpu().float(), oa.attention(q.cpu(), k.cpu(), v.cpu(), causal=True).float(), 1e-2, 5e-3, "raw ABI")
