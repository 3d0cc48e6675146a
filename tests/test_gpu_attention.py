"""GPU parity of the prefill attention kernel and the H2O column-sum / top-k path against the CPU oracle on
identical seeded inputs. Tolerances (from the task's north star): bf16 2e-2 abs / 1e-2 rel, fp16 1e-2 / 5e-3,
fp32 column sums 1e-3 rel (with a 1e-6 absolute floor for sums that are themselves ~1e-6), top-k index sets
identical with ties broken by the lowest index."""
import math

import numpy as np
import pytest
import torch

from conftest import assert_close, load_golden, progress
from deepgengraph_amd import attention as A
from deepgengraph_amd.compile import compile as dgg_compile
from oracle import attention as oa
from oracle import cases as ocases
from oracle import selection as osel

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (1e-2, 5e-3)}


def _qkv(B, Sq, Sk, Hq, Hkv, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Sq, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, Sk, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, Sk, Hkv, D, generator=g).to(dtype)
    return q, k, v


def _qkv_sinks(S, H, D, seed, sinks=16, dtype=torch.float16):
    """Self-attention inputs [1, S, H, D] with a few attention-sink keys (scaled up), as the H2O tests draw them."""
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(1, S, H, D, generator=g) for _ in range(3))
    k[:, torch.randperm(S, generator=g)[:sinks]] *= 4.0
    return q.to(dtype), k.to(dtype), v.to(dtype)


CASES = [
    # B, Sq, Sk, Hq, Hkv, D, dtype, causal, softcap, window
    (1, 256, 256, 2, 2, 128, torch.bfloat16, True, 0.0, 0),
    (2, 200, 200, 4, 2, 64, torch.float16, True, 0.0, 0),       # ragged tiles, GQA
    (1, 130, 300, 2, 1, 128, torch.bfloat16, True, 0.0, 0),     # Sq < Sk (bottom-right causal)
    (1, 300, 130, 2, 2, 128, torch.float16, True, 0.0, 0),      # Sq > Sk: first rows see nothing -> NaN
    (1, 192, 192, 2, 2, 256, torch.bfloat16, True, 50.0, 64),   # soft-cap + window, D = 256
    (1, 257, 257, 2, 2, 64, torch.bfloat16, False, 0.0, 0),     # non-causal
    (1, 128, 512, 2, 2, 128, torch.float16, False, 30.0, 0),    # non-causal soft-cap
    (1, 333, 333, 4, 1, 256, torch.float16, True, 0.0, 100),    # window + GQA 4:1
    (3, 64, 64, 1, 1, 128, torch.bfloat16, True, 0.0, 0),       # batch > 1, single tile
    (1, 1, 700, 2, 2, 128, torch.bfloat16, True, 0.0, 0),       # one query row (decode-like)
]


@pytest.mark.parametrize("B,Sq,Sk,Hq,Hkv,D,dtype,causal,softcap,window", CASES)
def test_prefill_matches_oracle(gpu, B, Sq, Sk, Hq, Hkv, D, dtype, causal, softcap, window):
    q, k, v = _qkv(B, Sq, Sk, Hq, Hkv, D, dtype, seed=Sq * 7 + Sk + D)
    ref, ref_lse = oa.attention(q, k, v, causal=causal, softcap=softcap or None, window=window or None,
                                return_lse=True)
    out, lse = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal, softcap=softcap, window=window,
                           return_lse=True)
    what = f"B{B} Sq{Sq} Sk{Sk} H{Hq}/{Hkv} D{D} {dtype} causal={causal} cap={softcap} win={window}"
    assert_close(out.cpu().float(), ref.float(), *TOL[dtype], what + " out")
    lse_c = lse.cpu()
    fin = torch.isfinite(ref_lse)
    assert torch.equal(torch.isfinite(lse_c), fin), what + " lse -inf pattern"
    assert_close(lse_c[fin], ref_lse[fin], 2e-2, 1e-2, what + " lse")


# Grouped-query head_dim-256 launches at sizes where an XCD runs more than one generation of workgroups per KV
# head (the KV-head orders of map_block_kv / map_block_kv_window: more than 32 workgroups per KV head), checked on
# a few whole heads.
GQA_LARGE_CASES = [
    # B, Sq, Sk, Hq, Hkv, dtype, causal, softcap, window
    (1, 2500, 2500, 16, 8, torch.bfloat16, True, 50.0, 1000),   # soft-cap + window, ragged Sk
    (1, 2300, 2333, 16, 8, torch.float16, False, 0.0, 0),       # non-causal, Sq != Sk
    (1, 2200, 2600, 16, 8, torch.bfloat16, True, 0.0, 0),       # bottom-right causal
    # B * Hkv = 16: two KV heads per XCD, a causal window, so both query-tile orders of map_block_kv_window run
    # (ascending for the first KV head of an XCD, whole-window tiles then the shorter ones for the second; head 15
    # reads KV head 7, a second one)
    (2, 1500, 1500, 16, 8, torch.bfloat16, True, 30.0, 600),
    (2, 1400, 1700, 16, 8, torch.float16, True, 0.0, 900),      # Sq < Sk: the window start moves with the offset
]


@pytest.mark.parametrize("B,Sq,Sk,Hq,Hkv,dtype,causal,softcap,window", GQA_LARGE_CASES)
def test_prefill_d256_gqa_large_kv_order(gpu, B, Sq, Sk, Hq, Hkv, dtype, causal, softcap, window):
    D = 256
    q, k, v = _qkv(B, Sq, Sk, Hq, Hkv, D, dtype, seed=Sq + 3 * Sk)
    out = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal, softcap=softcap, window=window).cpu()
    G = Hq // Hkv
    for h in (0, 5, Hq - 1):
        ref = oa.attention(q[:, :, h:h + 1], k[:, :, h // G:h // G + 1], v[:, :, h // G:h // G + 1], causal=causal,
                           softcap=softcap or None, window=window or None)
        what = f"Sq{Sq} Sk{Sk} H{Hq}/{Hkv} {dtype} causal={causal} cap={softcap} win={window} head {h}"
        assert_close(out[:, :, h:h + 1].float(), ref.float(), *TOL[dtype], what)


FAST_CASES = [
    # bf16, head_dim 128, no lse / soft-cap / reference rounding: B, Sq, Sk, Hq, Hkv, causal, window
    (1, 512, 512, 2, 2, True, 0),
    (2, 300, 300, 4, 2, True, 0),       # ragged tiles, GQA, 256-row blocks with a partial second block
    (1, 130, 700, 2, 1, True, 0),       # Sq < Sk: every wave starts mid-sequence
    (1, 700, 130, 2, 2, True, 0),       # Sq > Sk: waves whose rows see no key (NaN rows)
    (1, 1000, 1000, 2, 2, True, 200),   # sliding window: masked tiles on both sides
    (1, 600, 600, 2, 2, False, 100),    # window without causal
    (1, 257, 383, 2, 2, False, 0),      # non-causal, ragged key tile
    (3, 64, 64, 1, 1, True, 0),         # one tile, most waves idle
    (1, 1, 700, 2, 2, True, 0),         # one query row
    (1, 100, 0, 2, 2, False, 0),        # no keys at all
]


@pytest.mark.parametrize("B,Sq,Sk,Hq,Hkv,causal,window", FAST_CASES)
def test_prefill_fast_path_matches_oracle(gpu, B, Sq, Sk, Hq, Hkv, causal, window):
    q, k, v = _qkv(B, Sq, Sk, Hq, Hkv, 128, torch.bfloat16, seed=Sq * 3 + Sk + 11)
    ref = oa.attention(q, k, v, causal=causal, window=window or None)
    out = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal, window=window)
    what = f"fast B{B} Sq{Sq} Sk{Sk} H{Hq}/{Hkv} causal={causal} win={window}"
    got = out.cpu().float()
    nan = torch.isnan(ref.float())
    assert torch.equal(torch.isnan(got), nan), what + " NaN rows"
    assert_close(got[~nan], ref.float()[~nan], *TOL[torch.bfloat16], what)


FP16_NOLSE_CASES = [
    # fp16 without lse: the v_dot2 row-sum instantiation that compile(Attn / Gemma2) runs for the reference's
    # default fp16 inputs. B, Sq, Sk, Hq, Hkv, D, causal, softcap, window
    (1, 512, 512, 2, 2, 128, True, 0.0, 0),
    (2, 300, 300, 4, 2, 128, True, 0.0, 0),      # ragged, GQA
    (1, 130, 700, 2, 2, 128, True, 0.0, 0),      # Sq < Sk
    (1, 700, 130, 2, 2, 128, True, 0.0, 0),      # Sq > Sk: NaN rows
    (1, 384, 384, 2, 2, 128, True, 50.0, 0),     # soft-cap
    (1, 333, 333, 2, 2, 128, True, 30.0, 100),   # soft-cap + window
    (1, 256, 256, 2, 2, 256, True, 0.0, 0),      # head_dim 256
    (1, 333, 517, 4, 2, 256, True, 0.0, 128),    # head_dim 256, window, GQA, Sq < Sk
    (1, 200, 200, 2, 2, 256, True, 50.0, 64),    # head_dim 256, soft-cap + window
    (1, 257, 383, 2, 2, 128, False, 0.0, 0),     # non-causal, ragged key tile
]


@pytest.mark.parametrize("B,Sq,Sk,Hq,Hkv,D,causal,softcap,window", FP16_NOLSE_CASES)
def test_prefill_fp16_no_lse_matches_oracle(gpu, B, Sq, Sk, Hq, Hkv, D, causal, softcap, window):
    q, k, v = _qkv(B, Sq, Sk, Hq, Hkv, D, torch.float16, seed=Sq * 5 + Sk + D + 3)
    ref = oa.attention(q, k, v, causal=causal, softcap=softcap or None, window=window or None)
    out = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal, softcap=softcap, window=window)
    what = f"fp16 no-lse B{B} Sq{Sq} Sk{Sk} H{Hq}/{Hkv} D{D} causal={causal} cap={softcap} win={window}"
    got, want = out.cpu().float(), ref.float()
    nan = torch.isnan(want)
    assert torch.equal(torch.isnan(got), nan), what + " NaN rows"
    assert_close(got[~nan], want[~nan], *TOL[torch.float16], what)


F32_CASES = [
    # B, Sq, Sk, Hq, Hkv, D, causal, softcap, window
    (1, 512, 512, 8, 8, 64, True, 0.0, 0),       # config 1's shape
    (2, 200, 300, 4, 2, 128, True, 0.0, 0),      # GQA, Sq < Sk
    (1, 300, 130, 2, 2, 64, True, 0.0, 0),       # Sq > Sk: NaN rows, lse -inf
    (1, 192, 192, 2, 1, 256, True, 50.0, 64),    # soft-cap + window, head_dim 256
    (1, 100, 170, 2, 2, 128, False, 0.0, 0),     # non-causal
]


@pytest.mark.parametrize("B,Sq,Sk,Hq,Hkv,D,causal,softcap,window", F32_CASES)
def test_prefill_fp32_matches_oracle(gpu, B, Sq, Sk, Hq, Hkv, D, causal, softcap, window):
    q, k, v = _qkv(B, Sq, Sk, Hq, Hkv, D, torch.float32, seed=Sq + Sk + D + 9)
    ref, ref_lse = oa.attention(q, k, v, causal=causal, softcap=softcap or None, window=window or None,
                                return_lse=True)
    out, lse = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal, softcap=softcap, window=window,
                           return_lse=True)
    what = f"fp32 B{B} Sq{Sq} Sk{Sk} H{Hq}/{Hkv} D{D} causal={causal} cap={softcap} win={window}"
    assert out.dtype == torch.float32
    assert_close(out.cpu(), ref, 1e-5, 1e-5, what + " out")
    fin = torch.isfinite(ref_lse)
    assert torch.equal(torch.isfinite(lse.cpu()), fin), what + " lse -inf pattern"
    assert_close(lse.cpu()[fin], ref_lse[fin], 1e-5, 1e-6, what + " lse")


def test_config1_fp32_on_gpu(gpu):
    # config 1 (fp32, B=1, H=8, S=512, D=64) through the C ABI: O and LSE against the oracle, and through the
    # drop-in compile(Attn) callable
    from deepgengraph_amd import configs as C

    cfg = C.CFG1
    q, k, v, _ = C.attn_inputs(cfg)
    ref, ref_lse = oa.attention(q, k, v, causal=True, return_lse=True)
    out, lse = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=True, return_lse=True)
    assert_close(out.cpu(), ref, 1e-5, 1e-5, "config 1 O")
    assert_close(lse.cpu(), ref_lse, 1e-5, 1e-6, "config 1 LSE")
    model = ocases.Attn(kv_head_num=8, head_num=8, head_dim=64)
    f = dgg_compile(model=model, input_names=["q", "k", "v"], inputs=[q, k, v], output_names=["out"],
                    system="mi355x")
    assert_close(f(q.to(gpu), k.to(gpu), v.to(gpu)).cpu(), ref, 1e-5, 1e-5, "config 1 via compile(Attn)")


def test_fp32_column_scores_match_oracle(gpu):
    # fp32 H2O / RoCo / Corm column passes (no 16-bit rounding point: reference rounding changes nothing)
    S, H, D = 300, 2, 64
    g = torch.Generator().manual_seed(21)
    q, k, v = (torch.randn(1, S, H, D, generator=g) for _ in range(3))
    k[:, torch.randperm(S, generator=g)[:5]] *= 4.0
    ref_out, ref_cs, _ = oa.h2o(q, k, v)
    out, cs = A.h2o_attention(q.to(gpu), k.to(gpu), v.to(gpu))
    assert_close(out.cpu(), ref_out, 1e-5, 1e-5, "fp32 h2o out")
    _colsum_check(cs.cpu(), ref_cs, "fp32 h2o colsum")
    _, s1, s2, _ = oa.roco(q, k, v)
    _, g1, g2 = A.roco_attention(q.to(gpu), k.to(gpu), v.to(gpu))
    _colsum_check(g1.cpu(), s1, "fp32 roco sum")
    _colsum_check(g2.cpu(), s2, "fp32 roco sum of squares")
    thr = oa.corm_mask(S, S)
    _, hit, _ = oa.corm(q, k, v, thr)
    _, ghit = A.corm_attention(q.to(gpu), k.to(gpu), v.to(gpu), thr.to(gpu))
    assert torch.equal(ghit.cpu(), hit)


@pytest.mark.parametrize("name,kw,dtype", [
    ("attn_d64_causal_bf16", dict(causal=True), torch.bfloat16),
    ("attn_d64_gqa_softcap_window_bf16", dict(causal=True, softcap=5.0, window=33), torch.bfloat16),
    ("attn_d64_h2o_sinks_f16", dict(causal=True), torch.float16),
])
def test_prefill_golden(gpu, name, kw, dtype):
    g = load_golden(name)
    q, k, v = (torch.from_numpy(g[x]).to(dtype).to(gpu) for x in "qkv")
    out, lse = A.attention(q, k, v, return_lse=True, **kw)
    assert_close(out.cpu().float(), torch.from_numpy(g["out"]), *TOL[dtype], name + " out")
    assert_close(lse.cpu(), torch.from_numpy(g["lse"]), 2e-2, 1e-2, name + " lse")


@pytest.mark.parametrize("B,Sq,Sk,Hq,Hkv,dtype,causal", [
    (1, 512, 512, 4, 4, torch.bfloat16, True),
    (2, 300, 300, 4, 2, torch.float16, True),     # GQA, ragged, batch-major table rows
    (1, 130, 700, 2, 2, torch.bfloat16, True),    # Sq < Sk
    (1, 257, 257, 2, 2, torch.float16, False),
])
def test_prefill_fused_query_rotary_matches_oracle(gpu, B, Sq, Sk, Hq, Hkv, dtype, causal):
    # attention(rope_cos_sin=...) on the unrotated q equals the oracle's rotary (pos_encoding.cu:64-113) of q followed
    # by the oracle attention; k is rotated beforehand as the block does; q is left unmodified
    from oracle import elementwise as oe

    q, k, v = _qkv(B, Sq, Sk, Hq, Hkv, 128, dtype, seed=Sq + 31 * Sk)
    pos = torch.arange(Sq, dtype=torch.int32).repeat(B) + (Sk - Sq)  # the query rows' positions
    q_rot, _ = oe.rotary_embedding_online(pos, q.reshape(B * Sq, Hq * 128), None, 128, 10000.0)
    ref = oa.attention(q_rot.view(B, Sq, Hq, 128), k, v, causal=causal)
    qg = q.to(gpu)
    cs = A.rotary_cos_sin(pos.to(gpu).contiguous(), 128, 10000.0)
    out = A.attention(qg, k.to(gpu), v.to(gpu), causal=causal, rope_cos_sin=cs)
    what = f"fused rotary B{B} Sq{Sq} Sk{Sk} H{Hq}/{Hkv} {dtype} causal={causal}"
    assert_close(out.cpu().float(), ref.float(), *TOL[dtype], what)
    assert torch.equal(qg.cpu(), q), "q must not be modified"
    # against the unfused GPU path (the rotary kernel on q, then attention): the table holds the rotary kernel's
    # own angles, so the two differ at most by the rounding of a multiply-add
    from deepgengraph_amd import ops

    q2 = qg.clone()
    ops.rotary_embedding_online(pos.to(gpu).contiguous(), q2.view(B * Sq, Hq * 128), None, 128, 10000.0)
    plain = A.attention(q2, k.to(gpu), v.to(gpu), causal=causal)
    assert_close(out.cpu().float(), plain.cpu().float(), *TOL[torch.float16], what + " vs unfused")
    # the table against float angles of the oracle (fp32 angles of positions ~1e3 carry ~1e-4 rad of rounding)
    oc, os_ = oe.rotary_cos_sin(pos, 128, 10000.0)
    assert_close(cs.cpu()[:, :64], oc, 2e-4, 0, what + " cos table")
    assert_close(cs.cpu()[:, 64:], os_, 2e-4, 0, what + " sin table")


def test_llama_block_fused_rotary_matches_unfused(gpu):
    # the config-2 block with the query rotation inside the attention kernel against the unfused block
    from deepgengraph_amd.llama import LlamaAttentionBlock

    g = torch.Generator().manual_seed(8)
    hidden, heads, S = 1024, 8, 384
    x = torch.randn(1, S, hidden, generator=g).bfloat16().to(gpu)
    w_norm = (1 + 0.02 * torch.randn(hidden, generator=g)).bfloat16().to(gpu)
    w_qkv = (0.02 * torch.randn(3 * hidden, hidden, generator=g)).bfloat16().to(gpu)
    w_o = (0.02 * torch.randn(hidden, hidden, generator=g)).bfloat16().to(gpu)
    fused = LlamaAttentionBlock(w_norm, w_qkv, w_o, heads=heads, kv_heads=heads, fuse_rope=True)
    plain = LlamaAttentionBlock(w_norm, w_qkv, w_o, heads=heads, kv_heads=heads, fuse_rope=False)
    assert fused.fuse_rope and not plain.fuse_rope
    assert_close(fused(x).cpu().float(), plain(x).cpu().float(), 2e-2, 1e-2, "fused vs unfused block")


def test_prefill_strided_views(gpu):
    # q/k/v as column slices of one fused QKV activation (row stride 3*H*D), output into a strided view
    S, H, D = 320, 4, 128
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(1, S, 3 * H * D, generator=g).bfloat16()
    q, k, v = (qkv[..., i * H * D:(i + 1) * H * D].reshape(1, S, H, D) for i in range(3))
    ref = oa.attention(q.contiguous(), k.contiguous(), v.contiguous())
    qg = qkv.to(gpu)
    views = [qg[..., i * H * D:(i + 1) * H * D].view(1, S, H, D) for i in range(3)]
    obuf = torch.zeros(1, S, H, 2 * D, dtype=torch.bfloat16, device=gpu)
    out = A.attention(*views, out=obuf[..., :D])
    assert_close(out.cpu().float(), ref.float(), 2e-2, 1e-2, "strided")
    assert torch.count_nonzero(obuf[..., D:]) == 0


def _colsum_check(got, ref, what):
    assert_close(got, ref, 1e-6, 1e-3, what)


@pytest.mark.parametrize("S,H,D,sinks,dtype", [
    (256, 2, 128, 4, torch.float16), (1000, 4, 128, 16, torch.float16), (300, 2, 64, 3, torch.float16),
    (512, 2, 128, 4, torch.bfloat16),   # bf16 scores rounded through the host-verified bf16 multiplier
])
def test_h2o_matches_oracle(gpu, S, H, D, sinks, dtype):
    g = torch.Generator().manual_seed(S + H)
    q = torch.randn(1, S, H, D, generator=g)
    k = torch.randn(1, S, H, D, generator=g)
    v = torch.randn(1, S, H, D, generator=g)
    k[:, torch.randperm(S, generator=g)[:sinks]] *= 4.0
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    ref_out, ref_cs, ref_lse = oa.h2o(q, k, v)
    out, cs = A.h2o_attention(q.to(gpu), k.to(gpu), v.to(gpu))
    what = f"h2o S{S} H{H} D{D} {dtype}"
    assert_close(out.cpu().float(), ref_out.float(), *TOL[dtype], what + " out")
    _colsum_check(cs.cpu(), ref_cs, what + " colsum")
    assert_close(cs.sum(-1).cpu(), torch.full((1, H), float(S)), 0, 1e-4, what + " sum of colsums = q_len")
    kk = min(64, S // 4)
    idx = A.topk_indices(cs, kk).cpu().numpy()
    np.testing.assert_array_equal(idx, osel.topk_indices(ref_cs.numpy(), kk))
    # the selection routine itself is bit-exact on identical scores
    np.testing.assert_array_equal(A.topk_indices(ref_cs.to(gpu), kk).cpu().numpy(), osel.topk_indices(ref_cs.numpy(), kk))


def _colsum_reference(q, k, causal, softcap, window, power=1):
    """Column sums of the reference's probabilities (scores rounded in the input dtype as attn.py:29 and
    gemma2.py:29-33 round them, fp32 softmax, masked pairs -inf, rows that see no key contributing nothing), per
    query head, summed in float64; power=2 sums their squares (roco.py:43-47). GQA: query head h reads KV head
    h // (Hq / Hkv)."""
    B, Sq, Hq, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    qt = q.transpose(1, 2)
    kT = k.transpose(1, 2).repeat_interleave(Hq // Hkv, 1).transpose(-2, -1)
    total = torch.zeros(B, Hq, Sk, dtype=torch.float64)
    for i0 in range(0, Sq, 256):
        n = min(256, Sq - i0)
        s = oa._scores(qt[:, :, i0:i0 + n], kT, D, softcap or None).float()
        m = oa._mask(i0, n, Sq, Sk, causal, window or None)
        if m is not None:
            s = s.masked_fill(m, float("-inf"))
        total += (torch.softmax(s, -1).nan_to_num(0.0).double() ** power).sum(2)
    return total


@pytest.mark.parametrize("D,Sq,Sk,causal,window,softcap,dtype,base2", [
    (64, 200, 200, True, 50, 20.0, torch.bfloat16, False),
    (128, 200, 200, True, 50, 20.0, torch.bfloat16, False),
    (128, 333, 517, True, 0, 0.0, torch.float16, True),
    (128, 517, 333, True, 0, 0.0, torch.bfloat16, False),   # Sq > Sk: leading rows see no key
    (128, 300, 300, False, 0, 0.0, torch.float16, True),
    (128, 640, 640, True, 100, 0.0, torch.float16, True),
    # long runs of mask-free query tiles (the software-pipelined column pass), ragged ends, Sq < Sk
    (128, 1100, 1300, True, 700, 0.0, torch.float16, True),
    (128, 1024, 1024, False, 0, 0.0, torch.bfloat16, False),
    (128, 900, 900, True, 0, 30.0, torch.bfloat16, True),
    (256, 160, 160, True, 0, 30.0, torch.bfloat16, False),
    (256, 300, 300, True, 64, 50.0, torch.float16, True),
])
def test_colsum_variants(gpu, D, Sq, Sk, causal, window, softcap, dtype, base2):
    # column sums (soft-cap, window, GQA, Sq != Sk, both lse forms) with the default reference rounding against the
    # reference's probabilities at the column-sum contract (1e-3 rel); the fp32-score opt-out against fp32 sums
    B, Hq, Hkv = 1, 4, 2
    q, k, v = _qkv(B, Sq, Sk, Hq, Hkv, D, dtype, 77 + D + Sq)
    kw = dict(causal=causal, softcap=softcap, window=window, lse_base2=base2)
    what = f"colsum D{D} Sq{Sq} Sk{Sk} causal{causal} w{window} sc{softcap} {dtype} base2={base2}"
    _, lse = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), return_lse=True, ref_rounding=True, **kw)
    cs = A.attention_colsum(q.to(gpu), k.to(gpu), lse, **kw).cpu()
    _colsum_check(cs, _colsum_reference(q, k, causal, softcap, window).float(), what + " reference rounding")
    _, lse = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), return_lse=True, ref_rounding=False, **kw)
    cs = A.attention_colsum(q.to(gpu), k.to(gpu), lse, ref_rounding=False, **kw).cpu()
    ref = _colsum_reference(q.float(), k.float(), causal, softcap, window).float()
    assert_close(cs, ref, 1e-3, 1e-2, what + " fp32 scores vs fp32 reference")


@pytest.mark.parametrize("Sq,Sk,Hq,Hkv,causal,window,dtype", [
    (256, 256, 4, 2, False, 0, torch.float16),     # exactly two mask-free query tiles: the shortest pipelined run
    (900, 1100, 4, 4, True, 500, torch.float16),   # window, Sq < Sk, ragged ends
    (1030, 1030, 4, 2, True, 0, torch.bfloat16),   # GQA, ragged last query tile
    # 64 keys per wave in two row groups: the second group's rows of the last query tile all past Sq, a wave's
    # second key block partly past Sk; a window shorter than a wave's keys; no mask with Sq < Sk and GQA
    (1088, 1000, 4, 2, True, 0, torch.float16),
    (1200, 1200, 2, 2, True, 40, torch.bfloat16),
    (700, 1500, 2, 1, False, 0, torch.float16),
])
def test_colscore_sum_and_sumsq_variants(gpu, Sq, Sk, Hq, Hkv, causal, window, dtype):
    # RoCo's epilogue (sums of p and p^2, roco.py:43-47) through the column-score primitive on the shapes the
    # software-pipelined column pass meets besides the causal square case: no mask, a window, GQA, ragged tiles
    from deepgengraph_amd import _lib

    D = 128
    q, k, v = _qkv(1, Sq, Sk, Hq, Hkv, D, dtype, 91 + Sq + Sk)
    kw = dict(causal=causal, window=window)
    what = f"colscore sum/sumsq Sq{Sq} Sk{Sk} H{Hq}/{Hkv} causal{causal} w{window} {dtype}"
    _, lse = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), return_lse=True, ref_rounding=True, lse_base2=True, **kw)
    s1, s2 = A.attention_colscore(q.to(gpu), k.to(gpu), lse, epilogue=_lib.COL_SUM_SQ, ref_rounding=True,
                                  lse_base2=True, **kw)
    _colsum_check(s1.cpu(), _colsum_reference(q, k, causal, 0.0, window).float(), what + " sum")
    _colsum_check(s2.cpu(), _colsum_reference(q, k, causal, 0.0, window, power=2).float(), what + " sum of squares")


def test_column_wrappers_reject_mismatched_k(gpu):
    # the column kernels take k's batch, head dim and dtype from q: a k that differs is refused on the host
    q = torch.zeros(1, 64, 2, 128, dtype=torch.bfloat16, device=gpu)
    lse = torch.zeros(1, 2, 64, dtype=torch.float32, device=gpu)
    bad = {"head dim": torch.zeros(1, 64, 2, 64, dtype=torch.bfloat16, device=gpu),
           "batch": torch.zeros(2, 64, 2, 128, dtype=torch.bfloat16, device=gpu),
           "dtype": torch.zeros(1, 64, 2, 128, dtype=torch.float16, device=gpu)}
    for what, k in bad.items():
        with pytest.raises(RuntimeError, match="incompatible shapes|dtypes differ"):
            A.attention_colsum(q, k, lse)
        with pytest.raises(RuntimeError, match="incompatible shapes|dtypes differ"):
            A.attention_colscore(q, k, lse, epilogue=0)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device=gpu)[::2]
    with pytest.raises(RuntimeError, match="workspace must be contiguous"):
        A.decode_attention(torch.zeros(1, 2, 128, dtype=torch.bfloat16, device=gpu),
                           torch.zeros(1, 2, 64, 128, dtype=torch.bfloat16, device=gpu),
                           torch.zeros(1, 2, 64, 128, dtype=torch.bfloat16, device=gpu), workspace=ws)


def test_topk_kernel_golden_and_ties(gpu):
    g = load_golden("topk_ties")
    x = torch.from_numpy(g["x"]).to(gpu)
    np.testing.assert_array_equal(A.topk_indices(x, 17).cpu().numpy(), g["out"])
    rng = np.random.default_rng(1)
    for n, k in ((4096, 256), (5000, 1), (777, 777), (65536, 1000), (3, 2)):
        vals = rng.integers(0, 50, size=(5, n)).astype(np.float32) / 7.0
        vals[0] = 0.0
        vals[1, ::2] = -0.0
        got = A.topk_indices(torch.from_numpy(vals).to(gpu), k).cpu().numpy()
        np.testing.assert_array_equal(got, osel.topk_indices(vals, k), err_msg=f"n={n} k={k}")


def test_topk_smallest_and_nan_order(gpu):
    # both directions (models/roco.py:55 takes the smallest) on rows with ties, signed zeros, infinities and NaNs,
    # across the three per-thread segment sizes of the kernel
    rng = np.random.default_rng(7)
    pool = np.array([0.0, -0.0, 1.0, -1.0, 2.5, -7.0, np.inf, -np.inf, np.nan, -np.nan], dtype=np.float32)
    for n, k in ((3, 2), (100, 37), (4096, 4000), (5000, 1), (16384, 9000), (65536, 1000), (40000, 39999)):
        progress(f"topk both directions n={n} k={k}")
        vals = rng.integers(0, 1 << 12, size=(4, n)).astype(np.float32) / 64.0 - 30.0
        vals[1] = rng.choice(pool, size=n)
        vals[2, ::3] = np.nan
        vals[3] = rng.integers(0, 3, size=n).astype(np.float32)
        x = torch.from_numpy(vals).to(gpu)
        for largest in (True, False):
            got = A.topk_indices(x, k, largest=largest).cpu().numpy()
            np.testing.assert_array_equal(got, osel.topk_indices(vals, k, largest), err_msg=f"n={n} k={k} {largest}")


@pytest.mark.parametrize("n", [65537, 131072, 1048576])
def test_topk_rows_longer_than_65536(gpu, n):
    # the multi-workgroup selection (several chunks per row, passes through a workspace): ties, signed zeros,
    # infinities and NaN, both directions, k at the edges and at chunk-crossing sizes
    rng = np.random.default_rng(n)
    pool = np.array([0.0, -0.0, 1.0, -1.0, 2.5, -7.0, np.inf, -np.inf, np.nan, -np.nan], dtype=np.float32)
    vals = rng.integers(0, 1 << 12, size=(5, n)).astype(np.float32) / 64.0 - 30.0
    vals[1] = rng.choice(pool, size=n)
    vals[2, ::3] = np.nan
    vals[3] = rng.integers(0, 3, size=n).astype(np.float32)
    vals[4] = 1.0  # one value: the tie rule alone decides
    x = torch.from_numpy(vals).to(gpu)
    for k in (1, 256, 20000, n - 1, n):
        progress(f"topk n={n} k={k}")
        for largest in (True, False):
            got = A.topk_indices(x, k, largest=largest).cpu().numpy()
            np.testing.assert_array_equal(got, osel.topk_indices(vals, k, largest), err_msg=f"n={n} k={k} {largest}")


@pytest.mark.parametrize("n", [131072, 1048576])
def test_topk_long_rows_continuous_values(gpu, n):
    # rows of distinct-looking values (normal, heavy-tailed positive, and a narrow band where the top bits agree):
    # few keys share the k-th key's 16-bit prefix, so the later passes load only a small part of the row
    rng = np.random.default_rng(n + 1)
    vals = np.stack([rng.standard_normal(n), rng.exponential(size=n) ** 3,
                     1.0 + rng.random(n) * 1e-3]).astype(np.float32)
    x = torch.from_numpy(vals).to(gpu)
    for k in (1, 256, 4096, n // 2, n - 1):
        progress(f"topk continuous n={n} k={k}")
        for largest in (True, False):
            got = A.topk_indices(x, k, largest=largest).cpu().numpy()
            np.testing.assert_array_equal(got, osel.topk_indices(vals, k, largest), err_msg=f"n={n} k={k} {largest}")


def test_topk_long_rows_two_stage_boundary(gpu):
    # at 1,048,576 keys (128 chunks of 8,192) k = 512 is the largest k of the two-stage selection (128 x 512
    # candidates, the merge's 64-per-thread form) and k = 513 the smallest of the pass form; ties across chunk
    # borders (a value repeated every 1,000 keys) decide both
    n = 1048576
    rng = np.random.default_rng(11)
    vals = rng.standard_normal((2, n)).astype(np.float32)
    vals[0, ::1000] = 3.5
    vals[1] = np.round(vals[1] * 4) / 4
    x = torch.from_numpy(vals).to(gpu)
    for k in (512, 513):
        progress(f"topk two-stage boundary n={n} k={k}")
        for largest in (True, False):
            got = A.topk_indices(x, k, largest=largest).cpu().numpy()
            np.testing.assert_array_equal(got, osel.topk_indices(vals, k, largest), err_msg=f"n={n} k={k} {largest}")


@pytest.mark.parametrize("n,q_len,recent,budget", [(131072, 4096, 256, 512), (1048576, 100, 4096, 30000),
                                                   (70000, 3, 0, 69999), (70000, 3, 70000, 0),
                                                   (131072, 4096, 0, 700), (131072, 4096, 700, 0),
                                                   (200000, 50, 1000, 3000),
                                                   (65600, 7, 3000, 7281), (65600, 7, 3000, 7282)])
def test_roco_select_rows_longer_than_65536(gpu, n, q_len, recent, budget):
    # RoCo's three chained selections over several workgroups per row, with ties and NaN std (negative variance);
    # recent and pick in two stages where chunks * k allows (the first and the fifth to eighth cases), with `other`
    # from recent's boundary, else all in passes. The last two sit at the two-stage form's candidate limit (9 chunks
    # of 8,192 keys x 7,281 = 65,529 candidates for `pick`), exactly at it and one past it (all in passes)
    rng = np.random.default_rng(n + recent)
    s1 = rng.integers(0, 50, size=(2, n)).astype(np.float32)
    s2 = rng.integers(0, 80, size=(2, n)).astype(np.float32) / 2.0
    s1[1] = rng.random(n).astype(np.float32)
    s2[1] = s1[1] * s1[1] / q_len + rng.random(n).astype(np.float32) * 1e-3
    progress(f"roco_select n={n} recent={recent} budget={budget}")
    got = A.roco_select(torch.from_numpy(s1).to(gpu), torch.from_numpy(s2).to(gpu), q_len, recent, budget)
    np.testing.assert_array_equal(got.cpu().numpy(), osel.roco_select(s1, s2, q_len, recent, budget),
                                  err_msg=f"n={n} q_len={q_len} recent={recent} budget={budget}")


def _roco_torch_gpu(s1, s2, q_len, recent, budget):
    """models/roco.py:54-61 as the reference writes it, run by torch on the GPU (its rounding of / q_len)."""
    std = torch.sqrt(s2 / q_len - (s1 / q_len) ** 2)
    _, other = torch.topk(std, largest=False, k=s1.shape[-1] - recent, dim=-1)
    _, rec = torch.topk(std, largest=True, k=recent, dim=-1)
    _, pick = torch.topk(s1.gather(dim=-1, index=other) / q_len, dim=-1, k=budget)
    return torch.cat([other.gather(dim=-1, index=pick), rec], dim=-1).sort(dim=-1)[0]


def _boundary_tied(vals, k, largest):
    """Per row: whether the k-th and (k+1)-th values in the direction are equal (torch's choice is then
    unspecified)."""
    nrows = int(np.prod(vals.shape[:-1]))
    if k == 0 or k >= vals.shape[-1]:
        return np.zeros(nrows, bool)
    rows = vals.reshape(nrows, vals.shape[-1])
    s = np.sort(np.where(np.isnan(rows), np.inf, rows), axis=-1)
    if largest:
        s = s[..., ::-1]
    return s[:, k - 1] == s[:, k]


@pytest.mark.parametrize("S,H,recent,budget", [(1024, 4, 256, 512), (4096, 2, 256, 1024), (300, 3, 0, 100),
                                                (300, 3, 300, 0), (5000, 2, 17, 4983)])
def test_roco_select_matches_oracle_and_torch(gpu, S, H, recent, budget):
    # the column sums of a real RoCo forward (fp16 inputs with attention sinks), then the selection of roco.py:54-61
    progress(f"roco_select S{S} H{H} recent{recent} budget{budget}")
    q, k, v = (t.to(gpu) for t in _qkv_sinks(S, H, 128, S + recent))
    _, s1, s2 = A.roco_attention(q, k, v)
    got = A.roco_select(s1, s2, S, recent, budget)
    assert got.shape == (1, H, budget + recent)
    np.testing.assert_array_equal(got.cpu().numpy(),
                                  osel.roco_select(s1.cpu().numpy(), s2.cpu().numpy(), S, recent, budget))
    # against torch on the GPU, on every row where its topk has no tie at a selection boundary
    std = torch.sqrt(s2 / S - (s1 / S) ** 2).cpu().numpy()
    other = torch.topk(torch.from_numpy(std), largest=False, k=S - recent, dim=-1)[1]
    picked = np.take_along_axis(s1.cpu().numpy(), other.numpy(), -1) * (np.float32(1) / np.float32(S))
    tied = _boundary_tied(std, recent, True) | _boundary_tied(std, S - recent, False) | \
        _boundary_tied(picked, budget, True)
    assert (~tied).sum() >= H - 1, f"{int(tied.sum())} of {H} rows tie at a selection boundary"
    ref = _roco_torch_gpu(s1, s2, S, recent, budget).cpu().numpy().reshape(H, -1)
    np.testing.assert_array_equal(got.cpu().numpy().reshape(H, -1)[~tied], ref[~tied])


def test_roco_select_ties_nan_and_edges(gpu):
    # quantised sums: ties everywhere, and s2 < s1^2 / q_len (negative variance: NaN std) in places
    rng = np.random.default_rng(5)
    for n, q_len, recent, budget in ((50, 3, 5, 20), (4096, 7, 256, 1024), (10000, 11, 1000, 2000),
                                     (65536, 100, 64, 512), (1, 1, 1, 0), (1, 1, 0, 1), (8, 2, 4, 4)):
        progress(f"roco_select ties n={n}")
        s1 = rng.integers(0, 5, size=(3, n)).astype(np.float32)
        s2 = rng.integers(0, 8, size=(3, n)).astype(np.float32) / 2.0
        got = A.roco_select(torch.from_numpy(s1).to(gpu), torch.from_numpy(s2).to(gpu), q_len, recent, budget)
        np.testing.assert_array_equal(got.cpu().numpy(), osel.roco_select(s1, s2, q_len, recent, budget),
                                      err_msg=f"n={n} q_len={q_len} recent={recent} budget={budget}")
    # nothing to select: an empty result, no launch
    s = torch.zeros(2, 10, device=gpu)
    assert A.roco_select(s, s, 10, 0, 0).shape == (2, 0)


@pytest.mark.parametrize("case_cls,kw,dtype,q_len,kv_len", [
    (ocases.Attn, dict(kv_head_num=4, head_num=4, head_dim=128), torch.bfloat16, 384, 384),
    (ocases.Gemma2, dict(kv_head_num=4, head_num=4, head_dim=128), torch.bfloat16, 384, 384),
    (ocases.H2O, dict(kv_head_num=4, head_num=4, head_dim=128), torch.float16, 384, 384),
    # the reference's default dtype (fp16, attn.py:36 / gemma2.py:41), ragged and unequal lengths
    (ocases.Attn, dict(kv_head_num=4, head_num=4, head_dim=128), torch.float16, 384, 384),
    (ocases.Attn, dict(kv_head_num=4, head_num=4, head_dim=128), torch.float16, 333, 517),
    (ocases.Gemma2, dict(kv_head_num=4, head_num=4, head_dim=128), torch.float16, 384, 384),
    (ocases.Gemma2, dict(kv_head_num=2, head_num=2, head_dim=256), torch.float16, 300, 300),
    (ocases.Gemma2, dict(kv_head_num=4, head_num=4, head_dim=128), torch.float16, 517, 333),
    # fp32 (config 1's dtype) and decode-shaped calls (q_len == 1: attn.py:22-23 masks nothing)
    (ocases.Attn, dict(kv_head_num=8, head_num=8, head_dim=64), torch.float32, 256, 256),
    (ocases.Attn, dict(kv_head_num=8, head_num=8, head_dim=128), torch.float16, 1, 4096),
    (ocases.Attn, dict(kv_head_num=4, head_num=4, head_dim=64), torch.bfloat16, 1, 1000),
    (ocases.Attn, dict(kv_head_num=4, head_num=4, head_dim=256), torch.float16, 1, 777),
])
def test_compile_drop_in(gpu, case_cls, kw, dtype, q_len, kv_len):
    # run_kernel.py:44-78 flow: build the case, prepare inputs, compile with the MI355X system, compare outputs
    model = case_cls(**kw).eval()
    specs = model.prepare(batch_size=2 if q_len == 1 else 1, q_len=q_len, kv_len=kv_len, dtype=dtype, seed=3)
    names = list(specs["input"].keys())
    inputs = [specs["input"][n] for n in names]
    f = dgg_compile(model=model, input_names=names, inputs=inputs, output_names=specs["output"], system="mi355x")
    outs = f(*[t.to(gpu) for t in inputs])
    refs = model(*inputs)
    tol = TOL.get(dtype, (1e-5, 1e-5))
    what = f"{case_cls.__name__} {dtype} q_len={q_len} kv_len={kv_len}"
    if isinstance(refs, tuple):
        assert isinstance(outs, tuple) and len(outs) == len(refs)
        assert_close(outs[0].cpu().float(), refs[0].float(), *tol, what + " out")
        _colsum_check(outs[1].cpu(), refs[1], what + " score")
        assert outs[1].shape == refs[1].shape
    else:
        assert outs.shape == refs.shape and outs.dtype == refs.dtype
        got, want = outs.cpu().float(), refs.float()
        nan = torch.isnan(want)
        assert torch.equal(torch.isnan(got), nan), what + " NaN rows"
        assert_close(got[~nan], want[~nan], *tol, what)


@pytest.mark.parametrize("B,H,Hkv,L,D,dtype", [
    (4, 8, 8, 4096, 128, torch.float16),
    (3, 8, 2, 3000, 64, torch.bfloat16),    # GQA, ragged split
    (2, 4, 4, 300, 256, torch.float16),
])
def test_decode_shaped_prefill_call_matches_oracle(gpu, B, H, Hkv, L, D, dtype):
    # attention() with one query row runs on the split-KV decode kernels, reading the case layout [B, L, H, D]
    # through its strides; output and lse (both bases) against the oracle
    q, k, v = _qkv(B, 1, L, H, Hkv, D, dtype, seed=L + D)
    ref, ref_lse = oa.attention(q, k, v, causal=True, return_lse=True)
    out, lse = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=True, return_lse=True)
    what = f"decode-shaped B{B} H{H}/{Hkv} L{L} D{D} {dtype}"
    assert_close(out.cpu().float(), ref.float(), *TOL[dtype], what + " out")
    assert_close(lse.cpu(), ref_lse, 1e-3, 1e-4, what + " lse")
    _, lse2 = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=True, return_lse=True, lse_base2=True)
    assert_close(lse2.cpu(), ref_lse * math.log2(math.e), 1e-3, 1e-4, what + " lse base 2")


def test_h2o_matches_torch_eager_on_gpu(gpu):
    """H2O with reference rounding against the reference formula run by torch itself on the GPU (the case module
    of the 'torch' system, h2o.py:18-38, on the same fp16 inputs with x4 sink keys): the scores go through torch's
    own GPU matmul rounding and GPU division by sqrt(D). Column sums within 1e-3 and identical top-256 sets; the
    score gap at the selection boundary is reported on failure."""
    from deepgengraph_amd import cases as tcases

    S, H, D, kk = 2048, 8, 128, 256
    g = torch.Generator().manual_seed(4242)
    q = torch.randn(1, S, H, D, generator=g)
    k = torch.randn(1, S, H, D, generator=g)
    v = torch.randn(1, S, H, D, generator=g)
    k[:, torch.randperm(S, generator=g)[:16]] *= 4.0
    q, k, v = (t.half().to(gpu) for t in (q, k, v))
    prev = torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction
    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = False  # fp32 accumulation, one rounding
    try:
        ref_out, ref_cs = tcases.H2O(kv_head_num=H, head_num=H, head_dim=D)(q, k, v)
    finally:
        torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = prev
    out, cs = A.h2o_attention(q, k, v)
    assert_close(out.cpu().float(), ref_out.cpu().float(), *TOL[torch.float16], "h2o out vs torch on GPU")
    _colsum_check(cs.cpu(), ref_cs.cpu(), "h2o score vs torch on GPU")
    got = A.topk_indices(cs, kk).cpu().numpy()
    want = osel.topk_indices(ref_cs.cpu().numpy(), kk)
    if not np.array_equal(got, want):
        srt = np.sort(ref_cs.cpu().numpy(), axis=-1)[..., ::-1]
        gap = srt[..., kk - 1] - srt[..., kk]
        raise AssertionError(f"top-{kk} sets differ; reference score gap at rank {kk}: min {gap.min():.3e}")
