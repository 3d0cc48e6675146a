"""Pins the CPU oracle (oracle/) against the float64 brute-force definitions, golden vectors, closed forms and
invariants. No GPU needed. Each check is chosen so that a plausible mistake (wrong mask diagonal, transposed
operand, wrong GQA head, dropped scale, wrong rotary pairing, unstable tie order) fails it."""
import math

import numpy as np
import pytest
import torch

from conftest import assert_close, load_golden
from oracle import attention as oa
from oracle import brute
from oracle import elementwise as oe
from oracle import selection as osel


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x))


@pytest.mark.parametrize("name,kw", [
    ("attn_tiny_causal_f32", dict(causal=True)),
    ("attn_tiny_gqa_softcap_window_f32", dict(causal=True, softcap=5.0, window=5)),
    ("attn_tiny_noncausal_f32", dict(causal=False)),
    ("attn_d64_causal_bf16", dict(causal=True)),
    ("attn_d64_gqa_softcap_window_bf16", dict(causal=True, softcap=5.0, window=33)),
])
def test_attention_matches_golden(name, kw):
    g = load_golden(name)
    out, lse = oa.attention(_t(g["q"]), _t(g["k"]), _t(g["v"]), return_lse=True, **kw)
    assert_close(out, g["out"], 1e-5, 1e-5, f"{name} out")
    assert_close(lse, g["lse"], 1e-5, 1e-5, f"{name} lse")


def test_fully_masked_rows_are_nan_like_the_reference():
    # Sq > Sk with bottom-right alignment: the first Sq - Sk rows see no key; softmax of an all -inf row is NaN.
    g = load_golden("attn_tiny_causal_sq_gt_sk_f32")
    out, lse = oa.attention(_t(g["q"]), _t(g["k"]), _t(g["v"]), return_lse=True)
    assert torch.isnan(out[0, :4]).all() and not torch.isnan(out[0, 4:]).any()
    assert torch.isinf(lse[0, 0, :4]).all() and (lse[0, 0, :4] < 0).all()
    assert_close(out, g["out"], 1e-5, 1e-5, "sq>sk out")


def test_h2o_colsum_matches_golden_and_invariant():
    g = load_golden("attn_d64_h2o_sinks_f16")
    q, k, v = _t(g["q"]), _t(g["k"]), _t(g["v"])
    out, colsum, lse = oa.h2o(q, k, v)
    assert_close(colsum, g["colsum"], 1e-6, 1e-5, "colsum")
    assert_close(out, g["out"], 1e-5, 1e-5, "h2o out")
    # every probability row sums to 1, so the column sums of a head add up to q_len
    assert_close(colsum.sum(-1), torch.full((1, 2), float(q.shape[1])), 0, 1e-5, "sum of colsums")
    # causal: the last key is seen only by the last query, so its column sum is that one probability
    s_last = (q[0, -1].double() * k[0, -1].double()).sum(-1) / math.sqrt(q.shape[-1])  # [H]
    assert_close(colsum[0, :, -1], torch.exp(s_last - lse[0, :, -1].double()), 1e-7, 1e-5, "last column")


def test_attention_closed_forms():
    torch.manual_seed(0)
    B, S, H, D = 1, 24, 2, 16
    v = torch.randn(B, S, H, D)
    # q = 0: every visible score is 0 -> lse_i = ln(#visible keys) = ln(i + 1); out_i = mean of v_0..v_i
    q = torch.zeros(B, S, H, D)
    k = torch.randn(B, S, H, D)
    out, lse = oa.attention(q, k, v, return_lse=True)
    assert_close(lse[0, 0], torch.log(torch.arange(1, S + 1, dtype=torch.float64)), 1e-6, 1e-6, "lse closed form")
    means = torch.cumsum(v, 1) / torch.arange(1, S + 1).view(1, S, 1, 1)
    assert_close(out, means, 1e-5, 1e-5, "uniform attention")
    # first query sees only key 0
    q = torch.randn(B, S, H, D)
    out = oa.attention(q, k, v)
    assert_close(out[:, 0], v[:, 0], 1e-6, 1e-6, "causal row 0")


def test_attention_reductions():
    torch.manual_seed(1)
    B, S, Hq, Hkv, D = 2, 40, 4, 2, 16
    q, k, v = torch.randn(B, S, Hq, D), torch.randn(B, S, Hkv, D), torch.randn(B, S, Hkv, D)
    base = oa.attention(q, k, v)
    # GQA == explicit head repeat (roco.py:25-27 convention)
    rep = oa.attention(q, k.repeat_interleave(2, dim=2), v.repeat_interleave(2, dim=2))
    assert torch.equal(base, rep)
    # window >= S reduces to causal; a huge soft-cap reduces to no soft-cap
    assert torch.equal(oa.attention(q, k, v, window=S), base)
    assert_close(oa.attention(q, k, v, softcap=1e6), base, 1e-5, 1e-5, "softcap->inf")
    # query chunking is exact
    assert_close(oa.attention(q, k, v, q_chunk=7), base, 1e-6, 1e-6, "chunking")
    # window 1 keeps only the diagonal: out_i = v_i
    assert_close(oa.attention(q, k, v, window=1), v.repeat_interleave(2, dim=2), 1e-6, 1e-6, "window 1")


def test_attention_low_precision_within_tolerance_of_fp32():
    # the bf16 oracle stays within the bf16 tolerance of the fp32 evaluation of the same (exactly representable)
    # inputs; the individual rounding points are pinned step by step in test_ref_rounding.py
    torch.manual_seed(2)
    q, k, v = (torch.randn(1, 64, 2, 64).bfloat16() for _ in range(3))
    lo = oa.attention(q, k, v)
    hi = oa.attention(q.float(), k.float(), v.float())
    assert lo.dtype == torch.bfloat16
    assert_close(lo.float(), hi, 2e-2, 1e-2, "bf16 vs fp32")


def test_config1_at_size_against_float64():
    """Config 1 (fp32 causal MHA, B=1, H=8, S=512, D=64, N(0,1) inputs, scale 1/8) at its full size: the oracle's
    O [B, S, H, D] and natural-log LSE [B, H, S] against a float64 numpy evaluation of the same formula."""
    from deepgengraph_amd import configs as C

    cfg = C.CFG1
    q, k, v, _ = C.attn_inputs(cfg)
    assert q.dtype == torch.float32 and tuple(q.shape) == (1, 512, 8, 64)
    out, lse = oa.attention(q, k, v, causal=True, return_lse=True)
    qn, kn, vn = (t.double().numpy().transpose(0, 2, 1, 3) for t in (q, k, v))  # [B, H, S, D]
    s = qn @ kn.transpose(0, 1, 3, 2) / 8.0
    s = np.where(np.triu(np.ones((512, 512), bool), 1), -np.inf, s)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    ref_lse = (m[..., 0] + np.log(e.sum(-1)))
    ref_out = ((e / e.sum(-1, keepdims=True)) @ vn).transpose(0, 2, 1, 3)
    assert_close(out, ref_out, 1e-5, 1e-5, "config 1 O")
    assert_close(lse, ref_lse, 1e-5, 1e-6, "config 1 LSE")


def _block_float64(x, w_norm, w_qkv, w_o, heads, kv_heads, eps, theta, *, rotate_v=False, split=("q", "k", "v"),
                   k_pos_offset=0):
    """models/attn.py:34-53 + LlamaLayer's norm (models/attn.py:71-74) composed from the float64 brute-force
    pieces, with both projections as explicit loops (y = x W^T, W stored [out, in]). The keyword arguments plant
    the mistakes the oracle must not make (rotating v, another split order, k rotated at shifted positions)."""
    S, hidden = len(x), len(x[0])
    D = hidden // heads
    h = brute.rms_norm(x, w_norm, eps)
    n_out = len(w_qkv)
    qkv = [[sum(h[t][i] * float(w_qkv[o][i]) for i in range(hidden)) for o in range(n_out)] for t in range(S)]
    sizes = {"q": heads * D, "k": kv_heads * D, "v": kv_heads * D}
    parts, c = {}, 0
    for name in split:
        parts[name] = [row[c:c + sizes[name]] for row in qkv]
        c += sizes[name]
    pos = list(range(S))
    q = brute.rotary(pos, parts["q"], D, theta)
    k = brute.rotary([t + k_pos_offset for t in pos], parts["k"], D, theta)
    v = brute.rotary(pos, parts["v"], D, theta) if rotate_v else parts["v"]
    q4 = [[[q[t][hh * D:(hh + 1) * D] for hh in range(heads)] for t in range(S)]]
    k4 = [[[k[t][hh * D:(hh + 1) * D] for hh in range(kv_heads)] for t in range(S)]]
    v4 = [[[v[t][hh * D:(hh + 1) * D] for hh in range(kv_heads)] for t in range(S)]]
    o, _ = brute.attention(q4, k4, v4, causal=True)
    of = [[o[0][t][hh][d] for hh in range(heads) for d in range(D)] for t in range(S)]
    return [[sum(of[t][i] * float(w_o[r][i]) for i in range(hidden)) for r in range(hidden)] for t in range(S)]


def test_attention_block_against_float64_composition():
    """oracle.llama.attention_block (config 2's block) on a tiny GQA block (hidden 64, 4 heads, 2 KV heads, S=16)
    against the float64 composition of brute.rms_norm, brute.rotary, brute.attention and loop projections. Each
    planted mistake of the composition (v rotated, W used untransposed, q/k split swapped, k rotated one position
    off q) must move the result far outside the tolerance, so the comparison can see it. (Shifting q and k by the
    same offset is invisible by construction: rotary scores depend only on the position difference, which
    test_rotary checks.)"""
    from oracle import llama as ol

    g = torch.Generator().manual_seed(11)
    S, hidden, heads, kv_heads = 16, 64, 4, 2
    D = hidden // heads
    x = torch.randn(1, S, hidden, generator=g)
    w_norm = 1 + 0.02 * torch.randn(hidden, generator=g)
    w_qkv = 0.2 * torch.randn((heads + 2 * kv_heads) * D, hidden, generator=g)
    w_o = 0.2 * torch.randn(hidden, hidden, generator=g)
    eps, theta = 1e-6, 100.0  # a small theta turns every rotary pair at these positions
    out = ol.attention_block(x, w_norm, w_qkv, w_o, heads=heads, kv_heads=kv_heads, eps=eps, theta=theta)
    args = (x[0].tolist(), w_norm.tolist(), w_qkv.tolist(), w_o.tolist(), heads, kv_heads, eps, theta)
    ref = torch.tensor(_block_float64(*args), dtype=torch.float64)
    assert_close(out[0], ref, 1e-4, 1e-4, "attention block")
    planted = {
        "v rotated": _block_float64(*args, rotate_v=True),
        "k/q split swapped": _block_float64(*args, split=("k", "q", "v")),
        "k positions off by one": _block_float64(*args, k_pos_offset=1),
    }
    # W used untransposed: only shapes where it multiplies at all, i.e. the square output projection
    wt = w_o.t().contiguous()
    planted["W_o untransposed"] = _block_float64(x[0].tolist(), w_norm.tolist(), w_qkv.tolist(), wt.tolist(), heads,
                                                 kv_heads, eps, theta)
    for what, bad in planted.items():
        err = (torch.tensor(bad, dtype=torch.float64) - ref).abs().max().item()
        assert err > 1e-2, f"planted mistake '{what}' is not visible ({err:.2e})"


def test_decode_matches_attention_and_splitkv():
    torch.manual_seed(3)
    B, H, Hkv, L, D = 2, 4, 2, 37, 16
    q = torch.randn(B, H, D)
    kc, vc = torch.randn(B, Hkv, L, D), torch.randn(B, Hkv, L, D)
    out, lse = oa.decode(q, kc, vc)
    # decode == Attn.forward with q_len == 1 (nothing masked) in the case layout
    ref, ref_lse = oa.attention(q.unsqueeze(1), kc.transpose(1, 2), vc.transpose(1, 2), return_lse=True)
    assert_close(out, ref[:, 0], 1e-6, 1e-6, "decode vs attention")
    assert_close(lse, ref_lse[:, :, 0], 1e-6, 1e-6, "decode lse")
    o1, l1 = oa.decode_splitkv(q, kc, vc, 1)
    for s in (2, 3, 7, L, L + 5):
        os_, ls_ = oa.decode_splitkv(q, kc, vc, s)
        np.testing.assert_allclose(os_, o1, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(ls_, l1, rtol=1e-12, atol=1e-12)
    assert_close(out, o1, 1e-5, 1e-5, "fp32 decode vs float64 split-kv")
    # brute force (float64 loops) pins the unsplit formula
    bo, bl = brute.attention(q.unsqueeze(1).tolist(), kc.transpose(1, 2).tolist(), vc.transpose(1, 2).tolist(),
                             causal=False)
    np.testing.assert_allclose(o1, np.array(bo)[:, 0], rtol=1e-10, atol=1e-10)


def test_rms_norm():
    g = load_golden("rms_norm_bf16")
    x, w = _t(g["x"]), _t(g["w"])
    assert_close(oe.rms_norm(x, w, 1e-6), g["out"], 1e-6, 1e-6, "fp32 rms_norm vs brute")
    got = oe.rms_norm(x.bfloat16(), w.bfloat16(), 1e-6)
    assert got.dtype == torch.bfloat16
    assert_close(got.float(), g["out"], 2e-2, 1e-2, "bf16 rms_norm")
    # the two rounding points: T(x*s) then T(T * w)
    s = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    assert torch.equal(got, ((x * s).bfloat16().float() * w).bfloat16())
    # scale invariance and unit RMS with w = 1
    assert_close(oe.rms_norm(x * 3.0, w, 0.0), oe.rms_norm(x, w, 0.0), 1e-6, 1e-5, "scale invariance")
    y = oe.rms_norm(x, torch.ones_like(w), 0.0)
    assert_close(y.pow(2).mean(-1), torch.ones(x.shape[0]), 1e-5, 1e-5, "unit rms")


def test_fused_add_rms_norm():
    torch.manual_seed(4)
    x, r = torch.randn(5, 32).half(), torch.randn(5, 32).half()
    w = (1 + 0.02 * torch.randn(32)).half()
    out, res = oe.fused_add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(res, (x.float() + r.float()).half())
    assert_close(out.float(), oe.rms_norm((x.float() + r.float()), w.float(), 1e-6), 1e-2, 5e-3, "fused add")


def test_silu_and_mul():
    g = load_golden("silu_and_mul_f16")
    x = _t(g["x"])
    assert_close(oe.silu_and_mul(x), g["out"], 1e-6, 1e-6, "fp32 silu vs brute")
    h = x.half()
    got = oe.silu_and_mul(h)
    d = x.shape[-1] // 2
    # library routine: torch.nn.functional.silu in fp32, rounded, times up in fp16
    assert torch.equal(got, torch.nn.functional.silu(h[:, :d].float()).half() * h[:, d:])
    assert float(oe.silu_and_mul(torch.zeros(1, 4))[0, 0]) == 0.0


def test_rotary():
    g = load_golden("rotary_d32_f32")
    pos, x = _t(g["pos"]), _t(g["x"])
    qo, ko = oe.rotary_embedding_online(pos, x, x[:, :32].contiguous(), 32, 10000.0)
    # fp32 angles at positions up to 4095 carry ~1e-4 rad of rounding
    assert_close(qo, g["out"], 2e-3, 1e-3, "rotary vs float64 brute")
    assert_close(ko, g["out"][:, :32], 2e-3, 1e-3, "rotary key")
    # pairing is (i, i + D/2): rotating a vector with only x_0 set moves mass to x_{D/2}
    e = torch.zeros(1, 32)
    e[0, 0] = 1.0
    r, _ = oe.rotary_embedding_online(torch.tensor([1], dtype=torch.int32), e, None, 32, 10000.0)
    assert abs(float(r[0, 16]) - math.sin(1.0)) < 1e-6 and abs(float(r[0, 0]) - math.cos(1.0)) < 1e-6
    torch.manual_seed(5)
    D = 128
    q = torch.randn(3, D)
    zero, _ = oe.rotary_embedding_online(torch.zeros(3, dtype=torch.int32), q, None, D, 10000.0)
    assert torch.equal(zero, q)  # pos 0 is the identity
    p = torch.tensor([5, 17, 300], dtype=torch.int32)
    rq, _ = oe.rotary_embedding_online(p, q, None, D, 10000.0)
    pair_norm = lambda t: t[:, : D // 2] ** 2 + t[:, D // 2:] ** 2  # noqa: E731
    assert_close(pair_norm(rq), pair_norm(q), 1e-5, 1e-5, "pair norms")
    # composition: rot(a) after rot(b) == rot(a + b)
    a, b = torch.tensor([7, 9, 11], dtype=torch.int32), torch.tensor([3, 20, 100], dtype=torch.int32)
    rab, _ = oe.rotary_embedding_online(a, oe.rotary_embedding_online(b, q, None, D, 10000.0)[0], None, D, 10000.0)
    assert_close(rab, oe.rotary_embedding_online(a + b, q, None, D, 10000.0)[0], 1e-4, 1e-4, "composition")
    # relative position: <rot_m q, rot_n k> depends only on m - n
    k = torch.randn(1, D)
    dots = []
    for m, n in ((10, 4), (106, 100), (1006, 1000)):
        qm, _ = oe.rotary_embedding_online(torch.tensor([m], dtype=torch.int32), q[:1], None, D, 10000.0)
        kn, _ = oe.rotary_embedding_online(torch.tensor([n], dtype=torch.int32), k, None, D, 10000.0)
        dots.append(float((qm * kn).sum()))
    assert max(dots) - min(dots) < 1e-3


def test_topk_selection():
    g = load_golden("topk_ties")
    got = osel.topk_indices(g["x"], 17)
    np.testing.assert_array_equal(got, g["out"])
    # +0.0 and -0.0 tie: the lowest indices win
    x = np.array([[0.0, -0.0, 0.0, -0.0, 1.0]], dtype=np.float32)
    np.testing.assert_array_equal(osel.topk_indices(x, 3), [[0, 1, 4]])
    rng = np.random.default_rng(0)
    for _ in range(20):
        row = rng.integers(0, 4, size=40).astype(np.float32)
        k = int(rng.integers(1, 40))
        np.testing.assert_array_equal(osel.topk_indices(row[None], k)[0], brute.topk_indices(row.tolist(), k))


def test_topk_direction_and_nan_order():
    # both directions against the exhaustive ranking, on rows full of ties, signed zeros, infinities and NaNs
    rng = np.random.default_rng(1)
    pool = np.array([0.0, -0.0, 1.0, -1.0, 2.5, np.inf, -np.inf, np.nan, -np.nan], dtype=np.float32)
    for _ in range(40):
        row = rng.choice(pool, size=30)
        k = int(rng.integers(1, 31))
        for largest in (True, False):
            np.testing.assert_array_equal(osel.topk_indices(row[None], k, largest)[0],
                                          brute.topk_indices(row.tolist(), k, largest))
    # torch.topk (the library routine the reference calls) on distinct values with one NaN: the same sets
    for seed in range(5):
        x = torch.randperm(200, generator=torch.Generator().manual_seed(seed)).float() - 100.0
        x[seed * 7] = float("nan")
        for largest in (True, False):
            for k in (1, 13, 199):
                ref = torch.topk(x, k, largest=largest)[1].sort()[0].numpy()
                np.testing.assert_array_equal(osel.topk_indices(x.numpy()[None], k, largest)[0], ref)


def _roco_reference_torch(s1, s2, q_len, recent, budget):
    """models/roco.py:54-61 as the reference writes it, in torch on the CPU."""
    std = torch.sqrt(s2 / q_len - (s1 / q_len) ** 2)
    kv_len = s1.shape[-1]
    _, other = torch.topk(std, largest=False, k=kv_len - recent, dim=-1)
    _, rec = torch.topk(std, largest=True, k=recent, dim=-1)
    _, pick = torch.topk(s1.gather(dim=-1, index=other) / q_len, dim=-1, k=budget)
    sel = torch.cat([other.gather(dim=-1, index=pick), rec], dim=-1)
    return sel.sort(dim=-1)[0]


def _roco_separated(seed, rows, n, q_len):
    """Column sums whose std and mean values lie far apart (no two within many ulps): any correct rounding of the
    reference's arithmetic orders them the same way."""
    g = torch.Generator().manual_seed(seed)
    mean = (torch.stack([torch.randperm(n, generator=g) for _ in range(rows)]).double() + 1.0) / (4.0 * n)
    std = (torch.stack([torch.randperm(n, generator=g) for _ in range(rows)]).double() + 1.0) / (8.0 * n)
    s1 = (mean * q_len).float()
    s2 = ((std ** 2 + mean ** 2) * q_len).float()
    return s1, s2


def test_roco_select_matches_reference_lines():
    for seed, (rows, n, q_len, recent, budget) in enumerate([(3, 64, 64, 8, 16), (2, 300, 300, 30, 100),
                                                             (4, 97, 50, 0, 40), (2, 50, 50, 50, 0),
                                                             (1, 128, 128, 1, 127)]):
        s1, s2 = _roco_separated(seed, rows, n, q_len)
        ref = _roco_reference_torch(s1, s2, q_len, recent, budget).numpy()
        got = osel.roco_select(s1.numpy(), s2.numpy(), q_len, recent, budget)
        np.testing.assert_array_equal(got, ref)
        # planted mistakes: the largest std as `other`, or the pick by the smallest column sums
        std = np.sqrt(s2.numpy() / q_len - (s1.numpy() / q_len) ** 2)
        if 0 < budget < n - recent:
            if recent > 0:
                wrong_other = osel.topk_indices(std, n - recent, largest=True)
                pick = osel.topk_indices(np.take_along_axis(s1.numpy(), wrong_other, -1), budget)
                wrong = np.sort(np.concatenate([np.take_along_axis(wrong_other, pick, -1),
                                                osel.topk_indices(std, recent)], -1), -1)
                assert not np.array_equal(wrong, ref)
            other = osel.topk_indices(std, n - recent, largest=False)
            pick = osel.topk_indices(np.take_along_axis(s1.numpy(), other, -1), budget, largest=False)
            wrong = np.sort(np.concatenate([np.take_along_axis(other, pick, -1), osel.topk_indices(std, recent)], -1), -1)
            assert not np.array_equal(wrong, ref)


def test_roco_select_ties_nan_and_invariants():
    rng = np.random.default_rng(3)
    for _ in range(30):
        n = int(rng.integers(2, 24))
        recent = int(rng.integers(0, n + 1))
        budget = int(rng.integers(0, n - recent + 1))
        s1 = rng.integers(0, 4, size=n).astype(np.float32)
        s2 = rng.integers(0, 6, size=n).astype(np.float32)  # s2 < s1**2 / q_len somewhere: NaN std
        q_len = int(rng.integers(1, 5))
        got = osel.roco_select(s1[None], s2[None], q_len, recent, budget)[0]
        # exhaustive-ranking restatement of roco.py:54-61 (float32 arithmetic, torch's GPU rounding of / q_len)
        rcp = np.float32(1) / np.float32(q_len)
        with np.errstate(invalid="ignore"):
            std = [float(np.sqrt(np.float32(b) * rcp - (np.float32(a) * rcp) * (np.float32(a) * rcp)))
                   for a, b in zip(s1, s2)]
        other = brute.topk_indices(std, n - recent, largest=False)
        rec = brute.topk_indices(std, recent, largest=True)
        pick = brute.topk_indices([float(np.float32(s1[i]) * rcp) for i in other], budget)
        want = sorted([other[p] for p in pick] + rec)
        np.testing.assert_array_equal(got, want)
        assert len(got) == budget + recent and np.all(np.diff(got) >= 0)
    # recent = 0 keeps the budget largest column sums (H2O's rule); budget = 0 keeps the largest std
    s1, s2 = _roco_separated(9, 2, 80, 80)
    np.testing.assert_array_equal(osel.roco_select(s1.numpy(), s2.numpy(), 80, 0, 20), osel.topk_indices(s1.numpy(), 20))
    std = np.sqrt(s2.numpy() / np.float32(80) - (s1.numpy() / np.float32(80)) ** 2)
    np.testing.assert_array_equal(osel.roco_select(s1.numpy(), s2.numpy(), 80, 10, 0), osel.topk_indices(std, 10))


def _sel_inputs(seed, B=1, S=20, H=2, D=8, Sk=None, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    Sk = S if Sk is None else Sk
    q = torch.randn(B, S, H, D, generator=g) * scale
    k = torch.randn(B, Sk, H, D, generator=g)
    v = torch.randn(B, Sk, H, D, generator=g)
    return q, k, v


def test_roco_matches_brute_and_invariants():
    q, k, v = _sel_inputs(5)
    out, s1, s2, lse = oa.roco(q, k, v)
    b1, b2, _ = brute.colscores(q.tolist(), k.tolist())
    assert_close(s1, torch.tensor(b1), 1e-6, 1e-5, "roco sum vs brute")
    assert_close(s2, torch.tensor(b2), 1e-6, 1e-5, "roco sum of squares vs brute")
    # the sum part is the H2O column sum; the last key is seen by the last query only, so s2 = s1^2 there
    assert_close(s1, oa.h2o(q, k, v)[1], 0, 0, "roco sum == h2o colsum")
    assert_close(s2[..., -1], s1[..., -1] ** 2, 1e-7, 1e-6, "single-probability column")
    assert (s2 <= s1 + 1e-7).all() and (s2 > 0).all()
    assert_close(s1.sum(-1), torch.full((1, 2), 20.0), 0, 1e-5, "sum of column sums = q_len")
    assert_close(out, oa.attention(q, k, v), 0, 0, "roco out == attention")


def test_snapkv_pool_matches_brute_and_closed_form():
    q, k, v = _sel_inputs(6, S=23)
    out, pooled, _ = oa.snapkv(q, k, v)
    cs = oa.h2o(q, k, v)[1]
    want = torch.tensor([[brute.avg_pool(cs[0, h].tolist(), 5) for h in range(2)]])
    assert_close(pooled, want, 1e-7, 1e-6, "snapkv pooled vs brute")
    # a constant row pools to 3/5, 4/5, 1, ..., 1, 4/5, 3/5 (zero padding counted)
    ones = torch.ones(2, 3, 9)
    p1 = osel.avg_pool1d(ones, 5)
    assert_close(p1[0, 0], torch.tensor([0.6, 0.8, 1, 1, 1, 1, 1, 0.8, 0.6]), 1e-7, 1e-6, "pool of ones")
    x = torch.randn(3, 17)
    for ks in (1, 3, 7):
        got = osel.avg_pool1d(x, ks)
        assert_close(got, torch.tensor([brute.avg_pool(r, ks) for r in x.tolist()]), 1e-6, 1e-6, f"pool k={ks}")


def test_corm_matches_brute_and_closed_form():
    q, k, v = _sel_inputs(7, S=18, scale=1.5)
    thr = oa.corm_mask(18, 18)
    out, hit, _ = oa.corm(q, k, v, thr)
    _, _, bh = brute.colscores(q.tolist(), k.tolist(), thr=thr.tolist())
    assert hit.dtype == torch.bool and hit.shape == (1, 2, 18)
    assert torch.equal(hit, torch.tensor(bh)), "corm any(p >= 1/(i+1)) vs brute"
    # key 0 is the whole row 0 (p = 1 >= 1): always selected
    assert hit[..., 0].all()
    # q = 0: every visible p is exactly 1/(i+1), equal to the threshold, so ">=" selects every key (">" would not)
    out0, hit0, _ = oa.corm(torch.zeros_like(q), k, v, thr)
    assert hit0.all()
    assert torch.equal(thr[3], torch.full((18,), 1.0 / 4, dtype=torch.float32))


def test_kv_gather_matches_loops():
    g = torch.Generator().manual_seed(8)
    B, S, H, D, n = 2, 30, 3, 8, 7
    k = torch.randn(B, S, H, D, generator=g).half()
    v = torch.randn(B, S, H, D, generator=g).half()
    idx = torch.stack([torch.stack([torch.sort(torch.randperm(S, generator=g)[:n])[0] for _ in range(H)])
                       for _ in range(B)])
    kv = osel.kv_gather(k, v, idx)
    assert kv.shape == (B, 2, n, H, D)
    for b in range(B):
        for h in range(H):
            for i in range(n):
                j = int(idx[b, h, i])
                assert torch.equal(kv[b, 0, i, h], k[b, j, h]) and torch.equal(kv[b, 1, i, h], v[b, j, h])
    ident = torch.arange(n).view(1, 1, n).expand(B, H, n).contiguous()
    assert torch.equal(osel.kv_gather(k, v, ident)[:, 0], k[:, :n])


def test_keyformer_matches_brute_and_invariants():
    q, k, v = _sel_inputs(9, S=19)
    er = oa.exp_rand(1, 2, 19, 19, torch.Generator().manual_seed(3))
    assert (er >= 1).all()
    out, score, lse2p = oa.keyformer(q, k, v, er, tau=1.5)
    want = brute.keyformer_colsum(q.tolist(), k.tolist(), er.tolist(), tau=1.5)
    assert_close(score, torch.tensor(want), 1e-6, 1e-5, "keyformer kf_score vs brute")
    # every perturbed softmax row sums to 1; the last key is seen by the last query alone
    assert_close(score.sum(-1), torch.full((1, 2), 19.0), 0, 1e-5, "sum of kf scores = q_len")
    assert_close(out, oa.attention(q, k, v), 0, 0, "keyformer out == attention")
    # exp_rand = 1 (gumbels 0) and tau = 1 reduce to the H2O column sums exactly; tau = 2 halves the logits
    ones = torch.ones_like(er)
    assert_close(oa.keyformer(q, k, v, ones, tau=1.0)[1], oa.h2o(q, k, v)[1], 0, 0, "kf(e=1, tau=1) == h2o")
    half = brute.keyformer_colsum((q / 2).tolist(), k.tolist(), ones.tolist(), tau=1.0)
    assert_close(oa.keyformer(q, k, v, ones, tau=2.0)[1], torch.tensor(half), 1e-6, 1e-5, "tau = 2 == q / 2")
    # the row lse of the perturbed scores: row 0 sees key 0 only, so lse2p = (s_00 - ln e_00) / tau / ln 2
    s00 = float((q[0, 0, 0] @ k[0, 0, 0]) / math.sqrt(8))
    assert abs(float(lse2p[0, 0, 0]) - (s00 - math.log(float(er[0, 0, 0, 0]))) / 1.5 / math.log(2)) < 1e-5


def test_nonzero_matches_loops():
    g = torch.Generator().manual_seed(12)
    x = torch.rand(2, 3, 17, generator=g) < 0.3
    got = osel.nonzero(x)
    want = [[b, h, j] for b in range(2) for h in range(3) for j in range(17) if bool(x[b, h, j])]
    assert got.dtype == torch.int64 and got.tolist() == want
    assert osel.nonzero(torch.zeros(4, 5, dtype=torch.bool)).shape == (0, 2)


def _rope_cache(max_pos, rot_dim, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    ang = torch.rand(max_pos, rot_dim // 2, generator=g, dtype=torch.float64) * 40.0
    return torch.cat([ang.cos(), ang.sin()], dim=1).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rotary_cache_rounding_points_against_torch_16bit_arithmetic(dtype):
    # the reference computes in its scalar_t: c10 Half / BFloat16 operators compute in float and round each product and
    # the result; torch's own 16-bit CPU tensor arithmetic does the same, so x*c - y*s written with 16-bit tensors
    # must give the oracle's bits for both pairings and a partial rot_dim
    g = torch.Generator().manual_seed(3)
    T, H, hs, rot = 7, 3, 64, 48
    cache = _rope_cache(50, rot, dtype, 4)
    pos = torch.randint(0, 50, (T,), generator=g, dtype=torch.int32)
    q = (torch.randn(T, H * hs, generator=g) * 3).to(dtype)
    for neox in (True, False):
        got, _ = oe.rotary_embedding(pos, q, None, hs, cache, neox)
        x = q.reshape(T, H, hs)
        c = cache[pos.long(), : rot // 2].unsqueeze(1)
        s = cache[pos.long(), rot // 2:].unsqueeze(1)
        a, b = (x[..., : rot // 2], x[..., rot // 2: rot]) if neox else (x[..., 0:rot:2], x[..., 1:rot:2])
        want = x.clone()
        if neox:
            want[..., : rot // 2], want[..., rot // 2: rot] = a * c - b * s, b * c + a * s
        else:
            want[..., 0:rot:2], want[..., 1:rot:2] = a * c - b * s, b * c + a * s
        assert torch.equal(got.reshape(T, H, hs), want), f"neox={neox}"
        assert torch.equal(got.reshape(T, H, hs)[..., rot:], x[..., rot:]), "dims past rot_dim must be unchanged"
    # and the roundings are observable: a single rounding of x*c - y*s differs on these inputs
    single = (a.float() * c.float() - b.float() * s.float()).to(dtype)
    assert not torch.equal(single, (a * c - b * s)), "inputs must make the product roundings observable"


def test_rotary_cache_pairing_and_layout():
    # NeoX with the cache of the online angles equals the online rotary (fp32); GPT-J on interleaved pairs equals NeoX on
    # the same pairs laid out as halves; an identity cache (cos 1, sin 0) changes nothing
    T, H, hs = 5, 2, 128
    g = torch.Generator().manual_seed(8)
    pos = torch.randint(0, 3000, (T,), generator=g, dtype=torch.int32)
    q = torch.randn(T, H * hs, generator=g)
    c, s = oe.rotary_cos_sin(torch.arange(3000, dtype=torch.int32), hs, 10000.0)
    cache = torch.cat([c, s], dim=1)
    got, _ = oe.rotary_embedding(pos, q, None, hs, cache, True)
    ref, _ = oe.rotary_embedding_online(pos, q, None, hs, 10000.0)
    assert_close(got, ref, 2e-6, 2e-6, "neox cache vs online")
    x = q.reshape(T, H, hs)
    inter = torch.stack([x[..., : hs // 2], x[..., hs // 2:]], dim=-1).reshape(T, H * hs)  # (x_i, y_i) adjacent
    gj, _ = oe.rotary_embedding(pos, inter, None, hs, cache, False)
    gj = gj.reshape(T, H, hs // 2, 2)
    assert torch.equal(torch.cat([gj[..., 0], gj[..., 1]], dim=-1), got.reshape(T, H, hs))
    ident = torch.cat([torch.ones(10, 32), torch.zeros(10, 32)], dim=1).half()
    qh = q.half()
    for neox in (True, False):
        assert torch.equal(oe.rotary_embedding(pos % 10, qh, None, hs, ident, neox)[0], qh)


def test_rotary_cache_brute_force_fp32():
    # float64 loops over every pair against the fp32 oracle
    T, H, hs, rot = 3, 2, 32, 16
    g = torch.Generator().manual_seed(9)
    pos = torch.randint(0, 20, (T,), generator=g, dtype=torch.int32)
    q = torch.randn(T, H * hs, generator=g)
    k = torch.randn(T, 1 * hs, generator=g)
    cache = _rope_cache(20, rot, torch.float32, 10)
    for neox in (True, False):
        gq, gk = oe.rotary_embedding(pos, q, k, hs, cache, neox)
        for t_in, t_out in ((q, gq), (k, gk)):
            want = t_in.double().clone()
            for t in range(T):
                cr = cache[int(pos[t])].double()
                for h in range(t_in.shape[1] // hs):
                    for i in range(rot // 2):
                        xi, yi = (i, rot // 2 + i) if neox else (2 * i, 2 * i + 1)
                        x, y = t_in[t, h * hs + xi].double(), t_in[t, h * hs + yi].double()
                        want[t, h * hs + xi] = x * cr[i] - y * cr[rot // 2 + i]
                        want[t, h * hs + yi] = y * cr[i] + x * cr[rot // 2 + i]
            assert_close(t_out, want, 1e-6, 1e-6, f"brute force neox={neox}")
