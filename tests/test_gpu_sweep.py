"""Seeded random sweeps over the launch space of the forward and selection entry points, against the CPU oracle at the
tolerances of test_gpu_attention.py (bf16 2e-2 abs / 1e-2 rel, fp16 1e-2 / 5e-3; index sets identical). Each seed
draws one configuration: head_dim, grouped query heads, causal / window / soft-cap, ragged and unequal Sq / Sk (so
one-row calls go to the decode kernels and short query blocks to the split-KV kernels, as attention() routes them),
dtype; rows of tie-heavy, NaN-holding or continuous scores, of 1 to 70,000 keys, for the selections; drawn widths
and dtypes for the elementwise ops; drawn shapes and sinks for the RoCo, SnapKV, Corm and KeyFormer cases; drawn
caches, split counts, indices and masks for decode, the KV-cache compaction, nonzero and the pooling. The case is
printed before it runs. The column-score cases compare with the reference probabilities of
test_gpu_attention.py (1e-3 rel)."""
import numpy as np
import pytest
import torch

from conftest import assert_close, progress
from deepgengraph_amd import attention as A
from oracle import attention as oa
from oracle import selection as osel

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (1e-2, 5e-3)}


def _draw_attention_case(seed):
    rng = np.random.default_rng(1000 + seed)
    D = int(rng.choice([64, 128, 256]))
    Hkv = int(rng.choice([1, 2]))
    G = int(rng.choice([1, 2, 4]))
    B = int(rng.choice([1, 2]))
    shape = rng.integers(0, 4)
    if shape == 0:  # one query row over a cache (decode kernels when Sk >= 256)
        Sq, Sk = 1, int(rng.integers(1, 1500))
    elif shape == 1:  # a short query block (split-KV kernels over >= 512 keys)
        Sq, Sk = int(rng.integers(2, 65)), int(rng.integers(64, 1500))
    else:
        Sq, Sk = int(rng.integers(1, 600)), int(rng.integers(1, 600))
    causal = bool(rng.integers(0, 2))
    softcap = float(rng.choice([0.0, 0.0, 20.0, 50.0]))
    window = int(rng.integers(1, Sk + 1)) if causal and rng.integers(0, 3) == 0 else 0
    dtype = torch.bfloat16 if rng.integers(0, 2) else torch.float16
    return B, Sq, Sk, Hkv * G, Hkv, D, dtype, causal, softcap, window


@pytest.mark.parametrize("seed", range(64))
def test_attention_random_launches_match_oracle(gpu, seed):
    B, Sq, Sk, Hq, Hkv, D, dtype, causal, softcap, window = _draw_attention_case(seed)
    what = f"seed {seed}: B{B} Sq{Sq} Sk{Sk} H{Hq}/{Hkv} D{D} {dtype} causal={causal} cap={softcap} win={window}"
    progress(what)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Sq, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, Sk, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, Sk, Hkv, D, generator=g).to(dtype)
    ref, ref_lse = oa.attention(q, k, v, causal=causal, softcap=softcap or None, window=window or None,
                                return_lse=True)
    out, lse = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal, softcap=softcap, window=window,
                           return_lse=True)
    assert_close(out.cpu().float(), ref.float(), *TOL[dtype], what + " out")
    lse_c = lse.cpu()
    fin = torch.isfinite(ref_lse)
    assert torch.equal(torch.isfinite(lse_c), fin), what + " lse -inf pattern"
    assert_close(lse_c[fin], ref_lse[fin], 2e-2, 1e-2, what + " lse")


def _draw_rows(rng, rows, n):
    kind = int(rng.integers(0, 4))
    if kind == 0:  # few distinct values: ties decide
        return (rng.integers(0, 7, size=(rows, n)).astype(np.float32) - 3.0) / 2.0, "ties"
    if kind == 1:  # signed zeros, infinities and NaN among ties
        pool = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 2.5], dtype=np.float32)
        return rng.choice(pool, size=(rows, n)), "specials"
    if kind == 2:  # a narrow band: the keys share their leading bytes
        return (1.0 + rng.random((rows, n)) * 1e-3).astype(np.float32), "band"
    return rng.standard_normal((rows, n)).astype(np.float32), "normal"


@pytest.mark.parametrize("seed", range(40))
def test_topk_random_rows_match_oracle(gpu, seed):
    rng = np.random.default_rng(2000 + seed)
    rows = int(rng.integers(1, 6))
    n = int(rng.choice([rng.integers(1, 5000), rng.integers(5000, 65537), rng.integers(65537, 70001)]))
    k = int(rng.choice([1, rng.integers(1, n + 1), min(n, 256), n]))
    largest = bool(rng.integers(0, 2))
    vals, kind = _draw_rows(rng, rows, n)
    what = f"seed {seed}: {rows} x {n} {kind} k={k} largest={largest}"
    progress(what)
    got = A.topk_indices(torch.from_numpy(vals).to(gpu), k, largest=largest).cpu().numpy()
    np.testing.assert_array_equal(got, osel.topk_indices(vals, k, largest), err_msg=what)


@pytest.mark.parametrize("seed", range(24))
def test_roco_select_random_rows_match_oracle(gpu, seed):
    rng = np.random.default_rng(3000 + seed)
    rows = int(rng.integers(1, 4))
    n = int(rng.choice([rng.integers(1, 65537), rng.integers(65537, 70001)]))
    q_len = int(rng.integers(1, 5000))
    recent = int(rng.choice([0, rng.integers(0, n + 1), min(n, 256)]))
    budget = int(rng.choice([0, rng.integers(0, n - recent + 1), min(n - recent, 512)]))
    if rng.integers(0, 2):  # integer sums: ties, and negative variances (NaN std)
        s1 = rng.integers(0, 40, size=(rows, n)).astype(np.float32)
        s2 = rng.integers(0, 60, size=(rows, n)).astype(np.float32) / 2.0
    else:
        s1 = rng.random((rows, n)).astype(np.float32) * q_len
        s2 = s1 * s1 / q_len + rng.random((rows, n)).astype(np.float32)
    what = f"seed {seed}: {rows} x {n} q_len={q_len} recent={recent} budget={budget}"
    progress(what)
    got = A.roco_select(torch.from_numpy(s1).to(gpu), torch.from_numpy(s2).to(gpu), q_len, recent, budget)
    np.testing.assert_array_equal(got.cpu().numpy(), osel.roco_select(s1, s2, q_len, recent, budget), err_msg=what)


@pytest.mark.parametrize("seed", range(32))
def test_colscore_random_launches_match_reference(gpu, seed):
    # the column-score pass (H2O sums, RoCo's sums and sums of squares) after the lse-writing forward with the
    # reference's score rounding, against the reference's probabilities at the column-sum contract (1e-3 rel)
    from deepgengraph_amd import _lib
    from test_gpu_attention import _colsum_check, _colsum_reference

    rng = np.random.default_rng(4000 + seed)
    D = int(rng.choice([64, 128, 256]))
    Hkv = int(rng.choice([1, 2]))
    Hq = Hkv * int(rng.choice([1, 2]))
    Sq, Sk = int(rng.integers(1, 700)), int(rng.integers(1, 700))
    causal = bool(rng.integers(0, 2))
    sumsq = bool(rng.integers(0, 2))
    softcap = 0.0 if sumsq else float(rng.choice([0.0, 0.0, 30.0]))
    window = int(rng.integers(1, Sk + 1)) if causal and rng.integers(0, 3) == 0 else 0
    dtype = torch.bfloat16 if rng.integers(0, 2) else torch.float16
    base2 = bool(rng.integers(0, 2))
    what = (f"seed {seed}: Sq{Sq} Sk{Sk} H{Hq}/{Hkv} D{D} {dtype} causal={causal} cap={softcap} win={window} "
            f"base2={base2} sumsq={sumsq}")
    progress(what)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, Sq, Hq, D, generator=g).to(dtype)
    k = torch.randn(1, Sk, Hkv, D, generator=g).to(dtype)
    v = torch.randn(1, Sk, Hkv, D, generator=g).to(dtype)
    kw = dict(causal=causal, window=window, lse_base2=base2)
    _, lse = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), return_lse=True, ref_rounding=True, softcap=softcap, **kw)
    if sumsq:
        s1, s2 = A.attention_colscore(q.to(gpu), k.to(gpu), lse, epilogue=_lib.COL_SUM_SQ, ref_rounding=True, **kw)
        _colsum_check(s1.cpu(), _colsum_reference(q, k, causal, 0.0, window).float(), what + " sum")
        _colsum_check(s2.cpu(), _colsum_reference(q, k, causal, 0.0, window, power=2).float(), what + " sum of squares")
    else:
        cs = A.attention_colsum(q.to(gpu), k.to(gpu), lse, softcap=softcap, **kw).cpu()
        _colsum_check(cs, _colsum_reference(q, k, causal, softcap, window).float(), what + " sum")


@pytest.mark.parametrize("seed", range(8))
def test_colscore_long_random_launches_match_reference(gpu, seed):
    # the head_dim-128 column pass on drawn shapes long enough for long software-pipelined runs of its 64-key waves
    # (several 128-row query tiles per wave, ragged ends, windows, GQA), H2O sums or RoCo's sums and sums of squares,
    # against the reference's probabilities at the column-sum contract (1e-3 rel)
    from deepgengraph_amd import _lib
    from test_gpu_attention import _colsum_check, _colsum_reference

    rng = np.random.default_rng(4500 + seed)
    D = 128
    Hkv = int(rng.choice([1, 2]))
    Hq = Hkv * int(rng.choice([1, 2]))
    Sq, Sk = int(rng.integers(700, 2400)), int(rng.integers(700, 2400))
    causal = bool(rng.integers(0, 4))
    sumsq = bool(rng.integers(0, 2))
    softcap = 30.0 if not sumsq and rng.integers(0, 4) == 0 else 0.0
    window = int(rng.integers(1, Sk + 1)) if causal and rng.integers(0, 3) == 0 else 0
    dtype = torch.bfloat16 if rng.integers(0, 2) else torch.float16
    base2 = bool(rng.integers(0, 2))
    what = (f"seed {seed}: Sq{Sq} Sk{Sk} H{Hq}/{Hkv} D{D} {dtype} causal={causal} cap={softcap} win={window} "
            f"base2={base2} sumsq={sumsq}")
    progress(what)
    g = torch.Generator().manual_seed(100 + seed)
    q = torch.randn(1, Sq, Hq, D, generator=g).to(dtype)
    k = torch.randn(1, Sk, Hkv, D, generator=g).to(dtype)
    v = torch.randn(1, Sk, Hkv, D, generator=g).to(dtype)
    kw = dict(causal=causal, window=window, lse_base2=base2)
    _, lse = A.attention(q.to(gpu), k.to(gpu), v.to(gpu), return_lse=True, ref_rounding=True, softcap=softcap, **kw)
    # bf16 scores: two fp32 accumulation orders of the same dot product (the MFMA's, the CPU matmul's, which itself
    # varies with the host's instruction set) can round to neighbouring bf16 values, which moves that probability
    # by up to |s| * 2^-8; in a short windowed column one such score can shift a sum of squares by ~1e-3. The exact
    # invariant below (each row that sees a key contributes 1 to the sums) holds either way.
    def check(got, ref, label):
        if dtype == torch.bfloat16:
            assert_close(got, ref, 1e-6, 4e-3, what + label)
        else:
            _colsum_check(got, ref, what + label)
    if sumsq:
        s1, s2 = A.attention_colscore(q.to(gpu), k.to(gpu), lse, epilogue=_lib.COL_SUM_SQ, ref_rounding=True, **kw)
        ref1 = _colsum_reference(q, k, causal, 0.0, window)
        check(s1.cpu(), ref1.float(), " sum")
        check(s2.cpu(), _colsum_reference(q, k, causal, 0.0, window, power=2).float(), " sum of squares")
        got1, rows = s1.cpu(), ref1.sum(-1)
    else:
        ref1 = _colsum_reference(q, k, causal, softcap, window)
        got1 = A.attention_colsum(q.to(gpu), k.to(gpu), lse, softcap=softcap, **kw).cpu()
        check(got1, ref1.float(), " sum")
        rows = ref1.sum(-1)
    assert_close(got1.double().sum(-1), torch.round(rows), 0, 1e-5, what + " sum over keys = rows that see a key")


def _draw_width(rng):
    """A row width: a multiple of 8 (the vector paths) or not (the scalar ones), small or wide."""
    w = int(rng.integers(1, 8193))
    return w - w % 8 if rng.integers(0, 2) and w >= 8 else w


@pytest.mark.parametrize("seed", range(24))
def test_elementwise_random_shapes_match_oracle(gpu, seed):
    # RMSNorm, fused add + RMSNorm, SiLU-and-mul and the online rotary (csrc/norm.cu, activation.cu,
    # pos_encoding.cu) on drawn shapes and dtypes, through the csrc-compatible wrappers
    from deepgengraph_amd import ops
    from oracle import elementwise as oe

    rng = np.random.default_rng(5000 + seed)
    dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    tol = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (1e-2, 5e-3), torch.float32: (1e-5, 1e-5)}[dtype]
    g = torch.Generator().manual_seed(seed)
    rows, hidden = int(rng.integers(1, 300)), _draw_width(rng)
    what = f"seed {seed}: rms_norm {rows}x{hidden} {dtype}"
    progress(what)
    x = torch.randn(rows, hidden, generator=g).to(dtype)
    r = torch.randn(rows, hidden, generator=g).to(dtype)
    w = (1.0 + 0.02 * torch.randn(hidden, generator=g)).to(dtype)
    out = torch.empty(rows, hidden, dtype=dtype, device=gpu)
    ops.rms_norm(out, x.to(gpu), w.to(gpu), 1e-6)
    assert_close(out.cpu().float(), oe.rms_norm(x, w, 1e-6).float(), *tol, what)
    ref_out, ref_res = oe.fused_add_rms_norm(x, r, w, 1e-6)
    xg, rg = x.to(gpu), r.to(gpu)
    ops.fused_add_rms_norm(xg, rg, w.to(gpu), 1e-6)
    assert torch.equal(rg.cpu(), ref_res), what + ": fused residual = T(input + residual) must be exact"
    assert_close(xg.cpu().float(), ref_out.float(), *tol, what + " fused")

    arows, d = int(rng.integers(1, 300)), _draw_width(rng)
    what = f"seed {seed}: silu_and_mul {arows}x{d} {dtype}"
    progress(what)
    gu = (3.0 * torch.randn(arows, 2 * d, generator=g)).to(dtype)
    act = torch.empty(arows, d, dtype=dtype, device=gpu)
    ops.silu_and_mul(act, gu.to(gpu))
    assert_close(act.cpu().float(), oe.silu_and_mul(gu).float(), *tol, what)

    tokens, hk = int(rng.integers(1, 200)), int(rng.integers(1, 5))
    # head_dim: multiples of 16 up to 256 (the wrapper's range; the reference asserts 128, pos_encoding.cu:193)
    hq, D = hk * int(rng.integers(1, 4)), 16 * int(rng.integers(1, 17))
    pad = int(rng.choice([0, 0, 3, 8]))
    what = f"seed {seed}: rotary T{tokens} {hq}/{hk} D{D} pad{pad} {dtype}"
    progress(what)
    qkv = torch.randn(tokens, (hq + 2 * hk) * D + pad, generator=g).to(dtype)
    pos = torch.randint(0, 8192, (tokens,), generator=g, dtype=torch.int32)
    q, k = qkv[:, : hq * D], qkv[:, hq * D: (hq + hk) * D]
    ref_q, ref_k = oe.rotary_embedding_online(pos, q.contiguous(), k.contiguous(), D, 10000.0)
    qkv_g = qkv.to(gpu)
    gq, gk = qkv_g[:, : hq * D], qkv_g[:, hq * D: (hq + hk) * D]
    ops.rotary_embedding_online(pos.to(gpu), gq, gk, D, 10000.0)
    rtol = tol if dtype != torch.float32 else (3e-3, 1e-3)  # the fp32 angle's own rounding (pos_encoding.cu:84)
    assert_close(gq.cpu().float(), ref_q.float(), *rtol, what + " q")
    assert_close(gk.cpu().float(), ref_k.float(), *rtol, what + " k")
    assert torch.equal(qkv_g[:, (hq + hk) * D:].cpu(), qkv[:, (hq + hk) * D:]), what + ": v part must be untouched"


@pytest.mark.parametrize("seed", range(24))
def test_selection_cases_random_shapes_match_oracle(gpu, seed):
    # RoCo, SnapKV, Corm and KeyFormer (roco.py, snapkv.py, corm.py, kf.py) end to end on drawn shapes, with attention
    # sinks, against the oracle (outputs fp16 1e-2 / 5e-3, scores 1e-3 rel; Corm's booleans up to exact ties)
    from test_gpu_selection import _corm_check, _qkv

    rng = np.random.default_rng(6000 + seed)
    case = ["roco", "snapkv", "corm", "keyformer"][seed % 4]
    S, H, D = int(rng.integers(2, 900)), int(rng.integers(1, 4)), int(rng.choice([64, 128]))
    sinks = int(rng.integers(0, min(S, 8) + 1))
    q, k, v = _qkv(S, H, D, 7000 + seed, sinks=sinks)
    what = f"seed {seed}: {case} S{S} H{H} D{D} sinks{sinks}"
    progress(what)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    if case == "roco":
        ref_out, ref_s1, ref_s2, _ = oa.roco(q, k, v)
        out, s1, s2 = A.roco_attention(qg, kg, vg)
        assert_close(s1.cpu(), ref_s1, 1e-6, 1e-3, what + " roco_score")
        assert_close(s2.cpu(), ref_s2, 1e-6, 1e-3, what + " roco_sq_score")
    elif case == "snapkv":
        ks = int(rng.choice([1, 3, 5, 7]))
        what += f" k{ks}"
        ref_out, ref_score, _ = oa.snapkv(q, k, v, kernel_size=ks)
        out, score = A.snapkv_attention(qg, kg, vg, kernel_size=ks)
        assert_close(score.cpu(), ref_score, 1e-6, 1e-3, what + " snapkv_score")
    elif case == "corm":
        thr = oa.corm_mask(S, S)
        ref_out, _, _ = oa.corm(q, k, v, thr)
        out, hit = A.corm_attention(qg, kg, vg, thr.to(gpu))
        _corm_check(hit, q, k, v, thr, what)
    else:
        tau = float(rng.choice([0.5, 1.0, 1.5, 3.0]))
        what += f" tau{tau}"
        er = oa.exp_rand(1, H, S, S, torch.Generator().manual_seed(seed))
        ref_out, ref_score, _ = oa.keyformer(q, k, v, er, tau=tau)
        out, score = A.keyformer_attention(qg, kg, vg, er.to(gpu), tau=tau)
        assert_close(score.cpu(), ref_score, 1e-6, 1e-3, what + " kf_score")
    assert_close(out.cpu().float(), ref_out.float(), 1e-2, 5e-3, what + " out")


@pytest.mark.parametrize("seed", range(24))
def test_decode_and_kv_ops_random_shapes_match_oracle(gpu, seed):
    # decode_attention on the [B, Hkv, L, D] cache with a drawn split count (1 .. more splits than keys, at most
    # 1,024), the KV-cache compaction with drawn indices, torch.nonzero's coordinates of a drawn mask, and SnapKV's
    # pooling of drawn rows
    rng = np.random.default_rng(8000 + seed)
    B, Hkv = int(rng.integers(1, 4)), int(rng.integers(1, 5))
    Hq, D = Hkv * int(rng.choice([1, 2, 4])), int(rng.choice([64, 128, 256]))
    L = int(rng.integers(1, 3000))
    splits = int(rng.choice([1, rng.integers(1, 65), min(1024, int(rng.integers(1, L + 8)))]))
    dtype = torch.bfloat16 if rng.integers(0, 2) else torch.float16
    what = f"seed {seed}: decode B{B} H{Hq}/{Hkv} L{L} D{D} splits{splits} {dtype}"
    progress(what)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, D, generator=g).to(dtype)
    kc = torch.randn(B, Hkv, L, D, generator=g).to(dtype)
    vc = torch.randn(B, Hkv, L, D, generator=g).to(dtype)
    ref, ref_lse = oa.decode(q, kc, vc)
    out, lse = A.decode_attention(q.to(gpu), kc.to(gpu), vc.to(gpu), splits=splits, return_lse=True)
    assert_close(out.cpu().float(), ref.float(), *TOL[dtype], what)
    assert_close(lse.cpu(), ref_lse, 2e-2, 1e-3, what + " lse")

    S, n = int(rng.integers(1, 2000)), int(rng.integers(1, 600))
    k = torch.randn(B, S, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, S, Hkv, D, generator=g).to(dtype)
    idx = torch.from_numpy(rng.integers(0, S, size=(B, Hkv, n))).long()
    what = f"seed {seed}: kv_gather B{B} S{S} H{Hkv} D{D} n{n}"
    progress(what)
    got = A.kv_gather(k.to(gpu), v.to(gpu), idx.to(gpu)).cpu()
    assert torch.equal(got, osel.kv_gather(k, v, idx)), what

    shape = tuple(int(x) for x in rng.integers(1, 40, size=int(rng.integers(1, 4))))
    mask = torch.from_numpy(rng.random(shape) < rng.random())
    what = f"seed {seed}: nonzero {shape}"
    progress(what)
    assert torch.equal(A.nonzero(mask.to(gpu)).cpu(), osel.nonzero(mask)), what

    x = torch.rand(int(rng.integers(1, 9)), int(rng.integers(1, 5000)), generator=g)
    ks = int(rng.choice([1, 3, 5, 7, 9]))
    what = f"seed {seed}: avg_pool1d {tuple(x.shape)} k{ks}"
    progress(what)
    assert_close(A.avg_pool1d(x.to(gpu), ks).cpu(), osel.avg_pool1d(x, ks), 1e-6, 1e-6, what)
