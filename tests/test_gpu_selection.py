"""GPU parity of the other KV-selection cases of the reference (RoCo, SnapKV, Corm, KeyFormer) and of the selection ops
around them (pooling, KV-cache compaction), against the CPU oracle on identical seeded inputs."""
import numpy as np
import pytest
import torch

from conftest import assert_close, progress
from deepgengraph_amd import _lib
from deepgengraph_amd import attention as A
from deepgengraph_amd.compile import compile as dgg_compile
from oracle import attention as oa
from oracle import cases as ocases
from oracle import selection as osel

pytestmark = pytest.mark.gpu

TOL_F16 = (1e-2, 5e-3)


def _qkv(S, H, D, seed, dtype=torch.float16, sinks=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, S, H, D, generator=g)
    k = torch.randn(1, S, H, D, generator=g)
    v = torch.randn(1, S, H, D, generator=g)
    if sinks:
        k[:, torch.randperm(S, generator=g)[:sinks]] *= 4.0
    return q.to(dtype), k.to(dtype), v.to(dtype)


def _corm_check(hit, q, k, v, thr, what):
    """Booleans must equal the oracle's; a differing key is accepted only when its deciding comparison is a
    tie to within 2e-6 relative (max_i (p - thr) / thr ~ 0), where fp32 rounding order decides."""
    _, ref, _ = oa.corm(q, k, v, thr)
    diff = hit.cpu() != ref
    if diff.any():
        rows, _, _ = oa._causal_probs(q, k, v, 256)
        rel = torch.full(ref.shape, float("-inf"))
        for i0, n, probs in rows:
            t = thr[i0:i0 + n]
            rel = torch.maximum(rel, ((probs - t) / t).amax(dim=2))
        assert (rel[diff].abs() < 2e-6).all(), f"{what}: {int(diff.sum())} keys differ away from a tie"
    return int(diff.sum())


@pytest.mark.parametrize("S,H,D", [(300, 2, 128), (1000, 4, 128), (257, 2, 64)])
def test_roco_matches_oracle(gpu, S, H, D):
    progress(f"roco S{S} H{H} D{D}")
    q, k, v = _qkv(S, H, D, S + D, sinks=4)
    ref_out, ref_s1, ref_s2, _ = oa.roco(q, k, v)
    out, s1, s2 = A.roco_attention(q.to(gpu), k.to(gpu), v.to(gpu))
    what = f"roco S{S} H{H} D{D}"
    assert_close(out.cpu().float(), ref_out.float(), *TOL_F16, what + " out")
    assert_close(s1.cpu(), ref_s1, 1e-6, 1e-3, what + " roco_score")
    assert_close(s2.cpu(), ref_s2, 1e-6, 1e-3, what + " roco_sq_score")
    assert_close(s1.sum(-1).cpu(), torch.full((1, H), float(S)), 0, 1e-4, what + " sum of colsums = q_len")


@pytest.mark.parametrize("S,H,D,ks", [(300, 2, 128, 5), (777, 2, 128, 3), (257, 2, 64, 5)])
def test_snapkv_matches_oracle(gpu, S, H, D, ks):
    progress(f"snapkv S{S} H{H} D{D} k{ks}")
    q, k, v = _qkv(S, H, D, 2 * S + D)
    ref_out, ref_score, _ = oa.snapkv(q, k, v, kernel_size=ks)
    out, score = A.snapkv_attention(q.to(gpu), k.to(gpu), v.to(gpu), kernel_size=ks)
    assert_close(out.cpu().float(), ref_out.float(), *TOL_F16, "snapkv out")
    assert_close(score.cpu(), ref_score, 1e-6, 1e-3, "snapkv_score")


@pytest.mark.parametrize("S,H,D", [(300, 2, 128), (1000, 2, 128), (257, 2, 64)])
def test_corm_matches_oracle(gpu, S, H, D):
    progress(f"corm S{S} H{H} D{D}")
    q, k, v = _qkv(S, H, D, 3 * S + D, sinks=3)
    thr = oa.corm_mask(S, S)
    out, hit = A.corm_attention(q.to(gpu), k.to(gpu), v.to(gpu), thr.to(gpu))
    assert hit.dtype == torch.bool and hit.shape == (1, H, S)
    ref_out, ref_hit, _ = oa.corm(q, k, v, thr)
    assert_close(out.cpu().float(), ref_out.float(), *TOL_F16, "corm out")
    _corm_check(hit, q, k, v, thr, f"corm S{S} H{H} D{D}")
    assert hit[..., 0].all()  # row 0 attends key 0 with p = 1 >= 1
    # q = 0: every visible p equals its threshold 1/(i+1) exactly, so every key is selected
    _, hit0 = A.corm_attention(torch.zeros_like(q).to(gpu), k.to(gpu), v.to(gpu), thr.to(gpu))
    assert hit0.all()


@pytest.mark.parametrize("S,H,D,aligned", [(300, 2, 128, True), (1000, 2, 128, True), (257, 2, 64, True),
                                            (301, 2, 128, False)])
def test_keyformer_matches_oracle(gpu, S, H, D, aligned):
    progress(f"keyformer S{S} H{H} D{D} aligned={aligned}")
    q, k, v = _qkv(S, H, D, 4 * S + D, sinks=4)
    g = torch.Generator().manual_seed(S)
    er = oa.exp_rand(1, H, S, S, g)
    if aligned:
        er_dev = er.to(gpu)
    else:  # rows of S + 1 floats from an offset of one element: the unaligned (4-byte load) path
        big = torch.ones(1, H, S, S + 2)
        big[..., 1:S + 1] = er
        er_dev = big.to(gpu)[..., 1:S + 1]
    out, score = A.keyformer_attention(q.to(gpu), k.to(gpu), v.to(gpu), er_dev, tau=1.5)
    ref_out, ref_score, _ = oa.keyformer(q, k, v, er, tau=1.5)
    what = f"keyformer S{S} H{H} D{D}"
    assert_close(out.cpu().float(), ref_out.float(), *TOL_F16, what + " out")
    assert_close(score.cpu(), ref_score, 1e-6, 1e-3, what + " kf_score")
    assert_close(score.sum(-1).cpu(), torch.full((1, H), float(S)), 0, 1e-4, what + " sum of kf scores = q_len")


def test_keyformer_wide_exp_rand_rows(gpu):
    # exp_rand rows 4.1M floats apart: the column pass's 32-bit tile offsets do not fit, every tile takes the
    # general addressing (a 4.2 GB device buffer of which the [256, 256] corner is used)
    S, H, D = 256, 1, 128
    progress("keyformer wide exp_rand rows")
    q, k, v = _qkv(S, H, D, 77, sinks=2)
    er = oa.exp_rand(1, H, S, S, torch.Generator().manual_seed(78))
    wide = 4_100_000
    buf = torch.empty(S, wide, dtype=torch.float32, device=gpu)
    buf[:, :S] = er[0, 0].to(gpu)
    er_dev = buf[:, :S].view(1, 1, S, S)
    out, score = A.keyformer_attention(q.to(gpu), k.to(gpu), v.to(gpu), er_dev, tau=1.5)
    ref_out, ref_score, _ = oa.keyformer(q, k, v, er, tau=1.5)
    assert_close(out.cpu().float(), ref_out.float(), *TOL_F16, "keyformer wide out")
    assert_close(score.cpu(), ref_score, 1e-6, 1e-3, "keyformer wide kf_score")
    del buf


@pytest.mark.parametrize("kind", ["never", "some_keys", "late_rows", "zero", "nan_inf"])
def test_corm_thresholds_that_decide_late_or_never(gpu, kind):
    # The head_dim-128 Corm column pass stops a workgroup once every key of every wave is flagged. These
    # thresholds keep keys undecided for the whole pass (never: p <= 1 < 2), for some key ranges only, until the
    # last rows, or decide them at once (zero); NaN never selects, -inf always does.
    S, H, D = 1100, 2, 128
    q, k, v = _qkv(S, H, D, 5 * S + len(kind), sinks=4)
    g = torch.Generator().manual_seed(17)
    thr = oa.corm_mask(S, S).clone()
    if kind == "never":
        thr.fill_(2.0)
    elif kind == "some_keys":
        thr[:, 300:700] = 2.0  # keys of these columns never pass; the others decide as usual
    elif kind == "late_rows":
        thr[: S - 40] = 2.0    # only the last 40 rows can flag anything
    elif kind == "zero":
        thr.zero_()            # p >= 0 everywhere, masked pairs included
    else:
        thr = torch.rand(S, S, generator=g)
        thr[torch.rand(S, S, generator=g) < 0.3] = float("nan")
        thr[torch.rand(S, S, generator=g) < 0.01] = float("-inf")
    progress(f"corm thresholds {kind}")
    _, hit = A.corm_attention(q.to(gpu), k.to(gpu), v.to(gpu), thr.to(gpu))
    n = _corm_check(hit, q, k, v, thr, f"corm thresholds {kind}")
    if kind == "never":
        assert not hit.any()
    if kind == "zero":
        assert hit.all()
    if kind == "some_keys":
        assert not hit[..., 300:700].any() and n == 0


def _corm_reference(q, k, thr, causal, window):
    """corm.py:35-37 over every query row: probs >= thr with the reference's probabilities (scores rounded in the
    input dtype, masked pairs -inf, so p = 0 there and NaN on rows that see no key), any over the rows. Also
    returns the float64 probabilities for the tie check."""
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    s = oa._scores(q.transpose(1, 2), k.transpose(1, 2).transpose(-2, -1), D).float()
    m = oa._mask(0, Sq, Sq, Sk, causal, window or None)
    if m is not None:
        s = s.masked_fill(m, float("-inf"))
    probs = torch.softmax(s, -1)
    return (probs >= thr).any(dim=2), probs.double()


@pytest.mark.parametrize("D,dtype,Sq,Sk,causal,window", [
    (128, torch.float16, 600, 600, True, 0),
    (128, torch.float16, 700, 400, True, 0),      # Sq > Sk: the first 300 rows see no key (NaN probabilities)
    (128, torch.bfloat16, 500, 500, True, 97),    # causal + window: masked pairs on both sides
    (128, torch.float16, 300, 450, False, 80),    # window without causal
    (64, torch.float16, 400, 300, True, 0),       # the generic column kernel
    (256, torch.bfloat16, 300, 300, True, 50),
    (128, torch.float32, 300, 200, True, 0),      # the fp32 column kernel
])
def test_corm_masked_pairs_and_empty_rows(gpu, D, dtype, Sq, Sk, causal, window):
    # thresholds 2 (never passed) except: <= 0 at random masked pairs, and at every pair of the rows that see
    # no key; plus random positive thresholds on a band so that visible pairs flag some keys too
    g = torch.Generator().manual_seed(D + Sq + Sk + window)
    q = torch.randn(1, Sq, 2, D, generator=g).to(dtype)
    k = torch.randn(1, Sk, 2, D, generator=g).to(dtype)
    v = torch.randn(1, Sk, 2, D, generator=g).to(dtype)
    thr = torch.full((Sq, Sk), 2.0)
    hidden = oa._mask(0, Sq, Sq, Sk, causal, window or None)
    pick = torch.rand(Sq, Sk, generator=g) < 0.002
    thr[hidden & pick] = torch.tensor([0.0, -0.0, -1.0, float("-inf")])[torch.randint(0, 4, (int((hidden & pick).sum()),),
                                                                                      generator=g)]
    if Sq > Sk and causal:
        thr[: Sq - Sk] = -1.0  # rows that see no key: NaN >= -1 is False, they flag nothing
    band = torch.rand(Sq, Sk, generator=g) < 0.05
    thr[band & ~hidden] = 0.02
    progress(f"corm masked pairs D{D} {dtype} Sq{Sq} Sk{Sk} causal={causal} w={window}")
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    _, lse = A.attention(qg, kg, vg, causal=causal, window=window, return_lse=True, ref_rounding=True, lse_base2=True)
    hit = A.attention_colscore(qg, kg, lse, epilogue=_lib.COL_ANY_GE, thr=thr.to(gpu), causal=causal, window=window,
                               lse_base2=True).cpu()
    ref, probs = _corm_reference(q, k, thr, causal, window)
    diff = hit != ref
    if diff.any():  # only a visible pair whose p ties its threshold to fp32 rounding may differ
        b, h, j = diff.nonzero()[0].tolist()
        col_p, col_t = probs[b, h, :, j], thr[:, j].double()
        assert ((col_p - col_t).abs() / col_t.abs() < 2e-6).any(), f"key {j} head {h} differs away from a tie"
    assert hit.any() and not hit.all()


def test_colscore_thresholds_and_strides(gpu):
    # a strided threshold view and an arbitrary threshold: any(p >= t) with t = 0.05 everywhere
    S, H, D = 200, 2, 128
    q, k, v = _qkv(S, H, D, 91)
    big = torch.full((S, S + 40), 0.05, dtype=torch.float32)
    thr = big[:, 8:8 + S]
    out, hit = A.corm_attention(q.to(gpu), k.to(gpu), v.to(gpu), big.to(gpu)[:, 8:8 + S])
    _corm_check(hit, q, k, v, thr.contiguous(), "corm strided threshold")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_kv_gather_matches_oracle(gpu, dtype):
    g = torch.Generator().manual_seed(5)
    B, S, H, D, n = 2, 500, 4, 128, 64
    k = torch.randn(B, S, H, D, generator=g).to(dtype)
    v = torch.randn(B, S, H, D, generator=g).to(dtype)
    idx = torch.stack([torch.stack([torch.sort(torch.randperm(S, generator=g)[:n])[0] for _ in range(H)])
                       for _ in range(B)]).contiguous()
    got = A.kv_gather(k.to(gpu), v.to(gpu), idx.to(gpu)).cpu()
    assert torch.equal(got, osel.kv_gather(k, v, idx))
    # strided k/v views (the fused QKV activation), and indices outside [0, S) -> zero rows
    kv = torch.randn(B, S, H, 3 * D, generator=g).to(dtype)
    kview, vview = kv[..., :D], kv[..., D:2 * D]
    bad = idx.clone()
    bad[0, 1, 3] = -1
    bad[1, 2, 7] = S
    got = A.kv_gather(kview.to(gpu), vview.to(gpu), bad.to(gpu)).cpu()
    want = osel.kv_gather(kview.contiguous(), vview.contiguous(), bad.clamp(0, S - 1))
    want[0, :, 3, 1] = 0
    want[1, :, 7, 2] = 0
    assert torch.equal(got, want)


@pytest.mark.parametrize("shape,density", [((1, 32, 4096), 0.02), ((2, 3, 1000), 0.5), ((5,), 0.6),
                                           ((3, 2, 2, 300), 1.0), ((4, 700), 0.0), ((3, 0), 0.5)])
def test_nonzero_matches_oracle(gpu, shape, density):
    g = torch.Generator().manual_seed(len(shape) * 7 + int(density * 10))
    x = torch.rand(*shape, generator=g) < density
    got = A.nonzero(x.to(gpu))
    want = osel.nonzero(x)
    assert got.dtype == torch.int64 and got.shape == want.shape, (got.shape, want.shape)
    assert torch.equal(got.cpu(), want)
    if x.numel():
        assert torch.equal(A.nonzero(x.to(torch.uint8).to(gpu)).cpu(), want)  # uint8 input


def test_corm_selection_nonzero(gpu):
    # models/corm.py:45-55: the keys Corm flags, as coordinates (b, h, j) in row-major order
    S, H, D = 500, 3, 128
    q, k, v = _qkv(S, H, D, 17, sinks=3)
    thr = oa.corm_mask(S, S)
    _, hit = A.corm_attention(q.to(gpu), k.to(gpu), v.to(gpu), thr.to(gpu))
    sel = A.nonzero(hit)
    assert torch.equal(sel.cpu(), torch.nonzero(hit.cpu()))
    assert sel.shape[1] == 3 and (sel[:, 2] == 0).sum().item() == H  # key 0 is flagged in every head


def test_avg_pool1d_matches_oracle(gpu):
    x = torch.randn(6, 1000, generator=torch.Generator().manual_seed(2))
    for ks in (1, 3, 5, 9):
        assert_close(A.avg_pool1d(x.to(gpu), ks).cpu(), osel.avg_pool1d(x, ks), 1e-6, 1e-6, f"pool k={ks}")


@pytest.mark.parametrize("case_cls", [ocases.RoCo, ocases.SnapKV, ocases.Corm, ocases.KeyFormer])
def test_compile_drop_in_selection_cases(gpu, case_cls):
    # run_kernel.py:44-78 flow for the other selection cases
    model = case_cls(kv_head_num=4, head_num=4, head_dim=128).eval()
    specs = model.prepare(q_len=384, kv_len=384, dtype=torch.float16, seed=11)
    names = list(specs["input"].keys())
    inputs = [specs["input"][n] for n in names]
    f = dgg_compile(model=model, input_names=names, inputs=inputs, output_names=specs["output"], system="mi355x")
    outs = f(*[t.to(gpu) for t in inputs])
    refs = model(*inputs)
    assert isinstance(outs, tuple) and len(outs) == len(refs) == len(specs["output"])
    assert_close(outs[0].cpu().float(), refs[0].float(), *TOL_F16, f"{case_cls.__name__} out")
    for o, r in zip(outs[1:], refs[1:]):
        assert o.shape == r.shape and o.dtype == r.dtype
        if r.dtype == torch.bool:
            _corm_check(o, *[t for t in inputs[:3]], inputs[3], "compiled corm")
        else:
            assert_close(o.cpu(), r, 1e-6, 1e-3, f"{case_cls.__name__} score")


def test_selection_full_size_heads(gpu):
    # config-4 shapes (fp16, S = 4096, D = 128) on two heads: RoCo sums and Corm flags against the oracle,
    # then the top-256 selection and the compaction of the selected rows
    S, H, D = 4096, 2, 128
    progress("selection full size: oracle")
    q, k, v = _qkv(S, H, D, 4096, sinks=16)
    _, ref_s1, ref_s2, _ = oa.roco(q, k, v, q_chunk=512)
    progress("selection full size: gpu")
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    out, s1, s2 = A.roco_attention(qg, kg, vg)
    assert_close(s1.cpu(), ref_s1, 1e-6, 1e-3, "roco_score full")
    assert_close(s2.cpu(), ref_s2, 1e-6, 1e-3, "roco_sq_score full")
    idx = A.topk_indices(s1, 256)
    np.testing.assert_array_equal(idx.cpu().numpy(), osel.topk_indices(ref_s1.numpy(), 256))
    kv = A.kv_gather(kg, vg, idx).cpu()
    assert torch.equal(kv, osel.kv_gather(k, v, idx.cpu()))
    thr = oa.corm_mask(S, S)
    _, hit = A.corm_attention(qg, kg, vg, thr.to(gpu))
    n = _corm_check(hit, q, k, v, thr, "corm full")
    progress(f"corm full: {n} tie-decided keys")
    progress("keyformer full size")
    er = oa.exp_rand(1, H, S, S, torch.Generator().manual_seed(4))
    _, ref_kf, _ = oa.keyformer(q, k, v, er, q_chunk=512)
    _, kf = A.keyformer_attention(qg, kg, vg, er.to(gpu))
    assert_close(kf.cpu(), ref_kf, 1e-6, 1e-3, "kf_score full")
    np.testing.assert_array_equal(A.topk_indices(kf, 256).cpu().numpy(), osel.topk_indices(ref_kf.numpy(), 256))
