"""GPU parity of the elementwise kernels (RMSNorm, fused add + RMSNorm, SiLU-and-mul, rotary) against the CPU
oracle on identical seeded inputs, through the csrc-compatible wrappers (C ABI underneath).
Tolerances: bf16 2e-2 abs / 1e-2 rel, fp16 1e-2 / 5e-3, fp32 1e-5 / 1e-5."""
import pytest
import torch

from conftest import assert_close, load_golden
from deepgengraph_amd import ops
from oracle import elementwise as oe

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (1e-2, 5e-3), torch.float32: (1e-5, 1e-5)}


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _randn(shape, dtype, seed, scale=1.0, shift=0.0):
    return (shift + scale * torch.randn(*shape, generator=_gen(seed))).to(dtype)


@pytest.mark.parametrize("rows,hidden,dtype", [
    (4096, 4096, torch.bfloat16),   # config 2
    (64, 4096, torch.float16),      # config 5 pre-step
    (7, 1000, torch.float32),
    (5, 1001, torch.float16),       # odd width: scalar path
    (3, 65536, torch.bfloat16),     # widest vector path
    (2, 128, torch.bfloat16),
    (130, 1024, torch.float16),
    (9, 5120, torch.bfloat16),
])
def test_rms_norm(gpu, rows, hidden, dtype):
    x = _randn((rows, hidden), dtype, 1)
    w = _randn((hidden,), dtype, 2, 0.02, 1.0)
    ref = oe.rms_norm(x, w, 1e-6)
    out = torch.empty(rows, hidden, dtype=dtype, device=gpu)
    ops.rms_norm(out, x.to(gpu), w.to(gpu), 1e-6)
    got = out.cpu()
    assert_close(got.float(), ref.float(), *TOL[dtype], f"rms_norm {rows}x{hidden} {dtype}")
    if dtype != torch.float32:  # 16-bit outputs: differences only where fp32 noise crosses a rounding boundary
        exact = (got == ref).float().mean().item()
        assert exact > 0.99, f"only {exact:.4f} of elements bit-identical to the oracle"


def test_rms_norm_strided_and_inplace(gpu):
    base = _randn((16, 3 * 512), torch.bfloat16, 3).to(gpu)
    x = base[:, 512:1024]  # row stride 1536
    w = _randn((512,), torch.bfloat16, 4, 0.02, 1.0).to(gpu)
    ref = oe.rms_norm(x.cpu(), w.cpu(), 1e-5)
    out = torch.empty(16, 512, dtype=torch.bfloat16, device=gpu)
    ops.rms_norm(out, x, w, 1e-5)
    assert_close(out.cpu().float(), ref.float(), 2e-2, 1e-2, "strided rms_norm")
    y = x.clone()
    ops.rms_norm(y, y, w, 1e-5)  # out aliases input
    assert_close(y.cpu().float(), ref.float(), 2e-2, 1e-2, "in-place rms_norm")
    xw = _randn((6, 2 * 4096), torch.bfloat16, 10).to(gpu)[:, 4096:]  # 4096 wide, strided, in place
    ww = _randn((4096,), torch.bfloat16, 11, 0.02, 1.0).to(gpu)
    refw = oe.rms_norm(xw.cpu(), ww.cpu(), 1e-6)
    ops.rms_norm(xw, xw, ww, 1e-6)
    assert_close(xw.cpu().float(), refw.float(), 2e-2, 1e-2, "in-place strided rms_norm (4096 wide)")
    x3 = _randn((2, 8, 256), torch.float16, 5).to(gpu)  # leading dims flattened
    o3 = torch.empty_like(x3)
    w3 = torch.ones(256, dtype=torch.float16, device=gpu)
    ops.rms_norm(o3, x3, w3, 1e-6)
    assert_close(o3.cpu().float(), oe.rms_norm(x3.cpu(), w3.cpu(), 1e-6).float(), 1e-2, 5e-3, "3d rms_norm")


def test_rms_norm_golden(gpu):
    g = load_golden("rms_norm_bf16")
    x = torch.from_numpy(g["x"]).bfloat16().to(gpu)
    w = torch.from_numpy(g["w"]).bfloat16().to(gpu)
    out = torch.empty_like(x)
    ops.rms_norm(out, x, w, 1e-6)
    assert_close(out.cpu().float(), torch.from_numpy(g["out"]), 2e-2, 1e-2, "rms_norm golden")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fused_add_rms_norm(gpu, dtype):
    x = _randn((33, 4096), dtype, 6)
    r = _randn((33, 4096), dtype, 7)
    w = _randn((4096,), dtype, 8, 0.02, 1.0)
    ref_out, ref_res = oe.fused_add_rms_norm(x, r, w, 1e-6)
    xg, rg = x.to(gpu), r.to(gpu)
    ops.fused_add_rms_norm(xg, rg, w.to(gpu), 1e-6)
    assert torch.equal(rg.cpu(), ref_res), "residual = T(input + residual) must be exact"
    assert_close(xg.cpu().float(), ref_out.float(), *TOL[dtype], "fused_add_rms_norm")


@pytest.mark.parametrize("rows,d,dtype", [
    (64, 11008, torch.float16),   # config 5 pre-step
    (4096, 11008, torch.bfloat16),
    (5, 1001, torch.bfloat16),    # scalar path
    (3, 96, torch.float32),
])
def test_silu_and_mul(gpu, rows, d, dtype):
    x = _randn((rows, 2 * d), dtype, 9, 3.0)
    ref = oe.silu_and_mul(x)
    out = torch.empty(rows, d, dtype=dtype, device=gpu)
    ops.silu_and_mul(out, x.to(gpu))
    got = out.cpu()
    assert_close(got.float(), ref.float(), *TOL[dtype], f"silu_and_mul {rows}x{d} {dtype}")
    if dtype != torch.float32:
        exact = (got == ref).float().mean().item()
        assert exact > 0.99, f"only {exact:.4f} of elements bit-identical to the oracle"


@pytest.mark.parametrize("nrows,hidden,arows,d,dtype", [
    (64, 4096, 64, 11008, torch.float16),    # config 5 pre-step: one launch
    (3, 65536, 7, 96, torch.bfloat16),       # widest norm row (8 chunks per thread)
    (5, 1001, 4, 300, torch.float16),        # odd norm width: the two kernels one after the other
    (2, 512, 3, 1001, torch.bfloat16),       # odd SiLU width: the same
    (9, 1000, 6, 64, torch.float32),
    (0, 4096, 5, 128, torch.bfloat16),       # nothing to normalise
    (4, 4096, 0, 128, torch.bfloat16),       # nothing to activate
])
def test_rms_norm_silu_and_mul_one_launch(gpu, nrows, hidden, arows, d, dtype):
    # the pre-step's two ops in one launch: bit-identical to the two separate ops, and within tolerance of the oracle
    x = _randn((nrows, hidden), dtype, 21)
    w = _randn((hidden,), dtype, 22, 0.02, 1.0)
    gu = _randn((arows, 2 * d), dtype, 23, 3.0)
    xg, wg, gug = x.to(gpu), w.to(gpu), gu.to(gpu)
    normed, act = torch.empty_like(xg), torch.empty(arows, d, dtype=dtype, device=gpu)
    ops.rms_norm_silu_and_mul(normed, xg, wg, 1e-6, act, gug)
    n2, a2 = torch.empty_like(xg), torch.empty_like(act)
    if nrows:
        ops.rms_norm(n2, xg, wg, 1e-6)
    if arows:
        ops.silu_and_mul(a2, gug)
    assert torch.equal(normed.cpu(), n2.cpu()) and torch.equal(act.cpu(), a2.cpu()), "differs from the two ops"
    if nrows:
        assert_close(normed.cpu().float(), oe.rms_norm(x, w, 1e-6).float(), *TOL[dtype], "rms_norm part")
    if arows:
        assert_close(act.cpu().float(), oe.silu_and_mul(gu).float(), *TOL[dtype], "silu_and_mul part")


def test_silu_and_mul_golden(gpu):
    g = load_golden("silu_and_mul_f16")
    x = torch.from_numpy(g["x"]).half().to(gpu)
    out = torch.empty(x.shape[0], x.shape[1] // 2, dtype=torch.float16, device=gpu)
    ops.silu_and_mul(out, x)
    assert_close(out.cpu().float(), torch.from_numpy(g["out"]), 1e-2, 5e-3, "silu golden")


@pytest.mark.parametrize("tokens,hq,hk,D,dtype,pad", [
    (4096, 32, 32, 128, torch.bfloat16, 0),  # config 2
    (300, 16, 8, 256, torch.bfloat16, 0),
    (77, 8, 2, 64, torch.float16, 0),
    (50, 4, 4, 128, torch.float32, 0),
    (20, 3, 1, 48, torch.float16, 3),        # row stride not a multiple of 8: scalar path
])
def test_rotary(gpu, tokens, hq, hk, D, dtype, pad):
    qkv = _randn((tokens, (hq + 2 * hk) * D + pad), dtype, 10)
    pos = torch.randint(0, 8192, (tokens,), generator=_gen(11), dtype=torch.int32)
    pos[:4] = torch.tensor([0, 1, 4095, 8191], dtype=torch.int32)
    q, k = qkv[:, : hq * D], qkv[:, hq * D: (hq + hk) * D]
    ref_q, ref_k = oe.rotary_embedding_online(pos, q.contiguous(), k.contiguous(), D, 10000.0)
    g = qkv.to(gpu)
    gq, gk = g[:, : hq * D], g[:, hq * D: (hq + hk) * D]  # strided views, rotated in place
    ops.rotary_embedding_online(pos.to(gpu), gq, gk, D, 10000.0)
    # fp32: the angle pos / theta^(2i/D) is itself an fp32 value (pos_encoding.cu:84); at pos ~8191 one ulp is
    # ~5e-4 rad, so two correct fp32 evaluations (different powf) differ by up to ~1e-3 * |x| in the output.
    tol = TOL[dtype] if dtype != torch.float32 else (3e-3, 1e-3)
    assert_close(gq.cpu().float(), ref_q.float(), *tol, "rotary q")
    assert_close(gk.cpu().float(), ref_k.float(), *tol, "rotary k")
    assert torch.equal(g[:, (hq + hk) * D:].cpu(), qkv[:, (hq + hk) * D:]), "v part must be untouched"


def test_rotary_golden(gpu):
    g = load_golden("rotary_d32_f32")
    x = torch.from_numpy(g["x"]).to(gpu)
    ops.rotary_embedding_online(torch.from_numpy(g["pos"]).to(gpu), x, None, 32, 10000.0)
    assert_close(x.cpu(), torch.from_numpy(g["out"]), 2e-3, 1e-3, "rotary golden")


def test_wrapper_errors(gpu):
    x = torch.zeros(4, 64, dtype=torch.float64, device=gpu)
    with pytest.raises(RuntimeError, match="dtype"):
        ops.rms_norm(torch.empty_like(x), x, torch.ones(64, dtype=torch.float64, device=gpu), 1e-6)
    h = torch.zeros(4, 64, dtype=torch.float16, device=gpu)
    with pytest.raises(RuntimeError, match="dtypes differ"):
        ops.rms_norm(torch.empty_like(h), h, torch.ones(64, dtype=torch.float32, device=gpu), 1e-6)
    with pytest.raises(RuntimeError, match="head_dim"):
        ops.rotary_embedding_online(torch.zeros(4, dtype=torch.int32, device=gpu), torch.zeros(4, 100, device=gpu,
                                    dtype=torch.float16), None, 100, 1e4)
    with pytest.raises(RuntimeError, match="contiguous vector"):
        ops.fused_add_rms_norm(h, h.clone(), torch.ones(128, dtype=torch.float16, device=gpu)[::2], 1e-6)
    with pytest.raises(RuntimeError, match="must be positive"):
        ops.rotary_embedding_online(torch.zeros(4, dtype=torch.int32, device=gpu), h, None, 0, 1e4)


@pytest.mark.parametrize("tokens,hq,hk,hs,rot,dtype,neox,pad", [
    (4096, 32, 32, 128, 128, torch.bfloat16, True, 0),    # config-2 sized, NeoX, full rotary
    (300, 8, 2, 128, 128, torch.float16, False, 0),       # GPT-J pairs
    (77, 4, 4, 256, 64, torch.bfloat16, False, 0),        # partial rotary (GPT-J style rot_dim 64 of 256)
    (50, 3, 1, 64, 48, torch.float16, True, 8),           # NeoX partial, padded rows
    (33, 2, 2, 96, 40, torch.float16, True, 0),           # rot_dim/2 not a multiple of 8: scalar path
    (20, 2, 1, 64, 64, torch.float32, False, 4),
])
def test_rotary_cos_sin_cache(gpu, tokens, hq, hk, hs, rot, dtype, neox, pad):
    # csrc/pos_encoding.cu:7-61 (rotary_embedding with a cos/sin cache): bit-identical to the oracle in 16 bits (the
    # products are exact in fp32 and every rounding point is the reference's), fp32 within 1e-6
    g = torch.Generator().manual_seed(tokens + rot)
    max_pos = 5000
    ang = torch.rand(max_pos, rot // 2, generator=g, dtype=torch.float64) * 50.0
    cache = torch.cat([ang.cos(), ang.sin()], dim=1).to(dtype)
    pos = torch.randint(0, max_pos, (tokens,), generator=g, dtype=torch.int32)
    q = _randn((tokens, hq * hs + pad), dtype, 31, 2.0)
    k = _randn((tokens, hk * hs + pad), dtype, 32, 2.0)
    ref_q, ref_k = oe.rotary_embedding(pos, q[:, : hq * hs], k[:, : hk * hs], hs, cache, neox)
    qg, kg = q.to(gpu), k.to(gpu)
    ops.rotary_embedding(pos.to(gpu), qg[:, : hq * hs], kg[:, : hk * hs], hs, cache.to(gpu), neox)
    what = f"rotary cache T{tokens} {hq}/{hk} hs{hs} rot{rot} {dtype} neox={neox}"
    if dtype == torch.float32:
        assert_close(qg[:, : hq * hs].cpu(), ref_q, 1e-6, 1e-6, what + " q")
        assert_close(kg[:, : hk * hs].cpu(), ref_k, 1e-6, 1e-6, what + " k")
    else:
        assert torch.equal(qg[:, : hq * hs].cpu(), ref_q), what + " q"
        assert torch.equal(kg[:, : hk * hs].cpu(), ref_k), what + " k"
    assert torch.equal(qg[:, hq * hs:].cpu(), q[:, hq * hs:]), "row padding must be untouched"


def test_rotary_cos_sin_cache_positions_outside_the_cache(gpu):
    # a position outside [0, max_position) leaves its token unchanged (nothing is read outside the cache); key may be
    # omitted
    cache = torch.cat([torch.full((4, 8), 0.5), torch.full((4, 8), 0.25)], dim=1).half()
    q = _randn((5, 2 * 16), torch.float16, 40)
    pos = torch.tensor([0, 3, 4, -1, 2], dtype=torch.int32)
    qg = q.to(gpu)
    ops.rotary_embedding(pos.to(gpu), qg, None, 16, cache.to(gpu), True)
    got = qg.cpu()
    ok = torch.tensor([0, 1, 4])
    ref, _ = oe.rotary_embedding(pos[ok], q[ok], None, 16, cache, True)
    assert torch.equal(got[ok], ref)
    assert torch.equal(got[2:4], q[2:4])
