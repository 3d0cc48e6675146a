"""Rounding points of the reference's scores (deepgengraph_exp/cases/kernels/attn.py:29, h2o.py:29,
gemma2.py:29-33): `torch.matmul(q, k^T) / math.sqrt(D)` in the input dtype, i.e. the matmul result rounded to the
dtype, then divided by a Python float and rounded again; Gemma-2 then divides by the soft-cap (rounded), takes
tanh (rounded) and multiplies by the soft-cap (rounded).

torch evaluates `tensor / python_float` on the GPU as one fp32 multiply by the fp32 reciprocal of the fp32
divisor; on the CPU it divides. The reference runs on the GPU, so the oracle (oracle.attention.div_scalar) and the
kernels' reference-rounding mode follow the GPU form. The CPU tests pin the oracle against an explicit numpy
emulation of every rounding step; the GPU tests pin the emulation against torch's own GPU division and the kernels
against the oracle on inputs whose scores land exactly on the values where the two forms of division differ."""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oa

DIVISORS = [math.sqrt(64), math.sqrt(128), math.sqrt(256), 50.0, 30.0, 20.0, 5.0]


def _all_values(dtype):
    """Every finite value of the 16-bit dtype, as float32."""
    bits = np.arange(1 << 16, dtype=np.uint16)
    if dtype == torch.float16:
        x = bits.view(np.float16).astype(np.float32)
    else:
        x = (bits.astype(np.uint32) << 16).view(np.float32)
    return x[np.isfinite(x)]


def _round16(x32: np.ndarray, dtype) -> np.ndarray:
    """Round-to-nearest-even of fp32 values to the 16-bit dtype, returned as float32. fp16 through numpy's
    IEEE conversion; bf16 by the integer definition (add 0x7fff + lsb, truncate)."""
    x32 = np.ascontiguousarray(x32, dtype=np.float32)
    if dtype == torch.float16:
        with np.errstate(over="ignore"):
            return x32.astype(np.float16).astype(np.float32)
    u = x32.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def _emulate_div(x16: np.ndarray, d: float, dtype) -> np.ndarray:
    """RN16(RN32(x * RN32(1 / RN32(d)))) in numpy fp32 arithmetic."""
    inv = np.float32(1.0) / np.float32(d)
    with np.errstate(over="ignore"):
        return _round16(np.float32(x16) * inv, dtype)


def _true_div(x16: np.ndarray, d: float, dtype) -> np.ndarray:
    with np.errstate(over="ignore"):
        return _round16(np.float32(x16) / np.float32(d), dtype)


def _same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_div_scalar_is_the_reciprocal_multiply(dtype):
    """oracle.attention.div_scalar on every finite 16-bit x equals the numpy emulation bit for bit."""
    x = _all_values(dtype)
    xt = torch.from_numpy(x).to(dtype)
    for d in DIVISORS:
        got = oa.div_scalar(xt, d).float().numpy()
        assert _same_bits(got, _emulate_div(x, d, dtype)), f"d={d}"


def test_reciprocal_multiply_differs_from_true_division():
    """The two forms of `x / sqrt(128)` differ in the last fp16 bit of exactly 52 finite fp16 values (none for the
    power-of-two divisors, none in bf16 for these divisors): a restatement that divided would not match the
    reference on those scores."""
    x = _all_values(torch.float16)
    d = math.sqrt(128)
    diff = _emulate_div(x, d, torch.float16) != _true_div(x, d, torch.float16)
    assert int(diff.sum()) == 52
    for d in (8.0, 16.0):
        assert _same_bits(_emulate_div(x, d, torch.float16), _true_div(x, d, torch.float16))


def _crafted(dtype, n=512, seed=0):
    """q rows [a, b, 0, ...] and one key [1, 1, 0, ...]: the dot product a + b is exact in fp32 but needs more
    bits than the dtype holds, so the rounding of the matmul result is observable. Includes a row for each fp16
    value where the two division forms differ (a = that value, b = 0)."""
    rng = np.random.default_rng(seed)
    D = 128
    # |a| in [1, 8), |b| in [0.01, 0.02): a + b spans at most 2 - (-7 - 10) = 19 bits, exact in fp32
    sign = lambda: np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)  # noqa: E731
    a = _round16(sign() * (1 + 7 * rng.random(n)).astype(np.float32), dtype)
    b = _round16(sign() * (0.01 + 0.01 * rng.random(n)).astype(np.float32), dtype)
    if dtype == torch.float16:
        x = _all_values(torch.float16)
        crit = x[_emulate_div(x, math.sqrt(D), dtype) != _true_div(x, math.sqrt(D), dtype)]
        crit = crit[np.abs(crit) < 60000]
        a = np.concatenate([a, crit])
        b = np.concatenate([b, np.zeros_like(crit)])
    q = np.zeros((1, a.size, 1, D), np.float32)
    q[0, :, 0, 0], q[0, :, 0, 1] = a, b
    k = np.zeros((1, 1, 1, D), np.float32)
    k[0, 0, 0, :2] = 1.0
    dot = (a.astype(np.float64) + b.astype(np.float64)).astype(np.float32)
    assert np.array_equal(dot.astype(np.float64), a.astype(np.float64) + b.astype(np.float64)), "dot must be exact"
    return (torch.from_numpy(q).to(dtype), torch.from_numpy(k).to(dtype), dot)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_oracle_scores_round_twice(dtype):
    """attn.py:29 step by step: with one key and no mask, the row lse is the score itself, so the oracle's lse
    exposes s = RN16(RN32(RN16(q.k) * RN32(1/RN32(sqrt(D))))). A single rounding (no rounding of the matmul
    result) or a true division would each change some of these rows."""
    q, k, dot = _crafted(dtype)
    _, lse = oa.attention(q, k, k, causal=False, return_lse=True)
    want = _emulate_div(_round16(dot, dtype), math.sqrt(128), dtype)
    assert _same_bits(lse[0, 0].numpy(), want)
    single = _emulate_div(dot, math.sqrt(128), dtype)
    assert not _same_bits(single, want), "inputs must make the matmul rounding observable"
    if dtype == torch.float16:
        assert not _same_bits(_true_div(_round16(dot, dtype), math.sqrt(128), dtype), want)


def test_oracle_softcap_rounding_points():
    """gemma2.py:31-33: /= softcap, tanh, *= softcap, each rounded to the dtype (after attn.py:29's two)."""
    dtype = torch.bfloat16
    q, k, dot = _crafted(dtype, seed=1)
    cap = 5.0
    _, lse = oa.attention(q, k, k, causal=False, softcap=cap, return_lse=True)
    s = _emulate_div(_round16(dot, dtype), math.sqrt(128), dtype)
    s = _emulate_div(s, cap, dtype)
    s = _round16(torch.tanh(torch.from_numpy(s)).numpy(), dtype)
    s = _round16(s * np.float32(cap), dtype)
    assert _same_bits(lse[0, 0].numpy(), s)


# ---------------------------------------------------------------------------------------------------------------
# GPU: the claim about torch's GPU division, and the kernels on the crafted rows
# ---------------------------------------------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_torch_gpu_division_is_the_reciprocal_multiply(gpu, dtype):
    """torch on the GPU (the library the reference calls) divides every finite 16-bit x by a Python float exactly
    as div_scalar emulates it."""
    x = _all_values(dtype)
    xg = torch.from_numpy(x).to(dtype).to(gpu)
    for d in DIVISORS:
        got = (xg / d).float().cpu().numpy()
        assert _same_bits(got, _emulate_div(x, d, dtype)), f"d={d}"
        y = xg.clone()
        y /= d  # gemma2.py:31's in-place form
        assert _same_bits(y.float().cpu().numpy(), got)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_kernel_reference_rounding_on_crafted_scores(gpu, dtype):
    """The forward kernel's reference-rounding mode on rows whose scores sit where single rounding or a true
    division would differ: the lse (= the score, one key) must equal the oracle's to fp32 precision."""
    from deepgengraph_amd import attention as A

    q, k, dot = _crafted(dtype)
    _, ref_lse = oa.attention(q, k, k, causal=False, return_lse=True)
    _, lse = A.attention(q.to(gpu), k.to(gpu), k.to(gpu), causal=False, return_lse=True, ref_rounding=True)
    got, want = lse.cpu()[0, 0].double(), ref_lse[0, 0].double()
    err = ((got - want).abs() / want.abs().clamp_min(1e-3)).max().item()
    assert err < 2e-6, f"max relative lse error {err:.3e} (one 16-bit ulp of a score is ~1e-3)"


def _kernel_multiplier(d: float) -> np.float32:
    """The fp32 multiplier the library uses for scale = 1 / d: the divisor is recovered from the fp32 scale as
    RN32(1 / scale) (sqrt(D) itself for the default scale) and its fp32 reciprocal taken."""
    sf = np.float32(1.0 / d)
    div = np.float32(d) if d == math.sqrt(128) else np.float32(1.0 / np.float64(sf))
    return np.float32(1.0) / div


def _double_rounding_divisor() -> float:
    """A divisor whose fp16 multiply RN16(RN32(x * r)) differs from the single rounding RN16(x * r) for some x
    (about one multiplier in a hundred does; none of the 1/sqrt(D) defaults): where a kernel that rounded the
    exact product once (as the fp16 mixed-multiply instructions do) would be wrong."""
    x = _all_values(torch.float16)
    for i in range(2000):
        d = 3.0 + 0.00731 * i
        r = _kernel_multiplier(d)
        twice = _round16(x * r, torch.float16)
        once = (x.astype(np.float64) * np.float64(r)).astype(np.float16).astype(np.float32)
        if not _same_bits(twice, once):
            return d
    raise AssertionError("no such divisor found")


@pytest.mark.gpu
@pytest.mark.parametrize("which", ["default", "double_rounding"])
def test_kernel_fp16_multiply_on_every_value(gpu, which):
    """Every finite fp16 value x as the one score of a row (q = [x, 0, ...], one key [1, 0, ...]): the fp16
    reference-rounding forward at head_dim 128 must give lse = RN16(RN32(x * r)), for the default divisor and for
    a divisor whose multiplier rounds differently when the exact product is rounded once."""
    from deepgengraph_amd import attention as A

    d = math.sqrt(128) if which == "default" else _double_rounding_divisor()
    r = _kernel_multiplier(d)
    x = _all_values(torch.float16)
    want = _round16(x * r, torch.float16).astype(np.float64)
    once = (x.astype(np.float64) * np.float64(r)).astype(np.float16).astype(np.float64)
    D = 128
    q = np.zeros((1, x.size, 1, D), np.float32)
    q[0, :, 0, 0] = x
    k = np.zeros((1, 1, 1, D), np.float32)
    k[0, 0, 0, 0] = 1.0
    qg = torch.from_numpy(q).to(torch.float16).to(gpu)
    kg = torch.from_numpy(k).to(torch.float16).to(gpu)
    _, lse = A.attention(qg, kg, kg, causal=False, return_lse=True, ref_rounding=True,
                         scale=None if which == "default" else 1.0 / d)
    got = lse.cpu()[0, 0].double().numpy()
    rel = np.abs(got - want) / np.maximum(np.abs(want), 1e-3)
    assert rel.max() < 2e-6, f"{which}: max relative lse error {rel.max():.3e} at x = {x[rel.argmax()]}"
    if which == "double_rounding":  # the check can tell the two roundings apart
        assert (np.abs(once - want) / np.maximum(np.abs(want), 1e-3)).max() > 1e-4
