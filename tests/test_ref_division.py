"""The reference-rounding mode divides fp16 / bf16 scores by sqrt(D) (and by the soft-cap) as
`q = RN(x*y); r = x - q*d; q' = RN(q + r*y)` with y = RN(1/d) instead of a true division (ref_quot in
deepgengraph_amd/csrc/attention.hip). The result is always rounded on to the 16-bit input dtype, so the claim
checked here is: for every finite 16-bit x and every divisor used, RN16(q') == RN16(fp32 x / d), which is what
the reference computes (deepgengraph_exp/cases/kernels/attn.py:29, h2o.py:29, gemma2.py:31: an fp32 true
division of the rounded matmul output, rounded back to the input dtype).

The same three-fma sequence is compiled for the host with gcc (glibc's fmaf is correctly rounded) and run over
all 2^16 bit patterns of each dtype, for the divisors of the usual head dims and soft-caps plus 200 log-uniform
divisors in [0.01, 1000]."""
import ctypes
import shutil
import subprocess

import numpy as np
import pytest
import torch

C_SRC = r"""
#include <float.h>
#include <math.h>
void ref_quot_many(const float* x, float* out, long n, float d, float y) {
  for (long i = 0; i < n; ++i) {
    float q = fmaf(x[i], y, 0.0f);
    q = fminf(fmaxf(q, -FLT_MAX), FLT_MAX);
    const float r = fmaf(-q, d, x[i]);
    out[i] = fmaf(r, y, q);
  }
}
"""


@pytest.fixture(scope="module")
def ref_quot(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    d = tmp_path_factory.mktemp("refdiv")
    src, lib = d / "refdiv.c", d / "librefdiv.so"
    src.write_text(C_SRC)
    subprocess.run([gcc, "-O2", "-shared", "-fPIC", "-ffp-contract=off", "-o", str(lib), str(src), "-lm"], check=True)
    so = ctypes.CDLL(str(lib))
    so.ref_quot_many.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long, ctypes.c_float, ctypes.c_float]

    def run(x: np.ndarray, div: np.float32) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(x)
        so.ref_quot_many(x.ctypes.data, out.ctypes.data, x.size, float(div), float(np.float32(1.0) / div))
        return out

    return run


def _all_values(dtype):
    bits = np.arange(1 << 16, dtype=np.uint16)
    if dtype == torch.float16:
        x = bits.view(np.float16).astype(np.float32)
    else:
        x = (bits.astype(np.uint32) << 16).view(np.float32)
    return x[np.isfinite(x)]


def _round(x: np.ndarray, dtype) -> np.ndarray:
    """Rounds to dtype and back to fp32 values (so +0 and -0 compare equal: the +0 addend of the first fma turns
    a -0 score into +0, which changes neither the row maximum nor any exp)."""
    return torch.from_numpy(x).to(dtype).float().numpy()


def _divisors():
    out = [np.float32(1.0 / float(np.float32(1.0 / np.sqrt(D)))) for D in (64, 80, 96, 112, 128, 192, 256)]
    out += [np.float32(c) for c in (30.0, 50.0)]
    rng = np.random.default_rng(7)
    out += [np.float32(10.0 ** e) for e in rng.uniform(-2.0, 3.0, size=200)]
    return out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_markstein_quotient_rounds_like_true_division(ref_quot, dtype):
    x = _all_values(dtype)
    bad = []
    for d in _divisors():
        got = _round(ref_quot(x, d), dtype)
        want = _round((x / d).astype(np.float32), dtype)
        if not np.array_equal(got, want, equal_nan=True):
            i = int(np.flatnonzero(got != want)[0])
            bad.append((float(d), float(x[i])))
    assert not bad, f"rounded quotient differs from the true division for (d, x): {bad[:5]}"


def test_infinite_scores_stay_infinite(ref_quot):
    x = np.array([np.inf, -np.inf, 65504.0, -65504.0], dtype=np.float32)
    got = ref_quot(x, np.float32(11.313708))
    assert got[0] == np.inf and got[1] == -np.inf
    np.testing.assert_array_equal(got[2:], (x[2:] / np.float32(11.313708)).astype(np.float32))


@pytest.fixture(scope="module")
def lib():
    from deepgengraph_amd import _lib

    if not _lib.LIB_PATH.exists():
        from deepgengraph_amd import build

        build.build()
    return _lib.load()


def _multiplier(lib, dtype, d):
    import ctypes

    from deepgengraph_amd import _lib

    y = ctypes.c_float(0.0)
    rc = lib.dgg_ref_multiplier(_lib.dtype_code(dtype), float(d), ctypes.byref(y))
    assert rc in (0, 1), rc
    return rc == 1, np.float32(y.value)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_library_multiplier_rounds_like_true_division(lib, dtype):
    """dgg_ref_multiplier (the host search behind reference-rounding mode 2): whenever it reports a multiplier y,
    RN16(RN32(x * y)) must equal RN16(RN32(x / d)) for every finite 16-bit x, checked here independently with
    numpy's IEEE fp32 arithmetic and torch's rounding."""
    x = _all_values(dtype)
    found = 0
    for d in _divisors():
        ok, y = _multiplier(lib, dtype, d)
        if not ok:
            continue
        found += 1
        with np.errstate(over="ignore"):
            got = _round((x * y).astype(np.float32), dtype)
            want = _round((x / d).astype(np.float32), dtype)
        assert np.array_equal(got, want, equal_nan=True), f"multiplier {y!r} for d={d!r} is not exact"
    assert found >= len(_divisors()) // 2


def test_library_multiplier_needs_the_search(lib):
    """fp16, D = 128: RN(1/sqrt(128)) itself changes 52 of the rounded quotients, the next fp32 value up none;
    the search must return the latter (a plain reciprocal would break reference rounding)."""
    d = np.float32(1.0 / float(np.float32(1.0 / np.sqrt(128.0))))
    x = _all_values(torch.float16)
    y0 = np.float32(1.0) / d
    want = _round((x / d).astype(np.float32), torch.float16)
    assert np.count_nonzero(_round((x * y0).astype(np.float32), torch.float16) != want) == 52
    ok, y = _multiplier(lib, torch.float16, d)
    assert ok and y == np.nextafter(y0, np.float32(1.0))
    ok2, y2 = _multiplier(lib, torch.float16, np.float32(8.0))  # D = 64: the reciprocal is exact
    assert ok2 and y2 == np.float32(0.125)
