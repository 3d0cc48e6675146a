"""C ABI checks that need no GPU: the library loads, exports every function include/dgg.h declares with the
argument count the ctypes binding uses, and rejects bad arguments with the documented status codes before any
launch (so none of these calls touches a device)."""
import ctypes
import re
from pathlib import Path

import pytest

from deepgengraph_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "dgg.h"

OK, E_DTYPE, E_SHAPE, E_STRIDE, E_ALIGN, E_UNSUP, E_LAUNCH, E_NULL, E_WS = 0, -1, -2, -3, -4, -5, -6, -7, -8


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int|int64_t|const char\*)\s+(dgg_\w+)\s*\(([^)]*)\)\s*;", text):
        args = m.group(2).strip()
        decls[m.group(1)] = 0 if args in ("", "void") else len(args.split(","))
    return decls


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from deepgengraph_amd import build

        build.build()
    return _lib.load()


def test_header_and_binding_agree(lib):
    decls = _declared()
    assert len(decls) >= 11
    assert set(decls) == set(_lib.SIGNATURES), "ctypes SIGNATURES must mirror include/dgg.h"
    for name, nargs in decls.items():
        assert hasattr(lib, name), f"{name} not exported"
        assert len(_lib.SIGNATURES[name][1]) == nargs, f"{name}: binding has a different argument count"


def test_version_and_error_string(lib):
    assert lib.dgg_abi_version() == _lib.ABI_VERSION == 2
    assert isinstance(lib.dgg_last_error(), bytes)


def _strides(vals):
    return _lib.int64_array(vals)


FAKE = ctypes.c_void_p(0x10000)  # 16-byte aligned, never dereferenced: validation fails first
MIS = ctypes.c_void_p(0x10002)


def _prefill(lib, **kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, o=FAKE, lse=None, B=1, Sq=128, Sk=128, Hq=4, Hkv=2, D=128,
             strides=_strides([128 * 512, 512, 128] * 2 + [128 * 256, 256, 128] * 2), scale=0.088, softcap=0.0,
             window=0, flags=1, dtype=_lib.DGG_BF16)
    a.update(kw)
    return lib.dgg_attn_prefill(a["q"], a["k"], a["v"], a["o"], a["lse"], a["B"], a["Sq"], a["Sk"], a["Hq"],
                                a["Hkv"], a["D"], a["strides"], a["scale"], a["softcap"], a["window"], a["flags"],
                                a["dtype"], None)


def test_prefill_validation(lib):
    assert _prefill(lib, dtype=7) == E_DTYPE
    assert b"f32, f16 or bf16" in lib.dgg_last_error()
    assert _prefill(lib, D=96) == E_UNSUP
    assert _prefill(lib, Hq=3) == E_SHAPE
    assert _prefill(lib, B=-1) == E_SHAPE
    assert _prefill(lib, strides=_strides([1] * 12)) == E_STRIDE
    assert _prefill(lib, strides=None) == E_NULL
    assert _prefill(lib, scale=0.0) == E_SHAPE
    assert _prefill(lib, scale=float("nan")) == E_SHAPE
    assert _prefill(lib, softcap=-1.0) == E_SHAPE
    assert _prefill(lib, window=-3) == E_SHAPE
    assert _prefill(lib, q=None) == E_NULL
    assert _prefill(lib, q=MIS) == E_ALIGN
    assert _prefill(lib, o=MIS) == E_ALIGN
    assert _prefill(lib, B=0) == OK  # empty: nothing to launch
    assert _prefill(lib, Sq=0) == OK
    # no keys: the kernels still read q (and write o = 0), so q and o are checked whatever Sk is
    assert _prefill(lib, Sk=0, q=None) == E_NULL
    assert _prefill(lib, Sk=0, q=MIS) == E_ALIGN
    assert _prefill(lib, Sk=0, o=None) == E_NULL
    assert _prefill(lib, Sk=0, k=None, v=None, q=None) == E_NULL


def test_colsum_validation(lib):
    s = _strides([128 * 512, 512, 128] * 2)
    assert lib.dgg_attn_colsum(FAKE, FAKE, None, FAKE, 1, 64, 64, 2, 2, 128, s, 0.1, 0.0, 0, 1, _lib.DGG_F16,
                               None) == E_NULL
    assert lib.dgg_attn_colsum(FAKE, FAKE, FAKE, None, 1, 64, 64, 2, 2, 128, s, 0.1, 0.0, 0, 1, _lib.DGG_F16,
                               None) == E_NULL
    assert lib.dgg_attn_colsum(FAKE, FAKE, FAKE, FAKE, 1, 64, 64, 2, 2, 32, s, 0.1, 0.0, 0, 1, _lib.DGG_F16,
                               None) == E_UNSUP


def test_keyformer_validation(lib):
    s = _strides([128 * 512, 512, 128] * 2)
    er = _strides([32 * 64 * 64, 64 * 64, 64])
    # the KeyFormer passes take 16-bit inputs only (fp32 attention has its own forward and column kernels)
    assert lib.dgg_attn_kf_rowlse(FAKE, FAKE, FAKE, er, FAKE, 1, 64, 64, 2, 2, 128, s, 0.1, 1.5, 0, 1, _lib.DGG_F32,
                                  None) == E_DTYPE
    assert lib.dgg_attn_kf_colsum(FAKE, FAKE, FAKE, er, FAKE, FAKE, 1, 64, 64, 2, 2, 128, s, 0.1, 1.5, 0, 1,
                                  _lib.DGG_F32, None) == E_DTYPE
    assert lib.dgg_attn_kf_rowlse(FAKE, FAKE, FAKE, er, FAKE, 1, 64, 64, 2, 2, 128, s, 0.1, 0.0, 0, 1, _lib.DGG_F16,
                                  None) == E_SHAPE  # tau must be > 0
    assert lib.dgg_attn_kf_rowlse(FAKE, FAKE, None, er, FAKE, 1, 64, 64, 2, 2, 128, s, 0.1, 1.5, 0, 1, _lib.DGG_F16,
                                  None) == E_NULL


def test_decode_validation(lib):
    ws = lib.dgg_attn_decode_workspace_bytes(64, 32, 128, 64)
    assert ws == 64 * 32 * 64 * 130 * 4
    assert lib.dgg_attn_decode_workspace_bytes(-1, 1, 1, 1) == -1
    s = _strides([32 * 128, 128, 32 * 4096 * 128, 4096 * 128, 128, 32 * 4096 * 128, 4096 * 128, 128, 32 * 128, 128])

    def call(**kw):
        a = dict(ws=ws, B=64, Hq=32, Hkv=32, L=4096, D=128, splits=64, dtype=_lib.DGG_F16, scale=0.088, q=FAKE)
        a.update(kw)
        return lib.dgg_attn_decode(a["q"], FAKE, FAKE, FAKE, None, FAKE, a["ws"], a["B"], a["Hq"], a["Hkv"], a["L"],
                                   a["D"], s, a["splits"], a["scale"], a["dtype"], None)

    assert call(ws=ws - 4) == E_WS
    assert call(splits=0) == E_SHAPE
    assert call(splits=2000) == E_SHAPE
    assert call(L=0) == E_SHAPE
    assert call(Hkv=5) == E_SHAPE
    assert call(D=100) == E_UNSUP
    assert call(dtype=_lib.DGG_F32) == E_DTYPE
    assert call(q=MIS) == E_ALIGN
    assert call(B=0, ws=0) == OK


def test_elementwise_validation(lib):
    assert lib.dgg_rms_norm(FAKE, FAKE, FAKE, 4, 0, 0, 0, 1, 1e-6, None) == E_SHAPE
    assert lib.dgg_rms_norm(FAKE, FAKE, FAKE, 4, 64, 32, 64, 1, 1e-6, None) == E_STRIDE
    assert lib.dgg_rms_norm(FAKE, FAKE, FAKE, 4, 64, 64, 64, 9, 1e-6, None) == E_DTYPE
    assert lib.dgg_rms_norm(None, FAKE, FAKE, 4, 64, 64, 64, 1, 1e-6, None) == E_NULL
    assert lib.dgg_rms_norm(None, None, None, 0, 64, 64, 64, 1, 1e-6, None) == OK
    assert lib.dgg_fused_add_rms_norm(FAKE, FAKE, FAKE, 4, 64, 64, 10, 1, 1e-6, None) == E_STRIDE
    assert lib.dgg_silu_and_mul(FAKE, FAKE, 4, 64, 100, 64, 1, None) == E_STRIDE  # input row must hold 2d
    assert lib.dgg_silu_and_mul(FAKE, FAKE, -1, 64, 128, 64, 1, None) == E_SHAPE
    assert lib.dgg_rotary_embedding_online(FAKE, FAKE, FAKE, 8, 4, 4, 100, 400, 400, 1, 1e4, None) == E_UNSUP
    assert lib.dgg_rotary_embedding_online(FAKE, FAKE, FAKE, 8, 4, 4, 128, 100, 512, 1, 1e4, None) == E_STRIDE
    assert lib.dgg_rotary_embedding_online(FAKE, FAKE, FAKE, 8, 4, 4, 128, 512, 512, 5, 1e4, None) == E_DTYPE
    assert lib.dgg_rotary_embedding_online(None, FAKE, FAKE, 8, 4, 4, 128, 512, 512, 1, 1e4, None) == E_NULL


def test_rotary_cache_validation(lib):
    # positions, query, key, tokens, hq, hk, head_size, q_rs, k_rs, cache, rot_dim, max_position, is_neox, dtype
    assert lib.dgg_rotary_embedding(FAKE, FAKE, FAKE, 8, 4, 4, 128, 512, 512, FAKE, 128, 100, 1, 5, None) == E_DTYPE
    assert lib.dgg_rotary_embedding(FAKE, FAKE, FAKE, 8, 4, 4, 128, 512, 512, FAKE, 130, 100, 1, 1, None) == E_SHAPE
    assert lib.dgg_rotary_embedding(FAKE, FAKE, FAKE, 8, 4, 4, 128, 512, 512, FAKE, 63, 100, 0, 1, None) == E_SHAPE
    assert lib.dgg_rotary_embedding(FAKE, FAKE, FAKE, 8, 4, 4, 128, 500, 512, FAKE, 64, 100, 0, 1, None) == E_STRIDE
    assert lib.dgg_rotary_embedding(FAKE, FAKE, FAKE, 8, 4, 4, 128, 512, 512, None, 64, 100, 0, 1, None) == E_NULL
    assert lib.dgg_rotary_embedding(None, None, None, 0, 4, 4, 128, 512, 512, None, 64, 100, 0, 1, None) == OK


def test_topk_validation(lib):
    assert lib.dgg_topk_indices(FAKE, 4, 100, 0, FAKE, None) == E_SHAPE
    assert lib.dgg_topk_indices(FAKE, 4, 100, 101, FAKE, None) == E_SHAPE
    assert lib.dgg_topk_indices(FAKE, 4, 70000, 10, FAKE, None) == E_SHAPE
    assert lib.dgg_topk_indices(None, 4, 100, 10, FAKE, None) == E_NULL
    assert lib.dgg_topk_indices(None, 0, 100, 10, None, None) == OK
    for largest in (0, 1):
        assert lib.dgg_topk_select(FAKE, 4, 100, 0, largest, FAKE, None) == E_SHAPE
        assert lib.dgg_topk_select(FAKE, 4, 0, 1, largest, FAKE, None) == E_SHAPE
        assert lib.dgg_topk_select(FAKE, 4, 65537, 10, largest, FAKE, None) == E_SHAPE
        assert lib.dgg_topk_select(FAKE, 4, 100, 10, largest, None, None) == E_NULL
        assert lib.dgg_topk_select(None, 0, 100, 10, largest, None, None) == OK


def test_roco_select_validation(lib):
    # score, sq_score, rows, n, q_len, recent, budget, out
    assert lib.dgg_roco_select(FAKE, FAKE, 4, 0, 10, 0, 0, FAKE, None) == E_SHAPE
    assert lib.dgg_roco_select(FAKE, FAKE, 4, 70000, 10, 0, 1, FAKE, None) == E_SHAPE
    assert lib.dgg_roco_select(FAKE, FAKE, 4, 100, 0, 10, 10, FAKE, None) == E_SHAPE
    assert lib.dgg_roco_select(FAKE, FAKE, 4, 100, 100, 101, 0, FAKE, None) == E_SHAPE
    assert lib.dgg_roco_select(FAKE, FAKE, 4, 100, 100, -1, 0, FAKE, None) == E_SHAPE
    assert lib.dgg_roco_select(FAKE, FAKE, 4, 100, 100, 30, 71, FAKE, None) == E_SHAPE  # budget > n - recent
    assert lib.dgg_roco_select(FAKE, None, 4, 100, 100, 30, 70, FAKE, None) == E_NULL
    assert lib.dgg_roco_select(None, None, 0, 100, 100, 30, 70, None, None) == OK
    assert lib.dgg_roco_select(None, None, 4, 100, 100, 0, 0, None, None) == OK    # nothing to select


def test_select_workspace_validation(lib):
    # rows of more than 65536 keys: sizes, the workspace and its alignment are checked before any launch; shorter rows
    # go to the one-workgroup kernels and need no workspace
    assert lib.dgg_select_workspace_bytes(4, 65536) == 0
    need = lib.dgg_select_workspace_bytes(4, 1 << 20)
    assert need > 4 * (1 << 20) // 8 * 3
    assert lib.dgg_select_workspace_bytes(-1, 10) == -1
    ws = ctypes.c_void_p(0x100000)
    assert lib.dgg_topk_select_ws(FAKE, 4, 1 << 20, 10, 1, FAKE, ws, need - 1, None) == E_WS
    assert lib.dgg_topk_select_ws(FAKE, 4, 1 << 20, 10, 1, FAKE, None, need, None) == E_NULL
    assert lib.dgg_topk_select_ws(FAKE, 4, 1 << 20, 10, 1, FAKE, ctypes.c_void_p(0x100010), need, None) == E_ALIGN
    assert lib.dgg_topk_select_ws(FAKE, 4, (1 << 26) + 1, 10, 1, FAKE, ws, 1 << 40, None) == E_SHAPE
    assert lib.dgg_topk_select_ws(FAKE, 70000, 1 << 20, 10, 1, FAKE, ws, 1 << 40, None) == E_SHAPE
    assert lib.dgg_topk_select_ws(FAKE, 4, 1 << 20, 0, 1, FAKE, ws, need, None) == E_SHAPE
    assert lib.dgg_topk_select_ws(FAKE, 4, 100, 101, 1, FAKE, None, 0, None) == E_SHAPE  # short rows: as topk_select
    assert lib.dgg_roco_select_ws(FAKE, FAKE, 4, 1 << 20, 10, 30, (1 << 20) - 29, FAKE, ws, need, None) == E_SHAPE
    assert lib.dgg_roco_select_ws(FAKE, FAKE, 4, 1 << 20, 10, 30, 70, FAKE, ws, need - 1, None) == E_WS
    assert lib.dgg_roco_select_ws(None, None, 4, 1 << 20, 10, 0, 0, None, None, 0, None) == OK  # nothing to select


def test_decode_noalloc_validation(lib):
    # every argument is checked before the device's scratch is looked up (no GPU needed for these)
    s = _strides([32 * 128, 128, 32 * 4096 * 128, 4096 * 128, 128] + [32 * 4096 * 128, 4096 * 128, 128] + [32 * 128, 128])

    def call(**kw):
        a = dict(q=FAKE, k=FAKE, v=FAKE, o=FAKE, lse=None, B=2, Hq=32, Hkv=32, L=4096, D=128, strides=s, splits=8,
                 scale=0.088, dtype=_lib.DGG_F16)
        a.update(kw)
        return lib.dgg_attn_decode_noalloc(a["q"], a["k"], a["v"], a["o"], a["lse"], a["B"], a["Hq"], a["Hkv"], a["L"],
                                           a["D"], a["strides"], a["splits"], ctypes.c_float(a["scale"]), a["dtype"],
                                           None)

    assert call(dtype=_lib.DGG_F32) == E_DTYPE
    assert call(D=96) == E_UNSUP
    assert call(splits=0) == E_SHAPE
    assert call(strides=None) == E_NULL
    assert call(B=128, splits=64) == E_WS  # 136 MB of partials > the 96 MiB scratch
    assert b"fixed scratch" in lib.dgg_last_error()
    assert call(q=None) == E_NULL
    assert call(B=0) == OK


def test_fused_rotary_validation(lib):
    assert lib.dgg_rotary_cos_sin(FAKE, FAKE, 16, 100, 1e4, None) == E_UNSUP
    assert lib.dgg_rotary_cos_sin(None, FAKE, 16, 128, 1e4, None) == E_NULL
    assert lib.dgg_rotary_cos_sin(None, None, 0, 128, 1e4, None) == OK
    s = _strides([128 * 512, 512, 128] * 2 + [128 * 256, 256, 128] * 2)

    def call(**kw):
        a = dict(D=128, dtype=_lib.DGG_BF16, cs=FAKE)
        a.update(kw)
        return lib.dgg_attn_prefill_rope(FAKE, FAKE, FAKE, FAKE, None, 1, 128, 128, 4, 2, a["D"], s, 0.088, 0.0, 0, 1,
                                         a["dtype"], a["cs"], None)

    assert call(D=64) == E_UNSUP             # the reference's rotary is head_dim 128 only (pos_encoding.cu:195)
    assert call(dtype=_lib.DGG_F32) == E_UNSUP
    assert call(cs=None) == E_NULL
    assert call(cs=ctypes.c_void_p(0x10010)) == E_ALIGN


def test_clock_probe_validation(lib):
    assert lib.dgg_clock_probe(None, 100, None) == E_NULL
    assert lib.dgg_clock_probe(ctypes.c_void_p(0x10004), 100, None) == E_ALIGN
    assert lib.dgg_clock_probe(FAKE, 0, None) == E_SHAPE
    assert lib.dgg_clock_probe(FAKE, 2_000_000, None) == E_SHAPE


def test_python_wrappers_reject_cpu_tensors():
    import torch

    from deepgengraph_amd import attention, ops

    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        ops.rms_norm(torch.empty_like(x), x, torch.ones(64, dtype=torch.bfloat16), 1e-6)
    q = torch.zeros(1, 8, 2, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        attention.attention(q, q, q)


def test_column_pass_options_follow_the_lse_record():
    # the column passes take ref_rounding / lse_base2 from the record attention() keeps on its lse, refuse a value
    # that contradicts it, and need ref_rounding for an lse without one (host logic only: no launch)
    import torch

    from deepgengraph_amd import attention as A

    lse = torch.zeros(1, 2, 8)
    with pytest.raises(RuntimeError, match="carries no record"):
        A._lse_options("colsum", lse, None, None)
    assert A._lse_options("colsum", lse, True, None) == (True, False)
    assert A._lse_options("colsum", lse, False, True) == (False, True)
    for rr in (False, True):
        for b2 in (False, True):
            tagged = A._tag_lse(torch.zeros(1, 2, 8), rr, b2)
            assert A._lse_options("colsum", tagged, None, None) == (rr, b2)
            assert A._lse_options("colsum", tagged, rr, b2) == (rr, b2)
            with pytest.raises(RuntimeError, match="ref_rounding"):
                A._lse_options("colsum", tagged, not rr, None)
            with pytest.raises(RuntimeError, match="lse_base2"):
                A._lse_options("colsum", tagged, None, not b2)
