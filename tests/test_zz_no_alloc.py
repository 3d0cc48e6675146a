"""dgg_attn_decode_noalloc (the allocation-free decode entry point) against dgg_attn_decode (the same kernels with a
caller workspace), both called through the C ABI: two calls in a row, the second smaller, each bit-identical to the
workspace entry point; a call whose partials exceed the fixed scratch is refused with DGG_ERR_WORKSPACE. Runs last
(its file name sorts after every other test) and passes alone in a fresh process as well."""
import ctypes

import pytest
import torch

from deepgengraph_amd import _lib

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 96 << 20  # the fixed scratch of dgg_attn_decode_noalloc (include/dgg.h)
E_WS = -8


def _inputs(B, H, Hkv, L, D, dtype, seed, dev):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, D, generator=g).to(dtype).to(dev)
    k = torch.randn(B, Hkv, L, D, generator=g).to(dtype).to(dev)
    v = torch.randn(B, Hkv, L, D, generator=g).to(dtype).to(dev)
    return q, k, v


def _strides(q, k, v, o):
    return _lib.int64_array([*q.stride()[:2], *k.stride()[:3], *v.stride()[:3], *o.stride()[:2]])


def _run_both(dev, B, H, Hkv, L, D, dtype, splits, seed):
    lib = _lib.load()
    q, k, v = _inputs(B, H, Hkv, L, D, dtype, seed, dev)
    o_ws, o_na = torch.empty_like(q), torch.full_like(q, float("nan"))
    lse_ws = torch.empty(B, H, dtype=torch.float32, device=dev)
    lse_na = torch.full((B, H), float("nan"), dtype=torch.float32, device=dev)
    need = lib.dgg_attn_decode_workspace_bytes(B, H, D, splits)
    assert 0 < need <= SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    code = _lib.dtype_code(dtype)
    stream = _lib.stream_handle(dev)
    scale = ctypes.c_float(D ** -0.5)
    rc = lib.dgg_attn_decode(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o_ws), _lib.ptr(lse_ws), _lib.ptr(ws),
                             need, B, H, Hkv, L, D, _strides(q, k, v, o_ws), splits, scale, code, stream)
    assert rc == 0, lib.dgg_last_error()
    rc = lib.dgg_attn_decode_noalloc(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o_na), _lib.ptr(lse_na), B, H,
                                     Hkv, L, D, _strides(q, k, v, o_na), splits, scale, code, stream)
    assert rc == 0, lib.dgg_last_error()
    torch.cuda.synchronize()
    what = f"B{B} H{H}/{Hkv} L{L} D{D} {dtype} splits{splits}"
    assert torch.equal(o_na.cpu(), o_ws.cpu()), what + " output differs from dgg_attn_decode"
    assert torch.equal(lse_na.cpu(), lse_ws.cpu()), what + " lse differs from dgg_attn_decode"
    assert torch.isfinite(o_na.float()).all()


def test_scratch_is_taken_only_by_a_no_alloc_call(gpu):
    # the 96 MiB array lives in its own code object, which the runtime loads onto a device when the no-alloc entry
    # point is first used there: the other decode calls do not take it (this test must be the process's first no-alloc
    # call, so it comes first in the file and no other test file calls the entry point)
    lib = _lib.load()
    B, H, L, D = 2, 4, 1000, 128
    q, k, v = _inputs(B, H, H, L, D, torch.float16, 7, gpu)
    o = torch.empty_like(q)
    need = lib.dgg_attn_decode_workspace_bytes(B, H, D, 8)
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    stream = _lib.stream_handle(gpu)
    scale = ctypes.c_float(D ** -0.5)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    rc = lib.dgg_attn_decode(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), None, _lib.ptr(ws), need, B, H, H, L,
                             D, _strides(q, k, v, o), 8, scale, _lib.DGG_F16, stream)
    assert rc == 0, lib.dgg_last_error()
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    rc = lib.dgg_attn_decode_noalloc(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), None, B, H, H, L, D,
                                     _strides(q, k, v, o), 8, scale, _lib.DGG_F16, stream)
    assert rc == 0, lib.dgg_last_error()
    torch.cuda.synchronize()
    free2 = torch.cuda.mem_get_info()[0]
    assert free0 - free1 < SCRATCH_BYTES // 2, f"a workspace decode took {(free0 - free1) >> 20} MiB"
    assert free1 - free2 >= SCRATCH_BYTES, f"the first no-alloc call took only {(free1 - free2) >> 20} MiB"


def test_noalloc_decode_matches_workspace_entry_point(gpu):
    # a large call that fills most of the scratch, then a smaller one that reuses (and must not read) its contents
    _run_both(gpu, 16, 32, 8, 8192, 128, torch.float16, 64, seed=1)   # 17.0 MB of partials
    _run_both(gpu, 2, 8, 8, 1000, 64, torch.bfloat16, 8, seed=2)      # 0.03 MB of partials
    _run_both(gpu, 3, 4, 2, 37, 256, torch.float16, 50, seed=3)       # splits past the end of the cache


def test_noalloc_decode_refuses_oversized_partials(gpu):
    lib = _lib.load()
    B, H, D, splits = 64, 32, 128, 64  # config 5 at 64 splits: 68,157,440 bytes fit
    assert lib.dgg_attn_decode_workspace_bytes(B, H, D, splits) <= SCRATCH_BYTES
    B = 128  # twice the batch: 136 MB of partials
    q = torch.zeros(B, H, D, dtype=torch.float16, device=gpu)
    kv = torch.zeros(B, H, 16, D, dtype=torch.float16, device=gpu)
    o = torch.empty_like(q)
    rc = lib.dgg_attn_decode_noalloc(_lib.ptr(q), _lib.ptr(kv), _lib.ptr(kv), _lib.ptr(o), None, B, H, H, 16, D,
                                     _strides(q, kv, kv, o), splits, ctypes.c_float(0.088), _lib.DGG_F16,
                                     _lib.stream_handle(gpu))
    assert rc == E_WS
    assert b"fixed scratch" in lib.dgg_last_error()
