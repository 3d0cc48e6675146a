"""ctypes binding of libdgg_hip.so (declarations: include/dgg.h).

The library is loaded lazily on first use. There is no fallback: if the shared library is missing or
fails to load, every op raises RuntimeError naming the path and how to build it.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

# DGG_LIBRARY overrides the in-tree library path (e.g. to compare builds).
LIB_PATH = Path(os.environ.get("DGG_LIBRARY", Path(__file__).resolve().parent / "libdgg_hip.so"))

# The ABI version of include/dgg.h this binding is written against; a library reporting another is refused.
ABI_VERSION = 2

DGG_F32, DGG_F16, DGG_BF16 = 0, 1, 2
ATTN_CAUSAL = 0x1
ATTN_REF_ROUNDING = 0x2
ATTN_LSE_BASE2 = 0x4
COL_SUM, COL_SUM_SQ, COL_ANY_GE = 0, 1, 2

_DTYPE_CODE = {torch.float32: DGG_F32, torch.float16: DGG_F16, torch.bfloat16: DGG_BF16}

_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_u32 = ctypes.c_uint32
_f32 = ctypes.c_float
_vp = ctypes.c_void_p
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); mirrors include/dgg.h exactly.
SIGNATURES = {
    "dgg_abi_version": (_i32, []),
    "dgg_last_error": (ctypes.c_char_p, []),
    "dgg_rms_norm": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _f32, _vp]),
    "dgg_fused_add_rms_norm": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _f32, _vp]),
    "dgg_silu_and_mul": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp]),
    "dgg_rms_norm_silu_and_mul": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _vp, _vp, _i64, _i64, _i64, _i64,
                                         _i32, _vp]),
    "dgg_rotary_embedding_online": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _f32, _vp]),
    "dgg_attn_prefill": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64p, _f32, _f32,
                                _i64, _u32, _i32, _vp]),
    "dgg_attn_prefill_rope": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64p, _f32,
                                     _f32, _i64, _u32, _i32, _vp, _vp]),
    "dgg_rotary_cos_sin": (_i32, [_vp, _vp, _i64, _i64, _f32, _vp]),
    "dgg_rotary_embedding": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _i32, _i32,
                                    _vp]),
    "dgg_attn_colsum": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64p, _f32, _f32, _i64,
                               _u32, _i32, _vp]),
    "dgg_attn_colscore": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _i64p, _f32, _f32, _i64, _u32, _i32, _vp]),
    "dgg_attn_kf_rowlse": (_i32, [_vp, _vp, _vp, _i64p, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64p, _f32, _f32,
                                  _i64, _u32, _i32, _vp]),
    "dgg_attn_kf_colsum": (_i32, [_vp, _vp, _vp, _i64p, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64p, _f32,
                                  _f32, _i64, _u32, _i32, _vp]),
    "dgg_avg_pool1d": (_i32, [_vp, _vp, _i64, _i64, _i64, _vp]),
    "dgg_kv_gather": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64p, _i32, _vp]),
    "dgg_topk_indices": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp]),
    "dgg_topk_select": (_i32, [_vp, _i64, _i64, _i64, _i32, _vp, _vp]),
    "dgg_roco_select": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
    "dgg_select_workspace_bytes": (_i64, [_i64, _i64]),
    "dgg_topk_select_ws": (_i32, [_vp, _i64, _i64, _i64, _i32, _vp, _vp, _i64, _vp]),
    "dgg_roco_select_ws": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp]),
    "dgg_nonzero_workspace_bytes": (_i64, [_i64]),
    "dgg_nonzero": (_i32, [_vp, _i32, _i64p, _vp, _i64, _vp, _vp, _i64, _vp]),
    "dgg_clock_probe": (_i32, [_vp, _i64, _vp]),
    "dgg_attn_decode_noalloc": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64p, _i64, _f32, _i32,
                                       _vp]),
    "dgg_attn_decode_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "dgg_attn_splitkv_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "dgg_attn_splitkv": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64p, _i64,
                                _f32, _f32, _i64, _u32, _i32, _vp]),
    "dgg_attn_decode": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64p, _i64, _f32,
                               _i32, _vp]),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Returns the loaded library (loading it on first call). Raises RuntimeError if it is unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} not found: build it with `python -m deepgengraph_amd.build` "
                "(or __graft_entry__.build()); there is no non-HIP fallback")
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as e:
            raise RuntimeError(f"failed to load {LIB_PATH}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                raise RuntimeError(f"{LIB_PATH} does not export {name}: rebuild it with `python -m deepgengraph_amd.build`")
            fn.restype = res
            fn.argtypes = args
        version = lib.dgg_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} reports ABI version {version}, this binding expects {ABI_VERSION}: rebuild it")
        _lib = lib
        return lib


def call(name: str, *args) -> None:
    """Calls a status-returning entry point; raises RuntimeError with dgg_last_error() on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.dgg_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def dtype_code(t: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[t]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {t} (expected float32, float16 or bfloat16)") from None


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def int64_array(vals) -> ctypes.Array:
    return (ctypes.c_int64 * len(vals))(*[int(v) for v in vals])


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on the same HIP device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"expected a GPU tensor, got one on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev
