"""ctypes binding of libsimsd_kernels.so (the C ABI declared in include/simsd_kernels.h).

The library is built ahead of time into this directory (see ``build_lib.py``).
There is no fallback: if the library is missing or fails to load, every entry
point that needs it raises, so a GPU run can never silently take another path.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_NAME = "libsimsd_kernels.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 18

DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
SCORE_SOFTMAX = 0
SCORE_SIGMOID = 1
MOE_MAX_EXPERTS = 1024
MOE_MAX_SLOTS = 8192

_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_vp = ctypes.c_void_p
_f32 = ctypes.c_float

# name -> (restype, argtypes); must match include/simsd_kernels.h
SIGNATURES = {
    "simsd_abi_version": (_i32, []),
    "simsd_last_error_string": (ctypes.c_char_p, []),
    "simsd_thin_linear": (_i32, [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64,
                                 _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _vp]),
    "simsd_thin_linear_noalloc": (_i32, [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64,
                                         _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _vp]),
    "simsd_thin_linear_noalloc_max_scratch_bytes": (_i64, []),
    "simsd_thin_linear_silu_mul": (_i32, [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64,
                                          _vp, _i64, _i64, _i64, _i64, _i64, _i32,
                                          _i32, _i32, _i32, _i32, _vp, _i64, _vp]),
    "simsd_thin_linear_residual": (_i32, [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64,
                                          _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _vp]),
    "simsd_rmsnorm": (_i32, [_vp, _i64, _vp, _f32, _vp, _i64, _i64, _i64, _i32, _vp]),
    "simsd_thin_linear_partials": (_i32, [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64,
                                          _i32, _i32, _i32, _i32, _i32, _vp]),
    "simsd_reduce_residual_rmsnorm": (_i32, [_vp, _i32, _i64, _vp, _i64, _vp, _i64, _vp, _f32, _vp, _i64,
                                             _i64, _i64, _i32, _vp]),
    "simsd_rmsnorm_linear_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32, _i32, _i32, _i32]),
    "simsd_rmsnorm_thin_linear": (_i32, [_vp, _i64, _i64, _vp, _f32, _vp, _i64, _i64, _vp, _i64,
                                         _vp, _i64, _i64, _i64, _i64, _i64, _i32,
                                         _i32, _i32, _i32, _i32, _vp, _i64, _vp]),
    "simsd_rmsnorm_thin_linear_silu_mul": (_i32, [_vp, _i64, _i64, _vp, _f32, _vp, _i64, _i64,
                                                  _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64,
                                                  _i64, _i32, _i32, _i32, _i32, _i32, _vp, _i64,
                                                  _vp]),
    "simsd_thin_linear_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32, _i32, _i32, _i32]),
    "simsd_thin_linear_plan": (_i32, [_i64, _i64, _i64, _i32, _i32, _i32, _i32,
                                      ctypes.POINTER(ctypes.c_int)]),
    "simsd_softmax_argmax_workspace_bytes": (_i64, [_i64, _i64]),
    "simsd_softmax_argmax": (_i32, [_vp, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _i64, _vp, _i64, _vp]),
    "simsd_denoise_select": (_i32, [_vp, _i64, _i64, _i64, _i32, _vp, _i64, _i32, _vp, _i64, _vp, _i64,
                                    _vp, _vp, _vp, _i64, _vp]),
    "simsd_qkv_rope_cache": (_i32, [_vp, _i64, _vp, _vp, _f32, _vp, _vp, _i64, _i64, _vp, _vp, _vp,
                                    _vp, _vp, _i64, _i64, _vp, _i64, _i64,
                                    _i64, _i64, _i64, _i64, _i32, _vp]),
    "simsd_reduce_qkv_rope_cache": (_i32, [_vp, _i32, _i64, _vp, _vp, _f32, _vp, _vp, _i64, _i64, _vp, _vp, _vp,
                                           _vp, _vp, _i64, _i64, _vp, _i64, _i64,
                                           _i64, _i64, _i64, _i64, _i32, _vp]),
    "simsd_block_attention_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "simsd_block_attention": (_i32, [_vp, _i64, _i64, _vp, _vp, _i64, _i64,
                                     _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64,
                                     _f32, _i32, _vp, _i64, _vp]),
    "simsd_qkv_rope_attention": (_i32, [_vp, _i64, _vp, _vp, _f32, _vp, _vp, _i64, _i64, _vp,
                                        _vp, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _i64,
                                        _i64, _i64, _i64, _vp, _i64, _f32, _i32, _vp, _i64, _vp]),
    "simsd_block_mask": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _vp, _vp]),
    "simsd_moe_route_topk": (_i32, [_vp, _i64, _i64, _i64, _i32, _i32, _i32, _f32, _vp, _vp, _vp]),
    "simsd_moe_num_tiles": (_i32, [_i64, _i64]),
    "simsd_moe_align": (_i32, [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "simsd_moe_route_align": (_i32, [_vp, _i64, _i64, _i64, _i32, _i32, _i32, _f32, _vp, _vp,
                                      _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "simsd_moe_workspace_bytes": (_i64, [_i64, _i32, _i64, _i64, _i64, _i32]),
    "simsd_moe_grouped_ffn": (_i32, [
        _vp, _i64, _i64,                 # x
        _vp, _i64, _i64, _i64,           # w_gate
        _vp, _i64, _i64, _i64,           # w_up
        _vp, _i64, _i64, _i64,           # w_down
        _vp, _i64, _i64,                 # shared gate
        _vp, _i64, _i64,                 # shared up
        _vp, _i64, _i64, _i64,           # shared down, Is
        _vp, _vp, _i32,                  # slots, tile_expert, num_tiles
        _vp, _i64, _i64,                 # topk ids
        _vp, _i64, _i64,                 # topk weights
        _vp, _i64, _i64,                 # out
        _i64, _i32, _i64, _i64, _i64, _i32,   # T, k, E, H, I, dtype
        _vp, _i64, _vp]),                # workspace, bytes, stream
}

_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_NAME} is not built (expected at {LIB_PATH}); build it with "
                "`python simsd-release_amd/build_lib.py` or __graft_entry__.build()")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        got = handle.simsd_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"{LIB_NAME} ABI version {got}, expected {ABI_VERSION}")
        _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().simsd_last_error_string().decode(errors="replace")
        raise RuntimeError(f"{what} failed: {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one HIP device; returns it."""
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            f"the MI355X kernels need device (HIP) tensors, got a tensor on {dev}")
    for t in tensors[1:]:
        if t is not None and t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


class device_guard:
    """Make `dev` current for the launch (kernels go to the current device,
    not the tensors' device); a no-op when it already is."""

    __slots__ = ("dev", "prev")

    def __init__(self, dev: torch.device):
        self.dev = dev
        self.prev = None

    def __enter__(self):
        idx = self.dev.index if self.dev.index is not None else torch.cuda.current_device()
        cur = torch.cuda.current_device()
        if idx != cur:
            self.prev = cur
            torch.cuda.set_device(idx)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False
