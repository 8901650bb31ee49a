"""ctypes binding of libcast_amd.so (the C ABI declared in include/cast_amd.h).

There is no fallback: if the library is missing, every device entry point
raises.  ``torch`` is imported before the library is opened so that the
process maps torch's HIP runtime and the library binds to the same one.
"""
from __future__ import annotations

import contextlib
import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libcast_amd.so")

OK = 0
ERR_HEAD_RATIO = 2
ERR_PACK_TOO_LARGE = 3
ERR_HIP = 10
ERR_SCRATCH_LIMIT = 11
ERR_DEVICE = 12
ERR_ALIAS = 13

FLAG_BAD_PACK = 1
FLAG_BAD_OFFSETS = 2
FLAG_BAD_PARENT = 4
FLAG_TOO_LONG = 8

BF16, FP32, FP64, FP16 = 0, 1, 2, 3

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t

_ATTN_ARGS = [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
              _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, ctypes.c_float, _I32, _P, _SZ, _P, _P]

SIGNATURES = {
    "cast_abi_version": ([], ctypes.c_int),
    "cast_status_string": ([ctypes.c_int], ctypes.c_char_p),
    "cast_tree_bitmask": ([_P, _P, _I32, _I32, _I32, _P, _P, _P], ctypes.c_int),
    "cast_tree_attn_fwd": (_ATTN_ARGS, ctypes.c_int),
    "cast_tree_attn_partial": (_ATTN_ARGS, ctypes.c_int),
    "cast_tree_attn_combine": (_ATTN_ARGS, ctypes.c_int),
    "cast_tree_attn_store_fwd": ([_P] * 11 + [_I32] * 8 + [_I64] * 14 + [_I32, ctypes.c_float, _I32, _P, _SZ, _P, _P],
                                 ctypes.c_int),
    "cast_tree_attn_fwd_noalloc": (_ATTN_ARGS[:28] + _ATTN_ARGS[30:], ctypes.c_int),
    "cast_tree_attn_noalloc_limit": ([], _SZ),
    "cast_tree_attn_workspace_size": ([_I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32], _SZ),
    "cast_tree_attn_default_split": ([_I32, _I32, _I32, _I32, _I32, _I32, _I32], _I32),
    "cast_store_append": ([_P] * 4 + [_I32] + [_P] * 2 + [_I32] + [_P] * 3 + [_I32] * 5 + [_I64] * 10 +
                          [_I32, _P, _P], ctypes.c_int),
    "cast_draft_topk": ([_P, _I64, _I32, _I32, _I32, _I32, _P, _P, _I32, _P, _SZ, _P], ctypes.c_int),
    "cast_draft_topk_workspace_size": ([_I32, _I32, _I32, _I32, _I32], _SZ),
    "cast_build_trees": ([_P, _P, _I32, _I32, _I32, _I32] + [_P] * 8, ctypes.c_int),
    "cast_greedy_accept": ([_P, _I64, _I32, _I32, _P, _P, _P, _I32, _I32, _P, _P, _P, _P, _P, _P], ctypes.c_int),
}

_lib = None


class CastError(RuntimeError):
    """A C-ABI call returned an error status."""

    def __init__(self, status, what):
        self.status = status
        super().__init__(f"{what}: {status_string(status)} (status {status})")


def load():
    """Open the library once; raise if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m cast_amd.build` "
                           "(the HIP path has no CPU fallback)")
    import torch  # noqa: F401  (map torch's libamdhip64 first)
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def status_string(status):
    try:
        return load().cast_status_string(int(status)).decode()
    except Exception:
        return "unknown status"


def check(status, what):
    if status != OK:
        if status == ERR_HEAD_RATIO:
            raise AssertionError(f"{what}: query heads must be a multiple of KV heads")
        raise CastError(status, what)


def stream_of(tensor):
    """The raw HIP stream torch launches on for tensor's device (without
    building a torch Stream object: ~0.1 us against ~2 us; the public call
    where torch lacks the raw one)."""
    import torch
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is None:
        return ctypes.c_void_p(torch.cuda.current_stream(tensor.device).cuda_stream)
    return ctypes.c_void_p(raw(tensor.device.index))


_NO_SWITCH = contextlib.nullcontext()


def on_device(dev):
    """A context that makes dev the current HIP device for the launches inside
    it, switching only when another device is current."""
    import torch
    return _NO_SWITCH if torch.cuda.current_device() == dev.index else torch.cuda.device(dev)


def ptr(tensor):
    return ctypes.c_void_p(tensor.data_ptr()) if tensor is not None else ctypes.c_void_p(0)


def raise_device_flags(flags, what):
    """Turn the device status word into an exception (after a sync)."""
    flags = int(flags)
    if not flags:
        return
    parts = []
    if flags & FLAG_BAD_PACK:
        parts.append("a pack is empty or longer than the mask words allow (128 tokens, 64 with one word)")
    if flags & FLAG_BAD_OFFSETS:
        parts.append("cu_q / cu_kv / prefix_len / pack_len are inconsistent")
    if flags & FLAG_BAD_PARENT:
        parts.append("a parent index is not in [-1, own index)")
    if flags & FLAG_TOO_LONG:
        parts.append("a request's keys exceed the kernel's row addressing (2^24 rows / 2 GiB per source)")
    raise ValueError(f"{what}: " + "; ".join(parts))
