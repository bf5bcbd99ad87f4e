"""ctypes binding of libpace_kv.so (declared in include/pace_kv.h).

The library is loaded from the package directory.  torch is imported first so
that the library binds to the HIP runtime torch already loaded (both carry the
soname libamdhip64.so.7), which lets torch's streams and allocations be passed
straight through.  There is no fallback: if the library is missing, every
entry point raises.
"""
from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_int, c_int32, c_int64, c_uint64, c_void_p
from pathlib import Path

import torch  # noqa: F401  (binds the HIP runtime before the library loads)

LIB_PATH = Path(__file__).resolve().parent / "libpace_kv.so"
ABI_VERSION = 2
MAX_LAYERS_PER_LAUNCH = 64
NOALLOC_SCRATCH_BYTES = 64 << 20

PACE_KV_OK = 0
PACE_KV_EINVAL = -1
PACE_KV_ERANGE = -2
PACE_KV_ENOMEM = -3
PACE_KV_ESTATE = -4
PACE_KV_ETIMEDOUT = -5
PACE_KV_ECLOSED = -6

# name -> (restype, argtypes); mirrors include/pace_kv.h.
_VP = c_void_p
_I32P = POINTER(c_int32)
SIGNATURES = {
    "pace_kv_abi_version": (c_int, []),
    "pace_kv_last_error": (c_char_p, []),
    "pace_kv_pack": (c_int, [_VP, c_int, c_int64, _VP, c_int64, c_int64, _VP, c_int64, _VP, _VP]),
    "pace_kv_unpack": (c_int, [_VP, c_int64, _VP, c_int, c_int64, _VP, c_int64, c_int64, _VP, _VP]),
    "pace_kv_move": (c_int, [_VP, c_int64, _VP, _VP, c_int64, _VP, c_int, c_int64, c_int64, _VP, _VP]),
    "pace_kv_swap_out": (c_int, [_VP, c_int64, _VP, _VP, c_int64, _VP, c_int, c_int64, c_int64, _VP, _VP]),
    "pace_kv_swap_in": (c_int, [_VP, c_int64, _VP, _VP, c_int64, _VP, c_int, c_int64, c_int64, _VP, _VP]),
    "pace_kv_stager_create": (c_int, [c_int64, c_int, POINTER(c_void_p)]),
    "pace_kv_stager_destroy": (c_int, [_VP]),
    "pace_kv_pack_to_host": (
        c_int, [_VP, _VP, c_int, c_int64, _VP, c_int64, c_int64, c_int, _VP, _VP, _VP]),
    "pace_kv_unpack_from_host": (
        c_int, [_VP, _VP, _VP, c_int, c_int64, _VP, c_int64, c_int64, c_int, _VP, _VP]),
    "pace_kv_append": (
        c_int, [_VP, _VP, c_int64, c_int64, _VP, _VP, c_int, _VP, c_int64, _VP, c_int64, _VP, c_int,
                c_int64, _VP, _VP]),
    "pace_kv_append_indptr": (
        c_int, [_VP, _VP, c_int64, c_int64, _VP, c_int, _VP, c_int64, _VP, c_int64, _VP, _VP, c_int, c_int64,
                _VP, _VP]),
    "pace_kv_batch_indices_positions": (c_int, [_VP, _VP, c_int, c_int64, _VP, _VP, _VP]),
    "pace_kv_allocator_create": (c_int, [c_int64, _VP, c_int64, POINTER(c_void_p)]),
    "pace_kv_allocator_destroy": (c_int, [_VP]),
    "pace_kv_allocator_num_free": (c_int, [_VP, POINTER(c_int64)]),
    "pace_kv_allocator_allocate": (c_int, [_VP, c_int64, _VP]),
    "pace_kv_allocator_free": (c_int, [_VP, _VP, c_int64]),
    "pace_kv_allocator_snapshot": (c_int, [_VP, _VP, c_int64, POINTER(c_int64)]),
    "pace_kv_plan": (c_int, [_VP, c_int, _VP, _VP, c_int64, _VP, _VP, _VP]),
    "pace_kv_promoter_create": (c_int, [POINTER(c_void_p)]),
    "pace_kv_promoter_destroy": (c_int, [_VP]),
    "pace_kv_promote": (
        c_int,
        [_VP, _VP, _VP, c_int64, _VP, c_int64, c_int, c_int64, c_int, _VP, _VP, _VP, _VP, c_int64,
         c_int, _VP, _VP, _VP]),
    "pace_kv_channel_create": (c_int, [c_char_p, c_int64, c_int, c_int, POINTER(c_void_p)]),
    "pace_kv_channel_create_device": (c_int, [c_char_p, c_int64, c_int, c_int, c_int64, POINTER(c_void_p)]),
    "pace_kv_channel_device_info": (c_int, [_VP, POINTER(c_int64), POINTER(c_int)]),
    "pace_kv_channel_open": (c_int, [c_char_p, c_int, c_int, POINTER(c_void_p)]),
    "pace_kv_channel_close": (c_int, [_VP]),
    "pace_kv_channel_info": (c_int, [_VP, POINTER(c_int64), POINTER(c_int)]),
    "pace_kv_channel_unlink": (c_int, [c_char_p]),
    "pace_kv_channel_send": (
        c_int, [_VP, _VP, c_int, c_int64, _VP, c_int64, c_int64, _VP, c_int64, c_int, POINTER(c_uint64), _VP]),
    "pace_kv_channel_send_host": (
        c_int, [_VP, _VP, c_int, c_int64, c_int64, _VP, c_int64, c_int, POINTER(c_uint64)]),
    "pace_kv_channel_recv_header": (
        c_int, [_VP, _VP, c_int64, POINTER(c_int64), POINTER(c_int), POINTER(c_int64), POINTER(c_int64),
                POINTER(c_uint64), c_int]),
    "pace_kv_channel_recv": (
        c_int, [_VP, _VP, c_int, c_int64, _VP, c_int64, c_int64, _VP, c_int, _VP]),
    "pace_kv_channel_recv_host": (c_int, [_VP, _VP, c_int64, c_int]),
    "pace_kv_pack_to_host_noalloc": (
        c_int, [_VP, c_int, c_int64, _VP, c_int64, c_int64, _VP, c_int64, _VP, _VP]),
    "pace_kv_roundtrip": (
        c_int,
        [_VP, _VP, c_int64, _VP, _VP, c_int64, _VP, c_int, c_int64, c_int64, c_int, _VP, c_int64,
         _VP, _VP]),
}


class PaceKVError(RuntimeError):
    """A libpace_kv entry point returned a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"pace_kv status {status}: {message}")
        self.status = status


_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Returns the loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m paceserve_amd.build` "
                "(or __graft_entry__.build()); there is no non-HIP fallback")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.pace_kv_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {ver}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(status: int) -> None:
    """Raises PaceKVError for a non-zero status, with the library's message."""
    if status != PACE_KV_OK:
        msg = load().pace_kv_last_error()
        raise PaceKVError(status, msg.decode(errors="replace") if msg else "")


def pointer_array(ptrs) -> ctypes.Array:
    """A C array of device pointers (void*[n]) for the layer-table arguments."""
    arr_t = c_void_p * len(ptrs)
    return arr_t(*ptrs)
