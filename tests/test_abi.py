"""The C-ABI library: loads, exports every symbol include/pace_kv.h declares,
and rejects bad arguments on the host before any device work (no GPU here)."""
import ctypes
import re
from pathlib import Path

import pytest

from paceserve_amd import _native

HEADER = Path(__file__).resolve().parent.parent / "include" / "pace_kv.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(pace_kv_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _native.LIB_PATH.exists():
        pytest.fail(f"{_native.LIB_PATH} is not built (run python -m paceserve_amd.build)")
    return _native.load()


def test_header_declares_the_bound_functions():
    assert declared_functions() == sorted(_native.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_abi_version(lib):
    assert lib.pace_kv_abi_version() == _native.ABI_VERSION
    text = HEADER.read_text()
    assert f"#define PACE_KV_ABI_VERSION {_native.ABI_VERSION}" in text
    assert f"#define PACE_KV_MAX_LAYERS_PER_LAUNCH {_native.MAX_LAYERS_PER_LAUNCH}" in text


def _layers(n, base=0x10000):
    return _native.pointer_array([base + i * 0x100000 for i in range(n)])


def test_empty_work_is_a_no_op(lib):
    # zero layers or zero pages: success without touching the device
    assert lib.pace_kv_pack(None, 0, 10, None, 5, 65536, None, 0, None, None) == 0
    assert lib.pace_kv_pack(_layers(2), 2, 10, None, 0, 65536, None, 0, None, None) == 0
    assert lib.pace_kv_unpack(None, 0, _layers(2), 2, 10, None, 0, 65536, None, None) == 0
    assert lib.pace_kv_move(None, 10, None, None, 10, None, 0, 3, 65536, None, None) == 0


@pytest.mark.parametrize("call,code,msg", [
    (lambda L: L.pace_kv_pack(_layers(2), -1, 10, 0x100, 4, 65536, 0x1000, 4 * 65536, None, None),
     _native.PACE_KV_EINVAL, "num_layers"),
    (lambda L: L.pace_kv_pack(_layers(2), 2, 10, None, 4, 65536, 0x1000, 4 * 65536, None, None),
     _native.PACE_KV_EINVAL, "NULL"),
    (lambda L: L.pace_kv_pack(_layers(2), 2, 10, 0x100, 4, 65536, 0x1000, 65536, None, None),
     _native.PACE_KV_ERANGE, "out_layer_stride"),
    (lambda L: L.pace_kv_pack(_layers(2), 2, 10, 0x100, 4, 65536, 0x1000, 4 * 65536 + 8, None, None),
     _native.PACE_KV_EINVAL, "stride not a multiple of 16"),
    (lambda L: L.pace_kv_pack(_layers(2), 2, 10, 0x100, 4, 65530, 0x1000, 4 * 65536, None, None),
     _native.PACE_KV_EINVAL, "page_bytes must be a positive multiple of 16"),
    (lambda L: L.pace_kv_pack(_layers(2), 2, 10, 0x100, 4, 100, 0x1000, 4 * 112, None, None),
     _native.PACE_KV_EINVAL, "page_bytes"),
    (lambda L: L.pace_kv_pack(_native.pointer_array([0x10000, 0x10008]), 2, 10, 0x100, 4, 65536,
                              0x1000, 4 * 65536, None, None),
     _native.PACE_KV_EINVAL, "16-byte aligned"),
    (lambda L: L.pace_kv_pack(_native.pointer_array([0x10000, 0]), 2, 10, 0x100, 4, 65536,
                              0x1000, 4 * 65536, None, None),
     _native.PACE_KV_EINVAL, "NULL"),
    (lambda L: L.pace_kv_unpack(0x1000, 65536, _layers(2), 2, 10, 0x100, 4, 65536, None, None),
     _native.PACE_KV_ERANGE, "buf_layer_stride"),
    (lambda L: L.pace_kv_move(_layers(2), 10, 0x100, _layers(2), 10, None, 2, 4, 65536, None, None),
     _native.PACE_KV_EINVAL, "NULL page ids"),
    (lambda L: L.pace_kv_move(_layers(2), 10, 0x102, _layers(2), 10, 0x100, 2, 4, 65536, None, None),
     _native.PACE_KV_EINVAL, "4-byte aligned"),
    (lambda L: L.pace_kv_stager_create(1000, 3, ctypes.byref(ctypes.c_void_p())),
     _native.PACE_KV_EINVAL, "slot_bytes"),
    (lambda L: L.pace_kv_stager_create(1 << 20, 1, ctypes.byref(ctypes.c_void_p())),
     _native.PACE_KV_EINVAL, "num_slots"),
    (lambda L: L.pace_kv_pack_to_host(None, _layers(1), 1, 10, 0x100, 1, 65536, 1, 0x1000, None, None),
     _native.PACE_KV_EINVAL, "stager is NULL"),
])
def test_argument_errors_are_reported_on_the_host(lib, call, code, msg):
    assert call(lib) == code
    assert msg in lib.pace_kv_last_error().decode()


def test_check_raises_with_message(lib):
    rc = lib.pace_kv_pack(_layers(2), -1, 10, 0x100, 4, 65536, 0x1000, 4 * 65536, None, None)
    with pytest.raises(_native.PaceKVError, match="num_layers"):
        _native.check(rc)


@pytest.mark.parametrize("compiler,flags", [("gcc", ["-x", "c", "-std=c99"]), ("g++", ["-x", "c++", "-std=c++11"])])
def test_header_is_self_contained_c_and_cpp(tmp_path, compiler, flags):
    import shutil
    import subprocess

    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} not installed")
    src = tmp_path / "use_header.c"
    src.write_text('#include "pace_kv.h"\nint f(void) { return pace_kv_abi_version() + PACE_KV_OK; }\n')
    r = subprocess.run([compiler, *flags, "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{HEADER.parent}",
                        "-fsyntax-only", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_noalloc_pack_to_host_rejects_pages_beyond_its_scratch(lib):
    """A page larger than the 64 MiB scratch is refused before any device
    call (so this runs without a GPU), with the limit in the message."""
    big = _native.NOALLOC_SCRATCH_BYTES + 16
    rc = lib.pace_kv_pack_to_host_noalloc(_layers(1), 1, 4, 0x100, 1, big, 0x1000, 1 << 40, None, None)
    assert rc == _native.PACE_KV_ERANGE
    assert b"exceeds the 67108864-byte scratch" in lib.pace_kv_last_error()
    assert lib.pace_kv_pack_to_host_noalloc(_layers(1), 1, 4, 0x100, 1, 24, 0x1000, 1 << 40, None, None) == \
        _native.PACE_KV_EINVAL                                      # not a multiple of 16
    assert lib.pace_kv_pack_to_host_noalloc(None, 0, 4, None, 3, 65536, None, 0, None, None) == 0   # no work


def test_noalloc_pack_to_host_rejects_a_short_output(lib):
    """A payload larger than host_out_bytes is refused before any device call
    (so this runs without a GPU): 3 layers x 2 pages x 4 KiB need 24 KiB, one
    byte more than the caller gives."""
    rc = lib.pace_kv_pack_to_host_noalloc(_layers(3), 3, 4, 0x100, 2, 4096, 0x1000, 3 * 2 * 4096 - 1, None, None)
    assert rc == _native.PACE_KV_ERANGE
    assert b"needs 24576 bytes, host_out holds 24575" in lib.pace_kv_last_error()
    text = HEADER.read_text()
    assert "#define PACE_KV_NOALLOC_SCRATCH_BYTES (64 << 20)" in text
