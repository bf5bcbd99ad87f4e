"""pace_kv_pack_to_host_noalloc, the allocation-free pack into host memory,
called through the C ABI and compared with pace_kv_pack_to_host (a stager's
pipeline) and with torch's gather: the same host bytes on two calls in a row,
the first with layers larger than the scratch (runs of pages), the second
smaller (several layers per chunk), so that the second call's output cannot
pass on bytes left in the scratch by the first."""
import numpy as np
import pytest
import torch

from paceserve_amd import _native, workloads
from paceserve_amd.kv_transfer import ops

pytestmark = pytest.mark.gpu

SHAPE = workloads.KVShape(num_layers=6, num_kv_heads=8, head_dim=128, page_size=16, dtype=torch.bfloat16)
POOL = 2048
SENTINEL = 0xA5


def noalloc(pool, ids, host):
    lib = _native.load()
    stream = torch.cuda.current_stream(pool.device).cuda_stream
    _native.check(lib.pace_kv_pack_to_host_noalloc(
        pool.table(), pool.num_layers, pool.num_pages, ids.data_ptr(), ids.numel(), pool.page_bytes,
        host.data_ptr(), None, stream))


def staged(pool, ids, host):
    n = ids.numel()
    layer_bytes = n * pool.page_bytes
    with ops.Stager(-(-layer_bytes // 256) * 256, 2, pool.device) as st:
        st.pack_to_host(pool, ids, host.view(pool.dtype).view((pool.num_layers, n) + pool.page_shape), 1)
        torch.cuda.synchronize()


def host_buffer(pool, n):
    return torch.full((pool.num_layers * n * pool.page_bytes,), SENTINEL, dtype=torch.uint8, pin_memory=True)


def test_noalloc_matches_pack_to_host_on_two_calls(gpu):
    pool = ops.PagedPool(workloads.fill_pool(POOL, SHAPE, 31, "normal", gpu))
    rng = np.random.default_rng(31)
    # 1100 pages x 64 KiB = 68.75 MiB per layer: more than the 64 MiB scratch;
    # 300 pages = 18.75 MiB per layer: three layers per chunk
    sizes = [1100, 300]
    assert sizes[0] * pool.page_bytes > _native.NOALLOC_SCRATCH_BYTES > 3 * sizes[1] * pool.page_bytes
    cases = []
    for n in sizes:
        ids = torch.tensor(rng.permutation(POOL)[:n], dtype=torch.int32, device=gpu)
        cases.append((ids, host_buffer(pool, n), host_buffer(pool, n)))
    for ids, got, _ in cases:                  # two calls in a row on one stream
        print(f"noalloc call: {ids.numel()} pages x {pool.num_layers} layers", flush=True)
        noalloc(pool, ids, got)
    torch.cuda.synchronize()
    for ids, _, want in cases:
        staged(pool, ids, want)
    for ids, got, want in cases:
        n = ids.numel()
        assert torch.equal(got, want), f"{n} pages: noalloc differs from pack_to_host"
        gathered = torch.stack([t.index_select(0, ids.long()) for t in pool.layers]).cpu()
        assert torch.equal(got, gathered.view(torch.uint8).reshape(-1)), f"{n} pages: differs from torch gather"


def test_noalloc_refuses_pageable_host_memory(gpu):
    """host_out must be pinned: pageable memory is refused before any copy and
    stays untouched, and a valid call right after works."""
    pool = ops.PagedPool(workloads.fill_pool(64, SHAPE, 32, "normal", gpu))
    ids = torch.tensor([3, 7, 1], dtype=torch.int32, device=gpu)
    need = pool.num_layers * 3 * pool.page_bytes
    lib = _native.load()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    pageable = torch.full((need,), SENTINEL, dtype=torch.uint8)
    rc = lib.pace_kv_pack_to_host_noalloc(pool.table(), pool.num_layers, pool.num_pages, ids.data_ptr(), 3,
                                          pool.page_bytes, pageable.data_ptr(), None, stream)
    torch.cuda.synchronize()
    assert rc == _native.PACE_KV_EINVAL and b"not pinned" in lib.pace_kv_last_error()
    assert bool((pageable == SENTINEL).all())
    good = host_buffer(pool, 3)
    noalloc(pool, ids, good)
    torch.cuda.synchronize()
    gathered = torch.stack([t.index_select(0, ids.long()) for t in pool.layers]).cpu()
    assert torch.equal(good, gathered.view(torch.uint8).reshape(-1))
