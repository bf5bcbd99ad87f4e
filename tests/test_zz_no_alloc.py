"""pace_kv_pack_to_host_noalloc, the allocation-free pack into host memory,
called through the C ABI and compared with pace_kv_pack_to_host (a stager's
pipeline) and with torch's gather: the same host bytes on two calls in a row,
the first with layers larger than the scratch (runs of pages), the second
smaller (several layers per chunk), so that the second call's output cannot
pass on bytes left in the scratch by the first; a host_out one byte short
is refused before anything is written; and the call captured into a HIP
graph, replayed over changed pool contents, writes torch's gather each time
and allocates no device memory."""
import numpy as np
import pytest
import torch

from paceserve_amd import _native, workloads
from paceserve_amd.kv_transfer import ops

pytestmark = pytest.mark.gpu

SHAPE = workloads.KVShape(num_layers=6, num_kv_heads=8, head_dim=128, page_size=16, dtype=torch.bfloat16)
POOL = 2048
SENTINEL = 0xA5


def noalloc(pool, ids, host, host_bytes=None):
    lib = _native.load()
    stream = torch.cuda.current_stream(pool.device).cuda_stream
    nbytes = host.numel() * host.element_size() if host_bytes is None else host_bytes
    _native.check(lib.pace_kv_pack_to_host_noalloc(
        pool.table(), pool.num_layers, pool.num_pages, ids.data_ptr(), ids.numel(), pool.page_bytes,
        host.data_ptr(), nbytes, None, stream))


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
                                          pool.page_bytes, pageable.data_ptr(), need, None, stream)
    torch.cuda.synchronize()
    assert rc == _native.PACE_KV_EINVAL and b"not pinned" in lib.pace_kv_last_error()
    assert bool((pageable == SENTINEL).all())
    good = host_buffer(pool, 3)
    noalloc(pool, ids, good)
    torch.cuda.synchronize()
    gathered = torch.stack([t.index_select(0, ids.long()) for t in pool.layers]).cpu()
    assert torch.equal(good, gathered.view(torch.uint8).reshape(-1))


def gather(pool, ids):
    return torch.stack([t.index_select(0, ids.long()) for t in pool.layers]).cpu().view(torch.uint8).reshape(-1)


def test_noalloc_refuses_a_short_output(gpu):
    """A host_out one byte shorter than the payload is refused with
    PACE_KV_ERANGE before anything is enqueued, although the pinned
    allocation behind it is large enough (a short view of a larger block);
    the buffer stays untouched and the same call with the full size works."""
    pool = ops.PagedPool(workloads.fill_pool(64, SHAPE, 36, "normal", gpu))
    ids = torch.tensor([5, 60, 2, 33], dtype=torch.int32, device=gpu)
    need = pool.num_layers * 4 * pool.page_bytes
    host = torch.full((need + 4096,), SENTINEL, dtype=torch.uint8, pin_memory=True)
    lib = _native.load()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    rc = lib.pace_kv_pack_to_host_noalloc(pool.table(), pool.num_layers, pool.num_pages, ids.data_ptr(), 4,
                                          pool.page_bytes, host.data_ptr(), need - 1, None, stream)
    torch.cuda.synchronize()
    assert rc == _native.PACE_KV_ERANGE, lib.pace_kv_last_error()
    assert f"needs {need} bytes, host_out holds {need - 1}".encode() in lib.pace_kv_last_error()
    assert bool((host == SENTINEL).all())
    noalloc(pool, ids, host, need)
    torch.cuda.synchronize()
    assert torch.equal(host[:need], gather(pool, ids))
    assert bool((host[need:] == SENTINEL).all())


def test_noalloc_replays_from_a_hip_graph(gpu):
    """One call captured with torch.cuda.graph after a warm-up call outside
    capture (which looks up the scratch address), then replayed three times
    over pool contents rewritten in place between the replays (two different
    seeds, then the first again), with eager work and synchronisations in
    between: every replay's host bytes equal torch's gather of the contents
    at that time.  Repeated calls, eager and replayed, leave the device's
    free memory unchanged."""
    pool_pages, n = 512, 200
    pool = ops.PagedPool(workloads.fill_pool(pool_pages, SHAPE, 37, "normal", gpu))
    rng = np.random.default_rng(37)
    ids = torch.tensor(rng.permutation(pool_pages)[:n], dtype=torch.int32, device=gpu)
    host = host_buffer(pool, n)
    noalloc(pool, ids, host)                       # warm-up, outside capture
    torch.cuda.synchronize()
    assert torch.equal(host, gather(pool, ids))
    graph = torch.cuda.CUDAGraph()
    print("noalloc: capturing one call", flush=True)
    with torch.cuda.graph(graph):
        noalloc(pool, ids, host)
    torch.cuda.synchronize()
    for seed in (38, 39, 38):
        fresh = workloads.fill_pool(pool_pages, SHAPE, seed, "normal", gpu)
        for dst, src in zip(pool.layers, fresh):
            dst.copy_(src)
        del fresh
        host.fill_(SENTINEL)
        torch.cuda.synchronize()
        print(f"noalloc: replay over seed {seed}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(host, gather(pool, ids)), f"replay over seed {seed}"
    free_before = torch.cuda.mem_get_info(gpu)[0]
    for _ in range(3):
        noalloc(pool, ids, host)
        graph.replay()
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(gpu)[0] == free_before
    assert torch.equal(host, gather(pool, ids))
