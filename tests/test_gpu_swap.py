"""Swap-out / swap-in between a device pool and a pinned host page pool
(pace_kv_swap_out / pace_kv_swap_in), the host-pointer checks that keep the
kernel off unregistered memory, and SwapSpace for preempted requests."""

import numpy as np
import pytest
import torch

from paceserve_amd import _native, workloads
from paceserve_amd.core.block_manager import NativeBlockAllocator
from paceserve_amd.kv_transfer import ops
from paceserve_amd.kv_transfer.swap import SwapSpace

pytestmark = pytest.mark.gpu

SHAPE = workloads.KVShape(num_layers=5, num_kv_heads=8, head_dim=128, page_size=16, dtype=torch.float16)


def words(t):
    return t.view(torch.int16)


def dev_pool(gpu, pages, seed):
    return ops.PagedPool(workloads.fill_pool(pages, SHAPE, seed, "normal", gpu))


def test_swap_out_and_in_match_torch(gpu):
    dev = dev_pool(gpu, 64, 1)
    host = ops.HostPagePool.like(dev, 40)
    for t in host.layers:
        t.fill_(7.0)
    rng = np.random.default_rng(0)
    d_ids = rng.permutation(64)[:17].tolist()
    h_ids = rng.permutation(40)[:17].tolist()
    ops.swap_out(dev, d_ids, host, h_ids)
    torch.cuda.synchronize()
    untouched = sorted(set(range(40)) - set(h_ids))
    for l in range(SHAPE.num_layers):
        want = dev.layers[l][torch.tensor(d_ids, device=gpu)].cpu()
        assert torch.equal(words(host.layers[l][h_ids]), words(want))
        assert (host.layers[l][untouched] == 7.0).all()
    back = dev_pool(gpu, 64, 2)
    before = [words(t).clone() for t in back.layers]
    d2 = rng.permutation(64)[:17].tolist()
    ops.swap_in(host, h_ids, back, d2)
    torch.cuda.synchronize()
    rest = sorted(set(range(64)) - set(d2))
    for l in range(SHAPE.num_layers):
        assert torch.equal(words(back.layers[l][torch.tensor(d2, device=gpu)]),
                           words(dev.layers[l][torch.tensor(d_ids, device=gpu)]))
        assert torch.equal(words(back.layers[l])[rest], before[l][rest])


def _raw_swap_out(dev, host_ptrs, host_pages, n=2):
    ids = torch.arange(n, dtype=torch.int32, device=dev.device)
    table = _native.pointer_array(host_ptrs)
    return _native.load().pace_kv_swap_out(
        dev.table(), dev.num_pages, ids.data_ptr(), table, host_pages, ids.data_ptr(),
        dev.num_layers, n, dev.page_bytes, None, torch.cuda.current_stream().cuda_stream)


def test_swap_rejects_pageable_and_short_host_memory(gpu):
    dev = dev_pool(gpu, 8, 3)
    pageable = [torch.empty((8,) + SHAPE.page_shape, dtype=SHAPE.dtype) for _ in range(SHAPE.num_layers)]
    rc = _raw_swap_out(dev, [t.data_ptr() for t in pageable], 8)
    assert rc == _native.PACE_KV_EINVAL
    assert "not pinned host" in _native.load().pace_kv_last_error().decode()
    short = [torch.empty((2,) + SHAPE.page_shape, dtype=SHAPE.dtype, pin_memory=True)
             for _ in range(SHAPE.num_layers)]
    rc = _raw_swap_out(dev, [t.data_ptr() for t in short], 8)       # claims 8 pages, holds 2
    assert rc in (_native.PACE_KV_ERANGE, _native.PACE_KV_OK)
    if rc == _native.PACE_KV_OK:
        # the caching host allocator rounded the block up: the range check
        # passed because the allocation really holds 8 pages
        torch.cuda.synchronize()
    other = [t.data_ptr() for t in dev.layers]                     # device memory as "host"
    assert _raw_swap_out(dev, other, 8) == _native.PACE_KV_EINVAL
    with pytest.raises(ValueError):
        ops.PagedPool(pageable, host=True)


def test_swap_pool_inside_a_4gib_allocation(gpu):
    """Layers carved out of one device allocation of exactly 4 GiB, the last
    one ending at the allocation's end: the pointer check must see the whole
    allocation (hipPointerGetAttribute's RANGE_SIZE reads such a size modulo
    2^32, i.e. 0), and must still refuse a pool that runs one page past it."""
    torch.cuda.empty_cache()
    big = torch.empty(1 << 32, dtype=torch.uint8, device=gpu)
    pages, pb = 64, SHAPE.page_bytes
    lb = pages * pb
    offsets = [0, lb, 2 * lb, (1 << 32) - 2 * lb, (1 << 32) - lb]
    g = torch.Generator(device=gpu).manual_seed(11)
    layers = []
    for off in offsets:
        t = big[off:off + lb].view(SHAPE.dtype).view((pages,) + SHAPE.page_shape)
        t.copy_(torch.randn(t.shape, generator=g, device=gpu, dtype=torch.float32))
        layers.append(t)
    dev = ops.PagedPool(layers)
    host = ops.HostPagePool.like(dev, 8)
    d_ids, h_ids = [63, 0, 17, 40], [5, 1, 7, 0]
    ops.swap_out(dev, d_ids, host, h_ids)
    torch.cuda.synchronize()
    for l in range(SHAPE.num_layers):
        want = layers[l][torch.tensor(d_ids, device=gpu)].cpu()
        assert torch.equal(words(host.layers[l][h_ids]), words(want))
    back_ids = [2, 3, 62, 61]
    ops.swap_in(host, h_ids, dev, back_ids)
    torch.cuda.synchronize()
    for l in range(SHAPE.num_layers):
        assert torch.equal(words(layers[l][torch.tensor(back_ids, device=gpu)]),
                           words(layers[l][torch.tensor(d_ids, device=gpu)]))
    ids = torch.arange(2, dtype=torch.int32, device=gpu)
    rc = _native.load().pace_kv_swap_out(
        dev.table(), pages + 1, ids.data_ptr(), host.table(), 8, ids.data_ptr(),
        dev.num_layers, 2, pb, None, torch.cuda.current_stream().cuda_stream)
    assert rc == _native.PACE_KV_ERANGE
    assert "layer 4 allocation holds" in _native.load().pace_kv_last_error().decode()
    del layers, dev, big
    torch.cuda.empty_cache()


def test_swap_space_preemption_round_trip(gpu):
    dev = dev_pool(gpu, 128, 5)
    alloc = NativeBlockAllocator(16, 128)
    space = SwapSpace(dev, 64)
    table = alloc.allocate_many(20)
    saved = [words(t[torch.tensor(table, device=gpu)]).clone() for t in dev.layers]
    host_table = space.swap_out("req-1", table)
    assert len(host_table) == 20 and space.holds("req-1")
    torch.cuda.synchronize()
    alloc.free_many(table)                                  # preempted: device pages reused
    other = alloc.allocate_many(30)
    for t in dev.layers:                                    # someone else overwrites them
        t[torch.tensor(other, device=gpu)] = 0
    new_table = alloc.allocate_many(20)
    space.swap_in("req-1", new_table)
    torch.cuda.synchronize()
    assert not space.holds("req-1") and space.num_free_host_pages() == 64
    for l in range(SHAPE.num_layers):
        assert torch.equal(words(dev.layers[l][torch.tensor(new_table, device=gpu)]), saved[l])
    with pytest.raises(KeyError):
        space.swap_in("req-1", new_table)


def test_swap_space_rejected_swap_in_keeps_the_request(gpu):
    # A swap-in refused before its copy (a bad device id, a short table)
    # leaves the request swapped out with its host pages; a correct call
    # then brings the pages back.
    dev = dev_pool(gpu, 32, 9)
    space = SwapSpace(dev, 16)
    table = [3, 7, 11]
    saved = [words(t[torch.tensor(table, device=gpu)]).clone() for t in dev.layers]
    space.swap_out("req-x", table)
    with pytest.raises(IndexError):
        space.swap_in("req-x", [1, 2, 99])
    with pytest.raises(ValueError):
        space.swap_in("req-x", [1, 2])
    assert space.holds("req-x") and space.num_free_host_pages() == 13
    space.swap_in("req-x", [20, 21, 22])
    torch.cuda.synchronize()
    assert not space.holds("req-x") and space.num_free_host_pages() == 16
    for l in range(SHAPE.num_layers):
        assert torch.equal(words(dev.layers[l][torch.tensor([20, 21, 22], device=gpu)]), saved[l])


def test_swap_space_orders_work_across_streams(gpu):
    # Swap out on one stream and in on another with no host synchronisation:
    # the swap-in waits for the swap-out that wrote its host pages, and a
    # later swap-out reusing those host pages waits for the swap-in.
    dev = dev_pool(gpu, 1280, 9)
    alloc = NativeBlockAllocator(16, 1280)
    space = SwapSpace(dev, 400)
    ids = lambda t: torch.tensor(t, device=gpu)           # noqa: E731
    t1, t2 = alloc.allocate_many(400), alloc.allocate_many(400)
    saved1 = [words(t[ids(t1)]).clone() for t in dev.layers]
    saved2 = [words(t[ids(t2)]).clone() for t in dev.layers]
    new1 = alloc.allocate_many(400)
    torch.cuda.synchronize()
    a, b = torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)
    with torch.cuda.stream(a):
        space.swap_out("r1", t1)
    with torch.cuda.stream(b):
        space.swap_in("r1", new1)
    with torch.cuda.stream(a):
        space.swap_out("r2", t2)           # reuses r1's host pages
    torch.cuda.synchronize()
    for l in range(SHAPE.num_layers):
        assert torch.equal(words(dev.layers[l][ids(new1)]), saved1[l])
    alloc.free_many(new1)
    new2 = alloc.allocate_many(400)
    space.swap_in("r2", new2)
    torch.cuda.synchronize()
    for l in range(SHAPE.num_layers):
        assert torch.equal(words(dev.layers[l][ids(new2)]), saved2[l])


def test_swap_4k_request(gpu):
    w = workloads.get(workloads.PROMOTE)
    dev = ops.PagedPool(w.src_pool(gpu))
    host = ops.HostPagePool.like(dev, 256)
    ids = w.src_tables[0]
    ops.swap_out(dev, ids, host, list(range(256)))
    torch.cuda.synchronize()
    for l in (0, 13, 31):
        assert torch.equal(words(host.layers[l]), words(dev.layers[l][torch.tensor(ids, device=gpu)].cpu()))


def test_swap_space_waits_for_every_swap_in_that_read_reused_pages(gpu):
    # Two requests swap in on two streams, the first held back behind long
    # device copies; a third request then swaps out on a third stream into
    # host pages that both swap-ins read.  Its writes must wait for both
    # readers, not only for the swap-in enqueued last.
    dev = dev_pool(gpu, 1280, 11)
    alloc = NativeBlockAllocator(16, 1280)
    space = SwapSpace(dev, 400)
    ids = lambda t: torch.tensor(t, device=gpu)           # noqa: E731
    t1, t2, t3 = alloc.allocate_many(200), alloc.allocate_many(200), alloc.allocate_many(400)
    saved = {k: [words(t[ids(tab)]).clone() for t in dev.layers] for k, tab in (("r1", t1), ("r2", t2), ("r3", t3))}
    space.swap_out("r1", t1)
    space.swap_out("r2", t2)
    new1, new2 = alloc.allocate_many(200), alloc.allocate_many(200)
    x = torch.empty(4 << 30, dtype=torch.uint8, device=gpu).fill_(1)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    a, b, c = torch.cuda.Stream(gpu), torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)
    with torch.cuda.stream(a):
        for _ in range(8):                 # ~15 ms of copies ahead of r1's swap-in
            y.copy_(x)
        space.swap_in("r1", new1)
    with torch.cuda.stream(b):
        space.swap_in("r2", new2)
    with torch.cuda.stream(c):
        space.swap_out("r3", t3)           # all 400 host pages: r1's and r2's
    torch.cuda.synchronize()
    for l in range(SHAPE.num_layers):
        assert torch.equal(words(dev.layers[l][ids(new1)]), saved["r1"][l]), f"r1 layer {l}"
        assert torch.equal(words(dev.layers[l][ids(new2)]), saved["r2"][l]), f"r2 layer {l}"
    alloc.free_many(new1 + new2)
    new3 = alloc.allocate_many(400)
    space.swap_in("r3", new3)
    torch.cuda.synchronize()
    for l in range(SHAPE.num_layers):
        assert torch.equal(words(dev.layers[l][ids(new3)]), saved["r3"][l]), f"r3 layer {l}"
