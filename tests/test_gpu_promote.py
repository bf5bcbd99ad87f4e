"""Single-call promotion (pace_kv_promote) on the GPU: same destination
tables and bytes as the Python planner + ops path, id slots reused safely
across back-to-back calls, and no page left allocated on failure."""
import numpy as np
import pytest
import torch

from paceserve_amd import workloads
from paceserve_amd.core.block_manager import BlockAllocator, NativeBlockAllocator
from paceserve_amd.kv_transfer import migrate, ops

pytestmark = pytest.mark.gpu

SHAPE = workloads.KVShape(num_layers=6, num_kv_heads=8, head_dim=128, page_size=16, dtype=torch.bfloat16)
POOL = 2048


def pools(dev, seed):
    return (ops.PagedPool(workloads.fill_pool(POOL, SHAPE, seed, "normal", dev)),
            ops.PagedPool(workloads.fill_pool(POOL, SHAPE, seed + 1, "normal", dev)))


def words(t):
    return t.view(torch.int16)


# batches of up to 512 pages carry their ids in the kernel arguments; larger
# ones go through the promoter's pinned id slots
SIZES = {"inline": (7, 1, 30, 12), "uploaded": (300, 1, 250, 90)}


@pytest.mark.parametrize("mode", ["fused", "buffer"])
@pytest.mark.parametrize("size", ["inline", "uploaded"])
def test_native_promote_matches_python_path(gpu, mode, size):
    rng = np.random.default_rng(11)
    tables = [rng.permutation(POOL)[: int(k)].tolist() for k in SIZES[size]]
    dst_pages = [len(t) + (i % 2) for i, t in enumerate(tables)]
    free = rng.permutation(POOL).tolist()
    src, dst_py = pools(gpu, 5)
    _, dst_nat = pools(gpu, 5)
    py = migrate.KVMigrator(src, dst_py, BlockAllocator(16, POOL, free))
    nat = migrate.KVMigrator(src, dst_nat, NativeBlockAllocator(16, POOL, free))
    p1 = py.promote(tables, dst_pages, mode=mode, layers_per_chunk=4)
    p2 = nat.promote(tables, dst_pages, mode=mode, layers_per_chunk=4)
    torch.cuda.synchronize()
    assert p1.dst_tables == p2.dst_tables and p1.dst_ids == p2.dst_ids and p1.indptr == p2.indptr
    assert py.dst_allocator.free_blocks == nat.dst_allocator.free_blocks
    for l in range(SHAPE.num_layers):
        assert torch.equal(words(dst_py.layers[l]), words(dst_nat.layers[l])), f"layer {l}"


@pytest.mark.parametrize("lo,hi", [(1, 20), (513, 700)])
def test_back_to_back_promotions_reuse_id_slots(gpu, lo, hi):
    """Ten promotions of different sizes without synchronising in between:
    each must land its own pages (a slot overwritten early would scatter
    another call's ids)."""
    src, dst = pools(gpu, 9)
    alloc = NativeBlockAllocator(16, POOL)
    mig = migrate.KVMigrator(src, dst, alloc)
    rng = np.random.default_rng(2)
    plans = []
    for i in range(10):
        if alloc.get_num_free_blocks() < hi:
            break
        n = int(rng.integers(lo, hi))
        table = rng.permutation(POOL)[:n].tolist()
        plans.append(mig.promote([table], mode="fused" if i % 2 else "buffer"))
        if i % 3 == 2:                  # return some pages: later calls reuse them
            old = plans.pop(0)
            torch.cuda.synchronize()
            alloc.free_many(old.dst_tables[0])
    torch.cuda.synchronize()
    for plan in plans:
        s = torch.tensor(plan.src_ids, device=gpu)
        d = torch.tensor(plan.dst_ids, device=gpu)
        for l in range(SHAPE.num_layers):
            assert torch.equal(words(src.layers[l]).index_select(0, s), words(dst.layers[l]).index_select(0, d))


def test_native_promote_out_of_pages_leaves_allocator_unchanged(gpu):
    src, dst = pools(gpu, 13)
    alloc = NativeBlockAllocator(16, 8)
    dst8 = ops.PagedPool([t[:8] for t in dst.layers])
    mig = migrate.KVMigrator(src, dst8, alloc)
    before = [words(t).clone() for t in dst8.layers]
    with pytest.raises(ValueError, match="Out of memory"):
        mig.promote([[1, 2, 3, 4, 5], [6, 7, 8, 9]], mode="fused")
    assert alloc.free_blocks == list(range(8))
    torch.cuda.synchronize()
    for l in range(SHAPE.num_layers):
        assert torch.equal(words(dst8.layers[l]), before[l])


@pytest.mark.parametrize("native", [False, True])
def test_failed_copy_returns_the_destination_pages(gpu, native):
    # A pinned-host promotion whose host buffer is smaller than one layer
    # chunk is refused by the round trip after the plan allocated its pages:
    # the pages go back and the free list is exactly as before.
    src, dst = pools(gpu, 17)
    free = np.random.default_rng(5).permutation(POOL).tolist()
    alloc = (NativeBlockAllocator if native else BlockAllocator)(SHAPE.page_size, POOL, free_list=free)
    before = list(alloc.free_blocks)
    mig = migrate.KVMigrator(src, dst, alloc)
    tables = [list(range(0, 40)), list(range(100, 130))]
    tiny = torch.empty(1024, dtype=torch.uint8, pin_memory=True)
    with pytest.raises(Exception):
        mig.promote(tables, mode="pinned", host_buf=tiny)
    torch.cuda.synchronize()
    assert list(alloc.free_blocks) == before


def test_one_migrator_from_threads_on_their_own_streams(gpu):
    # Two threads promote through one migrator (its transfer buffer is
    # shared) on streams of their own, with no host synchronisation between.
    import threading

    src, dst = pools(gpu, 21)
    rng = np.random.default_rng(22)
    perm = rng.permutation(POOL).tolist()
    batches = [[perm[i * 40:(i + 1) * 40]] for i in range(8)]          # disjoint 40-page requests
    # The pools were filled on the default stream, which the workers' streams
    # (torch's pooled streams are non-blocking) do not wait for: without this,
    # a destination fill still running could overwrite the first promotions.
    torch.cuda.synchronize()
    for native in (False, True):
        alloc = (NativeBlockAllocator if native else BlockAllocator)(16, POOL)
        mig = migrate.KVMigrator(src, dst, alloc)
        plans, errors = {}, []

        def worker(t):
            try:
                stream = torch.cuda.Stream(gpu)
                with torch.cuda.stream(stream):
                    for i in range(t, len(batches), 2):
                        plans[i] = mig.promote(batches[i], mode="buffer")
                stream.synchronize()
            except Exception as e:                                     # reported by the main thread
                errors.append((t, repr(e)))

        ts = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
        for t in ts:
            t.start()
        for t in ts:
            t.join()
        torch.cuda.synchronize()
        assert not errors, errors
        for i, plan in plans.items():
            s_ids = torch.tensor(plan.src_ids, device=gpu)
            d_ids = torch.tensor(plan.dst_ids, device=gpu)
            for l in range(SHAPE.num_layers):
                assert torch.equal(words(src.layers[l]).index_select(0, s_ids),
                                   words(dst.layers[l]).index_select(0, d_ids)), f"native={native} batch {i}"
        for plan in plans.values():
            for t in plan.dst_tables:
                alloc.free_many(reversed(t))


def test_native_promote_normalises_negative_ids_and_rejects_out_of_range(gpu):
    """Tables go to the library as they are; an id the library refuses
    (negative, or past the pool) sends the call through torch's indexing
    rules: a negative id counts from the end, an id outside [-N, N) raises
    IndexError with no page allocated."""
    src, dst_a = pools(gpu, 21)
    _, dst_b = pools(gpu, 21)
    table = [5, -1, 700, -2048, 3]
    a = migrate.KVMigrator(src, dst_a, NativeBlockAllocator(16, POOL))
    b = migrate.KVMigrator(src, dst_b, NativeBlockAllocator(16, POOL))
    pa = a.promote([table], mode="buffer")
    pb = b.promote([[t % POOL for t in table]], mode="buffer")
    torch.cuda.synchronize()
    assert pa.src_ids == [5, POOL - 1, 700, 0, 3] and pa.dst_tables == pb.dst_tables
    for l in range(SHAPE.num_layers):
        assert torch.equal(words(dst_a.layers[l]), words(dst_b.layers[l])), f"layer {l}"
    free_before = a.dst_allocator.free_blocks
    for bad in ([1, POOL], [-POOL - 1], [2**40]):
        with pytest.raises(IndexError, match="out of bounds for dimension 0 with size 2048"):
            a.promote([bad], mode="buffer")
        assert a.dst_allocator.free_blocks == free_before


@pytest.mark.parametrize("seed", range(6))
def test_random_promotions_match_torch(gpu, seed):
    """Seeded random batches promoted back to back through one migrator on the
    native allocator: 1-6 requests of 1-200 pages (inline ids up to 512
    pages, uploaded ids above), n or n+1 destination pages per request, the
    buffer, fused or pinned mode, 1 to all layers per chunk.  Each promotion
    must pop the destination tables a Python LIFO allocator with the same
    free list pops, and leave the destination pool equal to torch's scatter
    of torch's gather into the pages those tables name (every other page
    unchanged); the source pool stays unchanged."""
    rng = np.random.default_rng(8000 + seed)
    src, dst = pools(gpu, 40 + seed)
    free = rng.permutation(POOL).tolist()
    alloc = NativeBlockAllocator(16, POOL, free)
    mirror = BlockAllocator(16, POOL, free)               # the expected LIFO order
    mig = migrate.KVMigrator(src, dst, alloc)
    host = torch.empty(SHAPE.num_layers * POOL * src.page_bytes, dtype=torch.uint8, pin_memory=True)
    src_before = [words(t).clone() for t in src.layers]
    for call in range(3):
        R = int(rng.integers(1, 7))
        sizes = rng.integers(1, 201, R)
        if call == 2:                           # a batch above 512 pages: ids uploaded, not inline
            R, sizes = 6, rng.integers(100, 201, 6)
        tables = [rng.permutation(POOL)[: int(k)].tolist() for k in sizes]
        dst_pages = [len(t) + int(rng.integers(0, 2)) for t in tables]
        mode = ["buffer", "fused", "pinned"][int(rng.integers(0, 3))]
        if call == 2:
            mode = ["buffer", "fused"][seed % 2]
        k = int(rng.integers(1, SHAPE.num_layers + 1))
        print(f"random promote seed {seed} call {call}: {R} requests, {sum(sizes)} pages, {mode}, "
              f"{k} layers per chunk", flush=True)
        expect_plan = migrate.plan_batch(tables, POOL, mirror, dst_pages)
        dst_before = [words(t).clone() for t in dst.layers]
        plan = mig.promote(tables, dst_pages, mode=mode, layers_per_chunk=k,
                           host_buf=host if mode == "pinned" else None)
        torch.cuda.synchronize()
        assert plan.dst_tables == expect_plan.dst_tables and plan.dst_ids == expect_plan.dst_ids
        si = torch.tensor(expect_plan.src_ids, dtype=torch.long, device=gpu)
        di = torch.tensor(expect_plan.dst_ids, dtype=torch.long, device=gpu)
        for l in range(SHAPE.num_layers):
            want = dst_before[l].index_copy_(0, di, words(src.layers[l]).index_select(0, si))
            assert torch.equal(words(dst.layers[l]), want), f"call {call} layer {l}"
            assert torch.equal(words(src.layers[l]), src_before[l]), f"call {call} source layer {l}"
        # the requests finish: their pages go back to both allocators alike
        done = [p for t in plan.dst_tables for p in t]
        alloc.free_many(reversed(done))
        mirror.free_many(reversed(done))
    assert alloc.free_blocks == mirror.free_blocks
