"""The library's C++ allocator and batch planner (host code, no GPU) against
the oracle's LIFO restatement and the Python planner."""
import numpy as np
import pytest

from oracle import kv_oracle as orc
from paceserve_amd import _native
from paceserve_amd.core.block_manager import BlockAllocator, BlockSpaceManager, NativeBlockAllocator
from paceserve_amd.core.sequence import Sequence
from paceserve_amd.kv_transfer.migrate import plan_batch


def test_fresh_pool_order_and_exhaustion():
    a = NativeBlockAllocator(16, 5)
    assert a.allocate_many(3) == [4, 3, 2]
    assert a.allocate() == 1
    assert a.get_num_free_blocks() == 1
    with pytest.raises(ValueError, match="Out of memory! No free blocks are available."):
        a.allocate_many(2)
    assert a.get_num_free_blocks() == 1          # all-or-nothing
    assert a.allocate_many(0) == []


def test_random_operations_match_oracle():
    rng = np.random.default_rng(7)
    free = rng.permutation(500).tolist()
    nat = NativeBlockAllocator(16, 500, free)
    ref = orc.BlockAllocator(500, free)
    py = BlockAllocator(16, 500, free)
    held = []
    for _ in range(400):
        if rng.random() < 0.55 and ref.num_free():
            n = int(rng.integers(0, min(40, ref.num_free()) + 1))
            got = nat.allocate_many(n)
            assert got == orc.allocate_table(ref, n) == py.allocate_many(n)
            held.append(got)
        elif held:
            t = held.pop(int(rng.integers(0, len(held))))
            t = t + t[: len(t) // 3]                # a table that repeats pages frees them once
            nat.free_many(t)
            orc.free_table(ref, t)
            py.free_many(t)
        assert nat.free_blocks == ref.free_blocks == py.free_blocks


def test_free_rejects_out_of_range_without_freeing():
    a = NativeBlockAllocator(16, 8)
    a.allocate_many(8)
    with pytest.raises(_native.PaceKVError, match="outside"):
        a.free_many([1, 8])
    assert a.get_num_free_blocks() == 0
    with pytest.raises(_native.PaceKVError):
        NativeBlockAllocator(16, 8, [0, 9])


def test_native_plan_matches_python_plan():
    rng = np.random.default_rng(3)
    tables = [rng.permutation(300)[: int(k)].tolist() for k in rng.integers(0, 30, 12)]
    dst_pages = [len(t) + int(rng.integers(0, 2)) for t in tables]
    free = rng.permutation(400).tolist()
    py_plan = plan_batch(tables, 300, BlockAllocator(16, 400, free), dst_pages)
    nat = NativeBlockAllocator(16, 400, free)
    indptr = np.zeros(len(tables) + 1, dtype=np.int64)
    np.cumsum([len(t) for t in tables], out=indptr[1:])
    flat = np.array(sum(tables, []), dtype=np.int32)
    dt, di = nat.plan(flat, indptr, 300, dst_pages)
    assert di.tolist() == py_plan.dst_ids
    assert dt.tolist() == sum(py_plan.dst_tables, [])


@pytest.mark.parametrize("case", ["n_plus_2", "src_range", "oom", "indptr"])
def test_native_plan_errors_leave_allocator_unchanged(case):
    nat = NativeBlockAllocator(16, 10)
    flat = np.array([0, 1, 2], dtype=np.int32)
    indptr = np.array([0, 3], dtype=np.int64)
    dst_pages = None
    if case == "n_plus_2":
        dst_pages = [5]
    elif case == "src_range":
        flat = np.array([0, 1, 300], dtype=np.int32)
    elif case == "oom":
        nat.allocate_many(8)
    elif case == "indptr":
        indptr = np.array([0, 5], dtype=np.int64)
        flat = np.array([0, 1, 2, 3, -1], dtype=np.int32)
    before = nat.free_blocks
    with pytest.raises((ValueError, _native.PaceKVError)):
        nat.plan(flat, indptr, 100, dst_pages)
    assert nat.free_blocks == before


def test_block_space_manager_native_backend():
    bm = BlockSpaceManager(16, 10, native=True)
    s = Sequence.of_length("a", 40, 16)
    bm.allocate(s)
    assert bm.get_block_table(s) == [9, 8, 7]
    bm.free(s)
    assert bm.get_num_free_gpu_blocks() == 10
    assert bm.gpu_allocator.free_blocks == [0, 1, 2, 3, 4, 5, 6, 9, 8, 7]


def test_concurrent_threads_never_share_a_page():
    # ctypes releases the GIL, so these calls run concurrently in the
    # library; its mutex must hand each page to one holder at a time.
    import threading

    pages, threads, rounds = 257, 8, 1500
    a = NativeBlockAllocator(16, pages)
    owner = np.full(pages, -1, dtype=np.int64)
    errors = []

    def worker(tid):
        rng = np.random.default_rng(tid)
        for _ in range(rounds):
            try:
                got = a.allocate_many(int(rng.integers(1, 9)))
            except ValueError:          # momentarily out of pages: try again
                continue
            for p in got:
                if owner[p] != -1:
                    errors.append((tid, p, int(owner[p])))
                owner[p] = tid
            for p in got:
                owner[p] = -1
            a.free_many(got)

    ts = [threading.Thread(target=worker, args=(t,)) for t in range(threads)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors[:5]
    assert a.get_num_free_blocks() == pages
    assert sorted(a.allocate_many(pages)) == list(range(pages))


def test_last_error_is_per_thread():
    import threading

    lib = _native.load()
    a = NativeBlockAllocator(16, 4)
    msgs = {}
    barrier = threading.Barrier(2)

    def fail_with(tid, bad):
        ids = np.array([bad], dtype=np.int32)
        rc = lib.pace_kv_allocator_free(a.handle, ids.ctypes.data, 1)
        barrier.wait()                 # both threads have failed before either reads
        msgs[tid] = (rc, lib.pace_kv_last_error().decode())

    ts = [threading.Thread(target=fail_with, args=(0, 4)), threading.Thread(target=fail_with, args=(1, -3))]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert msgs[0][0] == msgs[1][0] == _native.PACE_KV_ERANGE
    assert "page id 4 " in msgs[0][1] and "page id -3 " in msgs[1][1]
