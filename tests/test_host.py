"""Host-side logic of the path (no GPU): allocator, sequences, planning,
worker boundary and KVhelper conventions, checked against the oracle."""
import numpy as np
import pytest

from oracle import kv_oracle as orc
from paceserve_amd.core.block_manager import BlockAllocator, BlockSpaceManager, remap_dst_table
from paceserve_amd.core.kv_cache_obj import KVobj
from paceserve_amd.core.sequence import Sequence
from paceserve_amd.kv_transfer.kv_utils import (chunk_layers, dedup_keep_last, normalize_page_ids,
                                                grown_slot_bytes, roundtrip_chunk_layers)
from paceserve_amd.kv_transfer.migrate import flatten_tables, plan_batch
from paceserve_amd.kv_transfer.worker import KVStatus, KVWorker, WorkerSequenceManager


def test_allocator_matches_oracle_sequence_of_operations():
    rng = np.random.default_rng(0)
    free = rng.permutation(64).tolist()
    prod = BlockAllocator(16, 64, free)
    ref = orc.BlockAllocator(64, free)
    for step in range(200):
        if rng.random() < 0.6 and ref.num_free():
            n = int(rng.integers(0, ref.num_free() + 1))
            assert prod.allocate_many(n) == orc.allocate_table(ref, n)
        else:
            k = int(rng.integers(0, 5))
            pages = rng.integers(0, 64, k).tolist()
            prod.free_many(pages)          # repeats within one call free a page once
            orc.free_table(ref, pages)
        assert prod.free_blocks == ref.free_blocks


def test_allocate_many_is_all_or_nothing():
    a = BlockAllocator(16, 3)
    with pytest.raises(ValueError, match="Out of memory"):
        a.allocate_many(4)
    assert a.get_num_free_blocks() == 3
    assert a.allocate_many(3) == [2, 1, 0]


def test_sequence_logical_blocks():
    for n in [1, 15, 16, 17, 4095, 4096]:
        s = Sequence.of_length("s", n, 16)
        assert len(s.logical_token_blocks) == orc.pages_for_tokens(n, 16)
        assert s.logical_token_blocks[-1].num_tokens == orc.last_page_len(n, 16)
    s = Sequence.of_length("s", 16, 16)
    s.append_token_id(7)                    # first generated token opens page 2
    assert len(s.logical_token_blocks) == 2
    assert s.logical_token_blocks[-1].get_num_empty_slots() == 15


def test_block_space_manager_allocate_free():
    bm = BlockSpaceManager(16, 10)
    s = Sequence.of_length("a", 40, 16)     # 3 pages
    assert bm.can_allocate(s)
    bm.allocate(s)
    assert bm.get_block_table(s) == [9, 8, 7]
    bm.free(s)
    assert bm.get_num_free_gpu_blocks() == 10
    assert not bm.is_allocated(s)
    bm.free(s)                              # already freed: no-op


def test_remap_matches_oracle():
    for m in range(0, 6):
        for n in range(0, 5):
            assert remap_dst_table(list(range(m)), n) == orc.remap_dst_table(list(range(m)), n)


def test_plan_batch_against_oracle():
    rng = np.random.default_rng(1)
    src_tables = [rng.permutation(100)[:k].tolist() for k in (5, 1, 12)]
    dst_pages = [5, 2, 13]                  # n, n+1, n+1
    alloc = BlockAllocator(16, 40)
    plan = plan_batch(src_tables, 100, alloc, dst_pages)
    ref = orc.BlockAllocator(40)
    ids = []
    for t, m in zip(src_tables, dst_pages):
        table = orc.allocate_table(ref, m)
        ids += orc.remap_dst_table(table, len(t))
    assert plan.dst_ids == ids
    assert plan.src_ids == sum(src_tables, [])
    assert plan.indptr == [0, 5, 6, 18]
    assert [len(t) for t in plan.dst_tables] == dst_pages
    assert alloc.free_blocks == ref.free_blocks


def test_plan_batch_rejects_without_allocating():
    alloc = BlockAllocator(16, 4)
    with pytest.raises(ValueError):
        plan_batch([[0, 1], [2, 3, 4]], 10, alloc)          # needs 5 > 4
    assert alloc.get_num_free_blocks() == 4
    with pytest.raises(ValueError):
        plan_batch([[0, 1]], 10, alloc, [4])                 # n+2
    with pytest.raises(IndexError):
        plan_batch([[10]], 10, alloc)
    assert alloc.get_num_free_blocks() == 4


def test_normalize_and_dedup_follow_torch_semantics():
    assert normalize_page_ids([0, -1, 3], 4) == [0, 3, 3]
    with pytest.raises(IndexError):
        normalize_page_ids([4], 4)
    with pytest.raises(IndexError):
        normalize_page_ids([-5], 4)
    ids = [2, 0, 2, 1, 0]
    keep = dedup_keep_last(ids)
    pos, kept = orc.dedup_keep_last(ids, 4)
    assert keep == pos.tolist() and [ids[p] for p in keep] == kept.tolist()


def test_flatten_tables_matches_per_request_normalization():
    rng = np.random.default_rng(5)
    tables = [rng.integers(-64, 64, int(k)).tolist() for k in rng.integers(0, 20, 9)]
    ids, indptr, counts = flatten_tables(tables, 64)
    assert ids.dtype == np.int32 and indptr.dtype == np.int64
    assert counts == [len(t) for t in tables]
    assert indptr.tolist() == [0] + np.cumsum(counts).tolist()
    for r, t in enumerate(tables):
        assert ids[indptr[r]:indptr[r + 1]].tolist() == normalize_page_ids(t, 64)
    one, ip, _ = flatten_tables([[3, -1]], 8)
    assert one.tolist() == [3, 7] and ip.tolist() == [0, 2]
    empty, ip, _ = flatten_tables([], 8)
    assert empty.size == 0 and ip.tolist() == [0]
    for bad in ([[0, 8]], [[1], [-9]]):
        with pytest.raises(IndexError, match="out of bounds for dimension 0 with size 8"):
            flatten_tables(bad, 8)


def test_chunk_layers():
    MiB = 1 << 20
    assert chunk_layers(32, 64 * MiB) == 1
    assert chunk_layers(32, 16 * MiB) == 4       # 64 MiB chunks
    assert chunk_layers(32, 2 * MiB) == 32       # one 64 MiB chunk
    assert chunk_layers(32, 3 * MiB) == 22       # the fewest layers reaching 64 MiB
    assert chunk_layers(32, 512 * MiB) == 1
    assert chunk_layers(1, 1) == 1 and chunk_layers(5, 0) == 5


def test_grown_slot_bytes_at_least_double_within_the_cap():
    MiB = 1 << 20
    assert grown_slot_bytes(10 * MiB + 3) == 10 * MiB + 256          # first stager: what is needed
    assert grown_slot_bytes(12 * MiB, 10 * MiB) == 20 * MiB          # growing: at least double
    assert grown_slot_bytes(50 * MiB, 10 * MiB) == 50 * MiB          # more than double: what is needed
    assert grown_slot_bytes(1024 * MiB, 900 * MiB) == 1280 * MiB     # doubling capped 256 MiB past the need
    sizes, cur, replaced = [8 * MiB + i * MiB for i in range(200)], 0, 0
    for need in sizes:                                               # a run of growing requests
        if cur < need:
            cur, replaced = grown_slot_bytes(need, cur), replaced + 1
        assert cur >= need and cur % 256 == 0
    assert replaced <= 6


def test_roundtrip_chunk_layers_avoid_many_small_chunks():
    MiB = 1 << 20
    # 32 layers of Llama-3-8B pages: requests of 512 .. 8192 tokens
    got = {tok: roundtrip_chunk_layers(32, tok // 16 * 64 * 1024) for tok in (512, 1024, 2048, 4096, 8192)}
    assert got == {512: 4, 1024: 4, 2048: 4, 4096: 2, 8192: 2}
    assert roundtrip_chunk_layers(32, 128 * MiB) == 1     # large chunks: any count
    assert roundtrip_chunk_layers(32, 1 * MiB) == 8       # four 8 MiB chunks
    assert roundtrip_chunk_layers(32, 3 * MiB) == 4       # 12 MiB: 3 layers would make 11 chunks
    assert roundtrip_chunk_layers(32, MiB // 4) == 32     # 8 MiB in all: one chunk
    assert roundtrip_chunk_layers(80, 16 * MiB) == 5      # 80-layer cache: 16 chunks of 80 MiB
    # chunks evened out: two chunks of 16 layers, not 26 + 6 (or 22 + 10) ...
    assert roundtrip_chunk_layers(32, 5 * 64 * 1024) == 16
    assert roundtrip_chunk_layers(32, 6 * 64 * 1024) == 16
    # ... and three of 11, 11 and 10 layers, not 15 + 15 + 2
    assert roundtrip_chunk_layers(32, 9 * 64 * 1024) == 11
    for layers in (1, 7, 32, 80):
        for kib in (64, 320, 576, 1024, 3072, 8192, 40960, 307200):
            k = roundtrip_chunk_layers(layers, kib * 1024)
            assert 1 <= k <= layers
            # no fewer layers per chunk give the same number of chunks
            assert k == 1 or -(-layers // (k - 1)) > -(-layers // k)


class _FakeHelper:
    """Records insert calls; stands in for the device work."""

    def __init__(self):
        self.calls = []

    def insert_kv_cache(self, content, ids, device):
        self.calls.append(list(ids))
        return content.shape[1] == len(ids) or content.shape[1] == 1

    def get_kv_cache(self, seq, seq_manager):
        return "payload", seq_manager._get_block_table(seq)


class _Content:
    def __init__(self, n):
        self.shape = (2, n)

    def element_size(self):
        return 2

    def numel(self):
        return 2 * self.shape[1]


@pytest.mark.parametrize("prompt,outputs,src_pages,expect_ids", [
    (40, 0, 3, [9, 8, 7]),       # n pages on both sides
    (48, 1, 3, [9, 8, 7]),       # the first generated token opened page n+1: it stays untouched
    (40, 1, 3, [9, 8, 7]),
])
def test_worker_insert_remaps_like_reference(prompt, outputs, src_pages, expect_ids):
    helper = _FakeHelper()
    worker = KVWorker(helper, WorkerSequenceManager(16, 10))
    seq = Sequence.of_length("r", prompt, 16, outputs)
    kv = KVobj("r", _Content(src_pages), list(range(src_pages)))
    st = worker._insert_kv_cache(seq, kv, "cuda:0")
    assert isinstance(st, KVStatus) and st.status
    assert helper.calls == [expect_ids]
    assert st.allocate_time >= 0 and st.insertion_time >= 0


def test_worker_insert_checks_table_length_like_reference():
    """base_worker.py:265-266: a sequence whose last block holds one token and
    whose prompt does not fill whole pages must not get an extra page; the
    check raises the reference's AssertionError, and the pages go back."""
    helper = _FakeHelper()
    worker = KVWorker(helper, WorkerSequenceManager(16, 10))
    seq = Sequence.of_length("r", 49, 16)        # 49 prompt tokens: 4 pages, the last with 15 empty slots
    with pytest.raises(AssertionError, match="kv len: 4 block: 3 seq: "):
        worker._insert_kv_cache(seq, KVobj("r", _Content(3), [0, 1, 2]), 0)
    assert helper.calls == []
    assert worker.seq_manager.block_manager.get_num_free_gpu_blocks() == 10
    assert "r" not in worker.seq_manager.seq_map
    # a preempted sequence is not checked (its table may be a page longer)
    seq.state._preemption_count = 1
    st = worker._insert_kv_cache(seq, KVobj("r", _Content(3), [0, 1, 2]), 0)
    assert st.status and helper.calls == [[6, 7, 8]]      # the returned pages come back LIFO


def test_worker_alloc_lock_is_per_block_manager():
    a = KVWorker(_FakeHelper(), WorkerSequenceManager(16, 10))
    b = KVWorker(_FakeHelper(), WorkerSequenceManager(16, 10))
    la = a._alloc_lock(a.seq_manager.block_manager)
    assert la is a.seq_manager.block_manager.alloc_lock
    assert la is not b._alloc_lock(b.seq_manager.block_manager)

    class Bare:                                 # a manager without a lock of its own
        pass

    assert a._alloc_lock(Bare()) is a._alloc_lock(Bare())
    assert a._alloc_lock(Bare()) is not b._alloc_lock(Bare())


def test_worker_insert_without_room_returns_false():
    worker = KVWorker(_FakeHelper(), WorkerSequenceManager(16, 2))
    seq = Sequence.of_length("r", 40, 16)
    assert worker._insert_kv_cache(seq, KVobj("r", _Content(3), [0, 1, 2]), 0) is False
    assert not worker.seq_manager.block_manager.is_allocated(seq)


def test_worker_get_frees_source_pages():
    sm = WorkerSequenceManager(16, 10)
    worker = KVWorker(_FakeHelper(), sm)
    seq = Sequence.of_length("r", 20, 16)
    sm.add_seq(seq)
    sm.block_manager.allocate(seq)
    payload, ids, rank = worker._get_kv_cache_nofree(seq)
    assert ids == [9, 8] and rank == 0
    assert sm.block_manager.get_num_free_gpu_blocks() == 8
    worker._get_kv_cache(seq)
    assert sm.block_manager.get_num_free_gpu_blocks() == 10
    assert "r" not in sm.seq_map


def test_kvobj_size_in_megabytes():
    import torch
    t = torch.zeros(2, 3, 2, 16, 8, 128, dtype=torch.float16)
    assert KVobj("x", t, [0, 1, 2]).size == t.numel() * 2 / 1e6


def test_page_readers_return_each_reader_of_reused_pages_once():
    from paceserve_amd.kv_transfer.swap import PageReaders

    r = PageReaders()
    r.record([5, 6, 7], "swap_in_A")          # stream S1
    r.record([1, 2], "swap_in_B")             # stream S2, enqueued later
    # a swap-out reusing pages of both swap-ins waits for both, once each
    assert r.take([2, 7, 1, 6, 9]) == ["swap_in_B", "swap_in_A"]
    assert len(r) == 1                        # page 5 still remembers A
    assert r.take([5]) == ["swap_in_A"] and r.take([5]) == []
    # a later reader of a page replaces the earlier one
    r.record([3], "A")
    r.record([3], "C")
    assert r.take([3]) == ["C"]


def test_host_destination_ids_must_be_distinct():
    """Repeated destination ids given as host data are refused before any
    copy (two waves writing one page race); source ids may repeat."""
    import torch

    from paceserve_amd.kv_transfer import ops

    with pytest.raises(ValueError, match="destination page 3 appears more than once"):
        ops.device_ids([5, 3, 1, 3], torch.device("cpu"), distinct=True)
    with pytest.raises(ValueError, match="destination page 7 appears"):
        ops.device_ids(torch.tensor([7, 7]), torch.device("cpu"), distinct=True)
    assert ops.device_ids([], torch.device("cpu"), distinct=True).numel() == 0
