"""Worker-side migration methods: the caller boundary of the path.

Mirrors the three RPC methods of BaseWorker that reach KVhelper
(paceserve/worker/base_worker.py:235-281) with the same return shapes:
  - _get_kv_cache(seq)        -> (kv_cache, kv_indices, local_rank), then frees
                                 the sequence's source pages (:236-240);
  - _get_kv_cache_nofree(seq) -> same without the free (preemption swap-out,
                                 :245-247);
  - _insert_kv_cache(seq, kv_obj, device) -> KVStatus, or False when the
    destination cannot hold the sequence (:249-281).
and, over a cross-process KVChannel in place of a KVobj returned through
Ray, _send_kv_cache / _recv_kv_cache with the same free, allocation and
remap rules.

The reference's consistency check of the destination table's length
(:265-266) is kept: an AssertionError with the reference's message.  Three
reference defects are not reproduced: the allocate time is reported as a
positive duration (the reference subtracts the later stamp from the earlier
one, :280); when the last logical block has P-1 empty slots the reference
inserts the same pages twice (:265-277), where one insert leaves the same
bytes; and a failed consistency check returns the sequence's destination
pages before raising, where the reference keeps them allocated.
"""
from __future__ import annotations

import threading
import time
from dataclasses import dataclass
from typing import Dict

from ..core.block_manager import BlockSpaceManager


@dataclass
class KVStatus:
    status: bool
    insertion_time: float
    allocate_time: float


class WorkerSequenceManager:
    """The worker's sequence map plus its clone of the block manager
    (paceserve/core/sequence_manager/worker_sequence_manager.py:13-66)."""

    def __init__(self, block_size: int, num_gpu_blocks: int, max_model_len=None, free_list=None):
        self.seq_map: Dict[str, object] = {}
        self.block_manager = BlockSpaceManager(block_size, num_gpu_blocks, max_model_len,
                                               free_list=free_list)

    def add_seq(self, seq) -> None:
        self.seq_map[seq.seq_id] = seq

    def _free_seq(self, seq_id: str) -> None:
        if seq_id not in self.seq_map:
            raise KeyError(seq_id)
        seq = self.seq_map[seq_id]
        if self.block_manager.is_allocated(seq):
            self.block_manager.free(seq)
        del self.seq_map[seq_id]

    def _get_block_table(self, seq):
        return self.block_manager.get_block_table(seq)


def check_table_length(seq, n_dst: int, block_len: int) -> None:
    """The reference's consistency check after allocation
    (paceserve/worker/base_worker.py:265-266): a sequence that has not been
    preempted and whose last logical block holds one token (P-1 empty slots)
    must have received one destination page more than it sent exactly when
    its prompt fills whole pages (the first generated token then opened a
    page).  Sequences without the reference's attributes are not checked."""
    blocks = getattr(seq, "logical_token_blocks", None)
    state = getattr(seq, "state", None)
    if not blocks or state is None or not hasattr(seq, "prompt_token_ids"):
        return
    P = seq.block_size
    if blocks[-1].get_num_empty_slots() == P - 1 and getattr(state, "_preemption_count", 0) == 0:
        want = block_len + (len(seq.prompt_token_ids) % P == 0)
        assert n_dst == want, f"kv len: {n_dst} block: {block_len} seq: {seq}"


class KVWorkerMixin:
    """Provides the worker's KV methods; the host class supplies
    `kvhelper` (a KVhelper), `seq_manager` and `local_rank`."""

    _lock_guard = threading.Lock()

    def _alloc_lock(self, bm):
        """The lock under which inserting threads check for room and allocate
        as one step (the reference runs several insertion threads per
        instance, paceserve/disutil/decode_instance.py:50): the block
        manager's own, or one per worker for a manager without one."""
        lock = getattr(bm, "alloc_lock", None)
        if lock is not None:
            return lock
        with KVWorkerMixin._lock_guard:
            lock = self.__dict__.get("_worker_alloc_lock")
            if lock is None:
                lock = self._worker_alloc_lock = threading.Lock()
        return lock

    def _allocate_dst(self, seq, block_len: int):
        """Checks for room, allocates the sequence's destination table and
        applies the reference's length check; returns the table, or None when
        the destination cannot hold the sequence."""
        bm = self.seq_manager.block_manager
        with self._alloc_lock(bm):
            if bm.get_num_free_gpu_blocks() < bm.get_num_initial_blocks(seq):
                return None
            self.seq_manager.add_seq(seq)
            bm.allocate(seq)
        kv_indices = self.seq_manager._get_block_table(seq)
        try:
            check_table_length(seq, len(kv_indices), block_len)
        except AssertionError:
            self.seq_manager._free_seq(seq.seq_id)
            raise
        return kv_indices

    def _get_kv_cache(self, seq):
        kv_cache, kv_indices = self.kvhelper.get_kv_cache(seq, self.seq_manager)
        self.seq_manager._free_seq(seq.seq_id)
        return (kv_cache, kv_indices, self.local_rank)

    def _get_kv_cache_nofree(self, seq):
        kv_cache, kv_indices = self.kvhelper.get_kv_cache(seq, self.seq_manager)
        return (kv_cache, kv_indices, self.local_rank)

    def _insert_kv_cache(self, seq, kv_obj, device):
        block_len = len(kv_obj.kv_indices)
        cached_content = kv_obj.kv_cache
        allocate_start = time.monotonic()
        kv_indices = self._allocate_dst(seq, block_len)
        if kv_indices is None:
            return False
        insert_start = time.monotonic()
        # A destination table one page longer than the source (the first
        # generated token opened a page) leaves that last page untouched.
        ids = kv_indices if len(kv_indices) == block_len else kv_indices[:-1]
        status = self.kvhelper.insert_kv_cache(cached_content, ids, device)
        insert_time = time.monotonic() - insert_start
        return KVStatus(status, insert_time, insert_start - allocate_start)

    # ------------------------------------------------ cross-process channel

    def _send_kv_cache(self, seq, channel, left_prefill=None, kv_transfer_start=None):
        """_get_kv_cache through a KVChannel: the pages go into the channel,
        the sequence's source pages are freed, and (KVref, local_rank) is
        returned for the control plane in place of the KVobj's tensor."""
        ref = self.kvhelper.send_kv_cache(seq, self.seq_manager, channel, left_prefill, kv_transfer_start)
        self.seq_manager._free_seq(seq.seq_id)
        return (ref, self.local_rank)

    def _recv_kv_cache(self, seq, channel, device, timeout: float = 60.0):
        """_insert_kv_cache of the next channel message, which must carry
        `seq`: allocates the destination pages, receives the pages into them
        and returns KVStatus; False (with the message drained) when the
        destination cannot hold the sequence or the message is another
        sequence's."""
        from .channel import KVref

        with channel.message(timeout) as h:
            ref = KVref.from_header(h)
            if ref.seq_id != seq.seq_id:
                return False
            return self._insert_from_channel(seq, ref, channel, device, timeout)

    def _recv_next_kv_cache(self, lookup, channel, device, timeout: float = 60.0):
        """The next channel message, whichever sequence it carries, as the
        reference's insertion threads insert whichever transfer finishes
        first (paceserve/disutil/decode_instance.py:158-172): lookup(seq_id)
        returns the sequence (None drains the message).  Several threads may
        call this on one channel.  Returns (seq or seq_id, KVStatus or
        False)."""
        from .channel import KVref

        with channel.message(timeout) as h:
            ref = KVref.from_header(h)
            seq = lookup(ref.seq_id)
            if seq is None:
                return ref.seq_id, False
            return seq, self._insert_from_channel(seq, ref, channel, device, timeout)

    def _insert_from_channel(self, seq, ref, channel, device, timeout: float):
        """The allocation, remap and insert of _insert_kv_cache for a message
        whose header was just received; returns KVStatus, or False (the
        payload is then drained by the caller's message())."""
        block_len = len(ref.kv_indices)
        allocate_start = time.monotonic()
        kv_indices = self._allocate_dst(seq, block_len)
        if kv_indices is None:
            return False
        insert_start = time.monotonic()
        ids = kv_indices if len(kv_indices) == block_len else kv_indices[:-1]
        status = self.kvhelper.recv_kv_cache(channel, ids, device, timeout)
        insert_time = time.monotonic() - insert_start
        return KVStatus(status, insert_time, insert_start - allocate_start)


class KVWorker(KVWorkerMixin):
    """A standalone worker holding one KVhelper and its sequence manager."""

    def __init__(self, kvhelper, seq_manager: WorkerSequenceManager, local_rank: int = 0):
        self.kvhelper = kvhelper
        self.seq_manager = seq_manager
        self.local_rank = local_rank
