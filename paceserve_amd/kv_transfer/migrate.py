"""Batched promotion: move whole requests from a source pool to a destination
pool on one GPU (the additive batch API over the reference's per-request
get_kv_cache / _insert_kv_cache pair, paceserve/worker/base_worker.py:236-281).

One promote() call:
  1. allocates every request's destination pages from the destination's LIFO
     allocator, request by request, as BaseWorker._insert_kv_cache does
     (base_worker.py:255-262), all-or-nothing for the batch;
  2. remaps positionally, dropping a trailing extra destination page (the n vs
     n+1 rule, base_worker.py:264-277);
  3. uploads both id lists (CSR-concatenated over requests) with one pinned
     host-to-device copy;
  4. moves the pages in one of three modes:
       "buffer": pack into a device transfer buffer, then unpack - the
                 reference's two-step semantics, with the buffer as the
                 device-resident KVobj payload; layer-chunked when the
                 buffer would be large;
       "fused":  pool-to-pool move, no buffer (half the HBM traffic);
       "pinned": the full device->host->device round trip through pinned
                 memory, overlapped per layer chunk (pace_kv_roundtrip).
Each request's slice of the transfer buffer, buf[:, indptr[r]:indptr[r+1]],
is byte-identical to what the reference's get_kv_cache returns for it.
"""
from __future__ import annotations

import itertools
import threading
from array import array
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

from ..core.block_manager import BlockAllocator, NativeBlockAllocator, remap_dst_table
from . import ops
from .kv_utils import normalize_page_ids


@dataclass
class MigrationPlan:
    src_ids: List[int]          # concatenated source pages (CSR over requests)
    dst_ids: List[int]          # concatenated destination pages written
    dst_tables: List[List[int]]  # full destination block tables (incl. any +1 page)
    indptr: List[int]           # request r owns positions [indptr[r], indptr[r+1])

    @property
    def n_pages(self) -> int:
        return len(self.src_ids)


def plan_batch(src_tables: Sequence[Sequence[int]], src_num_pages: int, dst_allocator: BlockAllocator,
               dst_pages: Optional[Sequence[int]] = None) -> MigrationPlan:
    """Allocates destination pages for a batch of requests and remaps them.

    Request r gets dst_pages[r] pages (default len(src_tables[r])) popped from
    dst_allocator in request order; its source pages land positionally in the
    first len(src_tables[r]) of them (an extra trailing page stays untouched).
    Raises ValueError, allocating nothing, if a count is neither n nor n+1 or
    the destination cannot hold the batch; IndexError for a source id outside
    the source pool."""
    if dst_pages is None:
        dst_pages = [len(t) for t in src_tables]
    if len(dst_pages) != len(src_tables):
        raise ValueError("one destination page count per request")
    src_ids: List[int] = []
    indptr = [0]
    for t in src_tables:
        src_ids.extend(normalize_page_ids(t, src_num_pages))
        indptr.append(len(src_ids))
    for r, (t, m) in enumerate(zip(src_tables, dst_pages)):
        if remap_dst_table([0] * m, len(t)) is None:
            raise ValueError(f"request {r}: {m} destination pages cannot receive {len(t)} pages")
    pages = dst_allocator.allocate_many(sum(dst_pages))
    dst_tables: List[List[int]] = []
    dst_ids: List[int] = []
    pos = 0
    for t, m in zip(src_tables, dst_pages):
        table = pages[pos:pos + m]
        pos += m
        dst_tables.append(table)
        dst_ids.extend(remap_dst_table(table, len(t)))
    return MigrationPlan(src_ids, dst_ids, dst_tables, indptr)


def _csr_of_int32_tables(src_tables: Sequence[Sequence[int]]):
    """(ids array('i'), indptr array('q'), counts) of a batch whose ids all
    fit int32, or None (an id that does not, or is not an int).  The ids are
    not range-checked here: the library checks them before it allocates."""
    try:
        if len(src_tables) == 1:
            ids = array("i", src_tables[0])
            counts = [len(ids)]
        else:
            counts = [len(t) for t in src_tables]
            ids = array("i", itertools.chain.from_iterable(src_tables))
    except (OverflowError, TypeError):
        return None
    return ids, array("q", (0, *itertools.accumulate(counts))), counts


def flatten_tables(src_tables: Sequence[Sequence[int]], num_pages: int):
    """CSR form of a batch of source block tables: (ids int32, indptr int64,
    counts).  Ids follow torch advanced-indexing rules, as normalize_page_ids
    does: negative ids count from the end, and an id outside
    [-num_pages, num_pages) raises IndexError."""
    counts = [len(t) for t in src_tables]
    indptr = np.array([0, *itertools.accumulate(counts)], dtype=np.int64)
    total = int(indptr[-1])
    ids = src_tables[0] if len(counts) == 1 else itertools.chain.from_iterable(src_tables)
    flat = np.fromiter(ids, dtype=np.int64, count=total)
    if total:
        lo, hi = int(flat.min()), int(flat.max())
        if lo < -num_pages or hi >= num_pages:
            bad = flat[(flat < -num_pages) | (flat >= num_pages)][0]
            raise IndexError(f"index {bad} is out of bounds for dimension 0 with size {num_pages}")
        if lo < 0:
            flat = np.where(flat < 0, flat + num_pages, flat)
    return flat.astype(np.int32), indptr, counts


class KVMigrator:
    def __init__(self, src, dst, dst_allocator: BlockAllocator, *,
                 buffer_bytes_max: int = 8 << 30, stager: Optional[ops.Stager] = None):
        self.src = ops.as_pool(src)
        self.dst = ops.as_pool(dst)
        if not self.src.compatible(self.dst) or self.src.num_layers != self.dst.num_layers:
            raise ValueError("source and destination pools differ in layout, layers, dtype or device")
        self.dst_allocator = dst_allocator
        self.buffer_bytes_max = int(buffer_bytes_max)
        self.stager = stager
        self._buf: Optional[torch.Tensor] = None
        self._buf_view: Optional[torch.Tensor] = None
        self._elem = self.src.layers[0].element_size()
        self._promoter: Optional[ops.Promoter] = None
        # One migrator may be driven from several threads and streams: the
        # lock covers its host state (buffer, stager, promoter), and a call
        # on a stream other than the last user's first waits for that
        # stream's work, since the transfer buffer is shared.
        self._lock = threading.RLock()
        self._buf_stream: Optional[torch.cuda.Stream] = None
        self._buf_handle: Optional[int] = None

    # ------------------------------------------------------------ planning

    def plan(self, src_tables: Sequence[Sequence[int]],
             dst_pages: Optional[Sequence[int]] = None) -> MigrationPlan:
        """Allocates and remaps destination pages (see plan_batch)."""
        return plan_batch(src_tables, self.src.num_pages, self.dst_allocator, dst_pages)

    def upload(self, plan: MigrationPlan):
        """Both id lists as int32 device tensors, via one pinned copy."""
        n = plan.n_pages
        host = torch.empty(2 * n, dtype=torch.int32, pin_memory=True)
        host[:n] = torch.tensor(plan.src_ids, dtype=torch.int32)
        host[n:] = torch.tensor(plan.dst_ids, dtype=torch.int32)
        dev = host.to(self.src.device, non_blocking=True)
        return dev[:n], dev[n:]

    # ------------------------------------------------------------ movement

    def _order_after_last_user(self) -> int:
        """Orders the current stream after the stream that last used the
        transfer buffer (and lets torch's allocator know the buffer is used
        here), when the two differ; returns the current stream's handle.
        Caller holds the lock."""
        handle = ops._stream_handle(self.src.device)
        if handle != self._buf_handle:
            stream = torch.cuda.current_stream(self.src.device)
            if self._buf_stream is not None:
                stream.wait_stream(self._buf_stream)
                if self._buf is not None:
                    self._buf.record_stream(stream)
            self._buf_stream, self._buf_handle = stream, handle
        return handle

    def _buffer(self, layers: int, n: int) -> torch.Tensor:
        """A [layers, n, *page_shape] view of the migrator's transfer buffer
        (grown on demand; the last view is reused for the same shape).
        Caller holds the lock and has called _order_after_last_user."""
        v = self._buf_view
        if v is not None and v.shape[0] == layers and v.shape[1] == n:
            return v
        need = (layers, n) + self.src.page_shape
        numel = layers * n * self.src.page_bytes // self._elem
        if self._buf is None or self._buf.numel() < numel:
            self._buf_view = None
            self._buf = torch.empty(numel, dtype=self.src.dtype, device=self.src.device)
        self._buf_view = self._buf[:numel].view(need)
        return self._buf_view

    def chunk_layers(self, n: int) -> int:
        layer_bytes = max(1, n * self.src.page_bytes)
        return max(1, min(self.src.num_layers, self.buffer_bytes_max // layer_bytes))

    def move_pages(self, src_ids: torch.Tensor, dst_ids: torch.Tensor, mode: str = "buffer",
                   layers_per_chunk: Optional[int] = None,
                   host_buf: Optional[torch.Tensor] = None) -> None:
        with self._lock:
            self._move_pages(src_ids, dst_ids, mode, layers_per_chunk, host_buf)

    def _move_pages(self, src_ids, dst_ids, mode, layers_per_chunk, host_buf) -> None:
        n = src_ids.numel()
        if n == 0:
            return
        self._order_after_last_user()
        L = self.src.num_layers
        if mode == "fused":
            ops.move(self.src, src_ids, self.dst, dst_ids)
        elif mode == "buffer":
            k = layers_per_chunk or self.chunk_layers(n)
            buf = self._buffer(min(k, L), n)
            for lb in range(0, L, k):
                le = min(L, lb + k)
                ops.pack(self.src, src_ids, buf[: le - lb], layer_begin=lb, layer_end=le)
                ops.unpack(buf[: le - lb], self.dst, dst_ids, layer_begin=lb, layer_end=le)
        elif mode == "pinned":
            from .kv_utils import ROUNDTRIP_SLOTS, grown_slot_bytes, roundtrip_chunk_layers
            k = layers_per_chunk or roundtrip_chunk_layers(L, n * self.src.page_bytes)
            slot = k * n * self.src.page_bytes
            if self.stager is None or self.stager.slot_bytes < slot:
                current = 0
                if self.stager is not None:
                    current = self.stager.slot_bytes
                    torch.cuda.current_stream(self.src.device).synchronize()
                    self.stager.close()
                self.stager = ops.Stager(grown_slot_bytes(slot, current), ROUNDTRIP_SLOTS, self.src.device)
            if host_buf is None:
                host_buf = torch.empty(L * n * self.src.page_bytes, dtype=torch.uint8, pin_memory=True)
            self.stager.roundtrip(self.src, src_ids, self.dst, dst_ids, host_buf, k)
        else:
            raise ValueError(f"unknown mode {mode!r}")

    def promote_native(self, src_ids, indptr, dst_pages=None, mode: str = "fused",
                       layers_per_chunk: Optional[int] = None):
        """One library call (pace_kv_promote) for a CSR batch: src_ids int32
        (ids in [0, num_pages)), indptr int64, as numpy arrays or
        array.array('i') / array.array('q').  Needs a NativeBlockAllocator.
        Returns the destination tables concatenated (int32 array)."""
        tables, total = self._promote_native(src_ids, indptr, dst_pages, mode, layers_per_chunk, False)
        return np.frombuffer(tables, dtype=np.int32, count=total).copy()

    def _promote_native(self, src_ids, indptr, dst_pages, mode, layers_per_chunk, source_range_ok: bool):
        if not isinstance(self.dst_allocator, NativeBlockAllocator):
            raise TypeError("promote_native needs a NativeBlockAllocator")
        if mode not in ("buffer", "fused"):
            raise ValueError(f"promote_native supports modes 'buffer' and 'fused', not {mode!r}")
        if not isinstance(src_ids, array):
            src_ids = np.ascontiguousarray(src_ids, dtype=np.int32)
        if not isinstance(indptr, array):
            indptr = np.ascontiguousarray(indptr, dtype=np.int64)
        counts = None if dst_pages is None else np.ascontiguousarray(dst_pages, dtype=np.int32)
        n = int(indptr[-1])
        with self._lock:
            if self._promoter is None:
                self._promoter = ops.Promoter(self.src.device)
            stream = self._order_after_last_user()
            buf_ptr, stride, blayers = None, 0, 0
            if mode == "buffer":
                # The migrator's own view: contiguous [k, n, *page_shape] of the
                # pools' dtype on their device, so it needs no further checks.
                k = layers_per_chunk or self.chunk_layers(n)
                buf = self._buffer(min(k, self.src.num_layers), n)
                buf_ptr, stride, blayers = buf.data_ptr(), n * self.src.page_bytes, int(buf.shape[0])
            return self._promoter._launch(self.src, self.dst, self.dst_allocator, src_ids, indptr, counts,
                                          buf_ptr, stride, blayers, None, stream, source_range_ok)

    def promote(self, src_tables: Sequence[Sequence[int]], dst_pages: Optional[Sequence[int]] = None,
                mode: str = "buffer", layers_per_chunk: Optional[int] = None,
                host_buf: Optional[torch.Tensor] = None) -> MigrationPlan:
        """Plans, uploads and moves a batch of requests; returns the plan.  The
        work is enqueued on the current stream (synchronize to wait).  With a
        NativeBlockAllocator, the device modes run as one library call."""
        if isinstance(self.dst_allocator, NativeBlockAllocator) and mode in ("buffer", "fused"):
            # Only the work before the library call adds latency: the plan
            # below is built while the GPU copies.  Tables of int32 ids in
            # range go to the library as they are; the library refuses any
            # other id before allocating, and the ids are then normalised
            # with torch's indexing rules (negative ids count from the end)
            # or rejected with its IndexError.
            tables = None
            fast = _csr_of_int32_tables(src_tables)
            if fast is not None:
                src_ids, indptr, counts = fast
                tables, total = self._promote_native(src_ids, indptr, dst_pages, mode, layers_per_chunk, True)
            if tables is None:
                src_ids, indptr, counts = flatten_tables(src_tables, self.src.num_pages)
                tables, total = self._promote_native(src_ids, indptr, dst_pages, mode, layers_per_chunk, False)
            tables = tables[:total].tolist()
            sizes = counts if dst_pages is None else list(dst_pages)
            dst_tables, dst_ids, pos = [], [], 0
            for n, m in zip(counts, sizes):
                t = tables[pos:pos + m]
                pos += m
                dst_tables.append(t)
                dst_ids.extend(t[:n])
            return MigrationPlan(src_ids.tolist(), dst_ids, dst_tables, indptr.tolist())
        plan = self.plan(src_tables, dst_pages)
        if plan.n_pages:
            try:
                s_ids, d_ids = self.upload(plan)
                self.move_pages(s_ids, d_ids, mode, layers_per_chunk, host_buf)
            except BaseException:
                # Undo the allocation exactly (pages go back in reverse pop
                # order), as the native promotion does on failure.
                self.dst_allocator.free_many(reversed([p for t in plan.dst_tables for p in t]))
                raise
        return plan
