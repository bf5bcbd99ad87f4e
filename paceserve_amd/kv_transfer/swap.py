"""Swap space for preempted requests: a host-resident pinned page pool.

The reference parks a preempted decode request's KV cache in host DRAM by
packing it into a KVobj without freeing the worker's pages, and re-inserts it
when the request is scheduled again (paceserve/engine/decode_llm_engine.py:31-41,
paceserve/worker/base_worker.py:245-247, paceserve/disutil/decode_instance.py:176-192).
SwapSpace keeps those pages in a paged host pool instead: swap_out moves a
request's device pages into host pages allocated from the host pool's own LIFO
allocator (one kernel writing pinned memory across PCIe) and swap_in moves them
back into newly allocated device pages, after which the host pages are free.
"""
from __future__ import annotations

import threading
from typing import Dict, List

import torch

from ..core.block_manager import NativeBlockAllocator
from . import ops
from .kv_utils import normalize_page_ids


class PageReaders:
    """Which event each host page's last reader (a swap-in) recorded, so that
    a swap-out writing a page waits for exactly the swap-ins that read it,
    whichever streams they ran on.  Works with any event object that a
    stream can wait on; at most one entry per host page."""

    def __init__(self):
        self._last: Dict[int, object] = {}

    def record(self, pages, event) -> None:
        for p in pages:
            self._last[int(p)] = event

    def take(self, pages) -> list:
        """The distinct events recorded for `pages` (in first-seen order),
        forgotten: the caller orders its writes after them."""
        out, seen = [], set()
        for p in pages:
            ev = self._last.pop(int(p), None)
            if ev is not None and id(ev) not in seen:
                seen.add(id(ev))
                out.append(ev)
        return out

    def __len__(self) -> int:
        return len(self._last)


class SwapSpace:
    def __init__(self, dev_pool, num_host_pages: int):
        self.dev = ops.as_pool(dev_pool)
        self.host = ops.HostPagePool.like(self.dev, num_host_pages)
        self.host_allocator = NativeBlockAllocator(self.dev.page_shape[1], num_host_pages)
        self.tables: Dict[str, List[int]] = {}   # seq_id -> host pages
        # seq_id -> event recorded after its swap-out: its swap-in, on any
        # stream, reads the host pages only after they are written.
        self._swapped_out: Dict[str, torch.cuda.Event] = {}
        # The event recorded after the swap-in that last read each host page:
        # a swap-out that reuses the page waits for it, on any stream.
        self._readers = PageReaders()
        # The reference swaps in from several insertion threads while its
        # engine thread swaps out (paceserve/disutil/decode_instance.py:50-51,
        # paceserve/engine/decode_llm_engine.py:31-41).
        self._lock = threading.Lock()

    def num_free_host_pages(self) -> int:
        return self.host_allocator.get_num_free_blocks()

    def swap_out(self, seq_id: str, dev_table: List[int]) -> List[int]:
        """Copies the request's device pages into newly allocated host pages;
        the device pages stay allocated (the caller frees them)."""
        with self._lock:
            return self._swap_out(seq_id, dev_table)

    def _swap_out(self, seq_id: str, dev_table: List[int]) -> List[int]:
        if seq_id in self.tables:
            raise ValueError(f"sequence {seq_id} is already swapped out")
        ids = normalize_page_ids(dev_table, self.dev.num_pages)
        host_table = self.host_allocator.allocate_many(len(ids))
        stream = torch.cuda.current_stream(self.dev.device)
        readers = self._readers.take(host_table)
        try:
            for r in readers:
                stream.wait_event(r)
            ops.swap_out(self.dev, ids, self.host, host_table)
        except Exception:
            # The pages go back unwritten; an event on this stream, which
            # already waits for their readers, stands in for those readers.
            ev = torch.cuda.Event()
            ev.record(stream)
            self._readers.record(host_table, ev)
            self.host_allocator.free_many(reversed(host_table))
            raise
        ev = torch.cuda.Event()
        ev.record(stream)
        self._swapped_out[seq_id] = ev
        self.tables[seq_id] = host_table
        return host_table

    def swap_in(self, seq_id: str, dev_table: List[int]) -> None:
        """Copies the request's host pages into dev_table (allocated by the
        caller) and returns the host pages to the host allocator.  The copy
        waits for the request's swap_out, and a later swap_out that reuses any
        of these host pages, on any stream, waits for this copy before it
        writes them."""
        with self._lock:
            self._swap_in(seq_id, dev_table)

    def _swap_in(self, seq_id: str, dev_table: List[int]) -> None:
        # Nothing changes until the copy is enqueued: a rejected call leaves
        # the request swapped out, its host pages held.
        host_table = self.tables[seq_id]
        ids = normalize_page_ids(dev_table, self.dev.num_pages)
        if len(ids) != len(host_table):
            raise ValueError(f"{len(ids)} device pages for {len(host_table)} swapped pages")
        stream = torch.cuda.current_stream(self.dev.device)
        stream.wait_event(self._swapped_out[seq_id])
        ops.swap_in(self.host, host_table, self.dev, ids)
        ev = torch.cuda.Event()
        ev.record(stream)
        self._readers.record(host_table, ev)
        del self.tables[seq_id], self._swapped_out[seq_id]
        self.host_allocator.free_many(host_table)

    def holds(self, seq_id: str) -> bool:
        with self._lock:
            return seq_id in self.tables
