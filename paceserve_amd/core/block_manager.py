"""Block (page) allocation for paged KV pools.

Mirrors the reference's allocator semantics, which decide which destination
pages a migrated request lands in:
  - BlockAllocator: a LIFO free list over [0, num_blocks); a fresh pool hands
    out num_blocks-1, num_blocks-2, ...; an empty list raises
    ValueError("Out of memory! No free blocks are available.")
    (paceserve/core/block_space_manager/base_block_space_manager.py:11-47).
  - BlockSpaceManager: per-sequence block tables; allocate pops
    len(seq.logical_token_blocks) pages (decode_block_space_manager.py:12-13,
    base_block_space_manager.py:89-97); free returns each distinct page once
    (:112-121); get_block_table returns page ids (:136-138).

Page ids are plain ints here (the reference wraps them in PhysicalTokenBlock
objects and frees them in set() order, which follows object addresses and is
therefore unspecified; distinct pages are freed here in first-occurrence
order).
"""
from __future__ import annotations

import threading
from typing import Dict, Iterable, List, Optional

OOM_MESSAGE = "Out of memory! No free blocks are available."


class BlockAllocator:
    """LIFO free list of page ids."""

    def __init__(self, block_size: int, num_blocks: int, free_list: Optional[Iterable[int]] = None):
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.lock = threading.Lock()
        self.free_blocks: List[int] = list(range(num_blocks)) if free_list is None else list(free_list)

    def allocate(self) -> int:
        with self.lock:
            if not self.free_blocks:
                raise ValueError(OOM_MESSAGE)
            return self.free_blocks.pop()

    def allocate_many(self, n: int) -> List[int]:
        """n pages in the order n successive allocate() calls return them;
        all-or-nothing."""
        with self.lock:
            if n > len(self.free_blocks):
                raise ValueError(OOM_MESSAGE)
            if n == 0:
                return []
            got = self.free_blocks[-n:]
            del self.free_blocks[-n:]
            got.reverse()
            return got

    def free(self, block: int) -> None:
        with self.lock:
            self.free_blocks.append(block)

    def free_many(self, blocks: Iterable[int]) -> None:
        """Returns each distinct page of `blocks` once, in first-occurrence
        order (a table that repeats a page frees it once)."""
        with self.lock:
            self.free_blocks.extend(dict.fromkeys(blocks))

    def get_num_free_blocks(self) -> int:
        with self.lock:
            return len(self.free_blocks)


class NativeBlockAllocator:
    """BlockAllocator over the library's C++ allocator (pace_kv_allocator):
    same LIFO order and errors, with batch allocation, batch planning and
    single-call promotion done without per-page Python work."""

    def __init__(self, block_size: int, num_blocks: int, free_list: Optional[Iterable[int]] = None):
        import ctypes

        import numpy as np

        from .. import _native

        self._np = np
        self._ct = ctypes
        self._lib = _native.load()
        self.block_size = block_size
        self.num_blocks = num_blocks
        handle = ctypes.c_void_p()
        if free_list is None:
            _native.check(self._lib.pace_kv_allocator_create(num_blocks, None, 0, ctypes.byref(handle)))
        else:
            arr = np.ascontiguousarray(np.fromiter(free_list, dtype=np.int32))
            _native.check(self._lib.pace_kv_allocator_create(
                num_blocks, arr.ctypes.data, arr.size, ctypes.byref(handle)))
        self.handle = handle.value

    def _check(self, rc: int) -> None:
        from .. import _native

        if rc == _native.PACE_KV_ENOMEM:
            raise ValueError(OOM_MESSAGE)
        _native.check(rc)

    def allocate(self) -> int:
        return self.allocate_many(1)[0]

    def allocate_array(self, n: int):
        out = self._np.empty(n, dtype=self._np.int32)
        self._check(self._lib.pace_kv_allocator_allocate(self.handle, n, out.ctypes.data if n else None))
        return out

    def allocate_many(self, n: int) -> List[int]:
        return self.allocate_array(n).tolist()

    def free(self, block: int) -> None:
        self.free_many([block])

    def free_many(self, blocks: Iterable[int]) -> None:
        arr = self._np.ascontiguousarray(self._np.fromiter(blocks, dtype=self._np.int32))
        self._check(self._lib.pace_kv_allocator_free(self.handle, arr.ctypes.data if arr.size else None,
                                                     arr.size))

    def get_num_free_blocks(self) -> int:
        n = self._ct.c_int64()
        self._check(self._lib.pace_kv_allocator_num_free(self.handle, self._ct.byref(n)))
        return n.value

    @property
    def free_blocks(self) -> List[int]:
        n = self.get_num_free_blocks()
        out = self._np.empty(max(n, 1), dtype=self._np.int32)
        ln = self._ct.c_int64()
        self._check(self._lib.pace_kv_allocator_snapshot(self.handle, out.ctypes.data, out.size,
                                                         self._ct.byref(ln)))
        return out[: ln.value].tolist()

    def plan(self, src_ids, indptr, src_pool_pages: int, dst_pages=None):
        """pace_kv_plan: (dst_tables, dst_ids) as int32 arrays for the CSR
        batch (src_ids int32, indptr int64)."""
        np = self._np
        src_ids = np.ascontiguousarray(src_ids, dtype=np.int32)
        indptr = np.ascontiguousarray(indptr, dtype=np.int64)
        R = indptr.size - 1
        counts = np.diff(indptr) if dst_pages is None else np.ascontiguousarray(dst_pages, dtype=np.int32)
        tables = np.empty(max(int(counts.sum()), 1), dtype=np.int32)
        ids = np.empty(max(src_ids.size, 1), dtype=np.int32)
        dp = None if dst_pages is None else counts
        self._check(self._lib.pace_kv_plan(
            self.handle, R, indptr.ctypes.data, src_ids.ctypes.data, src_pool_pages,
            None if dp is None else dp.ctypes.data, tables.ctypes.data, ids.ctypes.data))
        return tables[: int(counts.sum())], ids[: src_ids.size]

    def close(self) -> None:
        if getattr(self, "handle", None):
            handle, self.handle = self.handle, None
            self._lib.pace_kv_allocator_destroy(handle)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class BlockSpaceManager:
    """Sequence id -> block table, over one BlockAllocator (the decode-style
    manager: a sequence initially gets one page per logical token block)."""

    def __init__(self, block_size: int, num_gpu_blocks: int, max_model_len: Optional[int] = None,
                 watermark: float = 0.01, free_list: Optional[Iterable[int]] = None,
                 native: bool = False):
        if watermark < 0.0:
            raise ValueError("watermark must be >= 0")
        self.block_size = block_size
        self.num_total_gpu_blocks = num_gpu_blocks
        self.max_model_len = max_model_len
        self.watermark = watermark
        self.watermark_blocks = int(watermark * num_gpu_blocks)
        cls = NativeBlockAllocator if native else BlockAllocator
        self.gpu_allocator = cls(block_size, num_gpu_blocks, free_list)
        self.block_tables: Dict[str, List[int]] = {}
        # Held by callers that check for room and then allocate, as one step
        # (several insertion threads share one manager).
        self.alloc_lock = threading.Lock()

    def get_num_initial_blocks(self, seq) -> int:
        return len(seq.logical_token_blocks)

    def can_allocate(self, seq) -> bool:
        need = self.get_num_initial_blocks(seq)
        return self.gpu_allocator.get_num_free_blocks() - need >= self.watermark_blocks

    def allocate(self, seq) -> None:
        self.block_tables[seq.seq_id] = self.gpu_allocator.allocate_many(self.get_num_initial_blocks(seq))

    def can_append_slot(self) -> bool:
        return self.gpu_allocator.get_num_free_blocks() > 0

    def append_slot(self, seq) -> None:
        table = self.block_tables[seq.seq_id]
        if len(table) < len(seq.logical_token_blocks):
            table.append(self.gpu_allocator.allocate())

    def _free_block_table(self, table: List[int]) -> None:
        self.gpu_allocator.free_many(table)

    def free(self, seq) -> None:
        table = self.block_tables.pop(seq.seq_id, None)
        if table is not None:
            self._free_block_table(table)

    def reset(self) -> None:
        for table in self.block_tables.values():
            self._free_block_table(table)
        self.block_tables.clear()

    def get_block_table(self, seq) -> List[int]:
        return list(self.block_tables[seq.seq_id])

    def get_num_free_gpu_blocks(self) -> int:
        return self.gpu_allocator.get_num_free_blocks()

    def is_allocated(self, seq) -> bool:
        return seq.seq_id in self.block_tables


def remap_dst_table(dst_table: List[int], n_src: int) -> Optional[List[int]]:
    """Destination page ids for n_src packed pages
    (BaseWorker._insert_kv_cache, paceserve/worker/base_worker.py:264-277).

    A table of n_src pages is used whole.  A table of n_src + 1 pages (the
    first generated token opened a new page on the destination) drops its
    last page, which is left untouched.  Any other length cannot be inserted
    (the reference's torch assignment raises on the shape mismatch): None."""
    if len(dst_table) == n_src:
        return list(dst_table)
    if len(dst_table) == n_src + 1:
        return list(dst_table[:-1])
    return None
