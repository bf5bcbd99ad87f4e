"""CPU oracle of PaceServe's KV-cache migration path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
CPU-baseline leg may import this module, and only as the expected answer that
results are compared with, or as the timed CPU baseline; the product path
(paceserve_amd) never calls it.

Each function restates one step of the reference's behaviour in plain numpy
(raw 16-bit words: the path copies bytes, it does no arithmetic) and cites
the reference file:line it follows.  How each is pinned (the checks in
tests/test_oracle.py):
  - pack / unpack / move:  the committed golden fixtures (written by an
    element-by-element loop in tests/golden/make_golden.py, not by this file),
    torch.index_select / Tensor.index_copy_ (the textbook routines the
    reference's advanced indexing reduces to for unique ids), and invariants:
    untouched pages stay unchanged, the source is never written, unpack(pack)
    restores the pages, a batch equals its requests one at a time.
  - zero_page_fallback: closed form (all-zero [L,1,...] and [0]).
  - BlockAllocator / allocate_table / free_table: closed forms of a LIFO list
    over [0, N): a fresh pool hands out N-1, N-2, ...; a free then allocate
    returns the freed pages; exhaustion raises the reference's message.
  - remap_dst_table: the three cases of the rule (len n, n+1, anything else).
  - pages_for_tokens / last_page_len: brute-force slot filling.
  - get_seq_lens / get_batch_indices_positions / append_paged_kv_cache: the
    reference's FlashInfer example as a known answer (fixture
    tests/golden/layout_flashinfer_example.npz, written by a token loop in
    make_golden.py), and consistency: appending a sequence token by token
    (decode steps) equals appending it at once (prefill), in any chunking.
"""
from __future__ import annotations

from typing import Iterable, List, Optional, Sequence, Tuple

import numpy as np

OOM_MESSAGE = "Out of memory! No free blocks are available."


# --------------------------------------------------------------------------
# Page copies
# --------------------------------------------------------------------------

def _norm_ids(ids: Iterable[int], num_pages: int) -> np.ndarray:
    """Torch advanced indexing semantics for page ids: negatives wrap once,
    anything outside [-num_pages, num_pages) raises IndexError."""
    a = np.asarray(list(ids), dtype=np.int64)
    if a.size and (a.min() < -num_pages or a.max() >= num_pages):
        raise IndexError(f"page id out of range for a pool of {num_pages} pages")
    return np.where(a < 0, a + num_pages, a)


def pack(layers: Sequence[np.ndarray], page_ids: Sequence[int]) -> np.ndarray:
    """out[l, j] = layers[l][page_ids[j]] -> [L, n, 2, P, H, D].

    Follows KVhelper.get_kv_cache, paceserve/kv_transfer/kv_utils.py:44-46
    (seq_cache = zeros(L, n, ...); seq_cache[i] = gpu_cache[i][tensor(ids)])."""
    num_pages = layers[0].shape[0]
    ids = _norm_ids(page_ids, num_pages)
    out = np.zeros((len(layers), ids.size) + layers[0].shape[1:], dtype=layers[0].dtype)
    for i, layer in enumerate(layers):
        out[i] = layer[ids]
    return out


def dedup_keep_last(page_ids: Sequence[int], num_pages: int) -> Tuple[np.ndarray, np.ndarray]:
    """(positions, ids) with each repeated destination page kept only at its
    last position: what a sequential index_put_ leaves behind."""
    ids = _norm_ids(page_ids, num_pages)
    last = {}
    for pos, pid in enumerate(ids.tolist()):
        last[pid] = pos
    pos = np.array(sorted(last.values()), dtype=np.int64)
    return pos, ids[pos]


def unpack(buf: np.ndarray, layers: Sequence[np.ndarray], page_ids: Sequence[int]) -> List[np.ndarray]:
    """Returns copies of `layers` with layers[l][page_ids[j]] = buf[l, j].

    Follows KVhelper.insert_kv_cache, paceserve/kv_transfer/kv_utils.py:49-52
    (gpu_cache[i][tensor(kv_indices)] = cached_content[i].to(device)), with a
    repeated page resolved as the last write."""
    num_pages = layers[0].shape[0]
    pos, ids = dedup_keep_last(page_ids, num_pages)
    if buf.shape[1] != len(page_ids) and buf.shape[1] != 1:
        raise ValueError(f"buffer holds {buf.shape[1]} pages for {len(page_ids)} ids")
    out = [l.copy() for l in layers]
    for i in range(len(layers)):
        src = buf[i] if buf.shape[1] == len(page_ids) else np.broadcast_to(buf[i], (len(page_ids),) + buf.shape[2:])
        out[i][ids] = src[pos]
    return out


def move(src_layers: Sequence[np.ndarray], src_ids: Sequence[int], dst_layers: Sequence[np.ndarray],
         dst_ids: Sequence[int]) -> List[np.ndarray]:
    """get_kv_cache on the source followed by insert_kv_cache on the
    destination (paceserve/worker/base_worker.py:236-281)."""
    return unpack(pack(src_layers, src_ids), dst_layers, dst_ids)


def zero_page_fallback(num_layers: int, page_shape: Tuple[int, ...], dtype) -> Tuple[np.ndarray, List[int]]:
    """A sequence with no block table yields one all-zero page and ids [0]
    (paceserve/kv_transfer/kv_utils.py:34-42)."""
    return np.zeros((num_layers, 1) + tuple(page_shape), dtype=dtype), [0]


# --------------------------------------------------------------------------
# Block tables
# --------------------------------------------------------------------------

def pages_for_tokens(num_tokens: int, page_size: int) -> int:
    """Logical blocks of a sequence: ceil(tokens / page_size)
    (paceserve/core/datatypes/sequence.py:73-93, block.py:12-50;
    DecodeBlockSpaceManager.get_num_initial_blocks,
    paceserve/core/block_space_manager/decode_block_space_manager.py:12-13)."""
    return (num_tokens + page_size - 1) // page_size


def last_page_len(num_tokens: int, page_size: int) -> int:
    """Valid slots of the last page: tokens % P or P
    (paceserve/model_executor/attention/flashinfer_attention_wrapper.py:139-141)."""
    return num_tokens % page_size or page_size


class BlockAllocator:
    """LIFO free list over [0, num_blocks)
    (paceserve/core/block_space_manager/base_block_space_manager.py:11-47)."""

    def __init__(self, num_blocks: int, free_list: Optional[Sequence[int]] = None):
        self.num_blocks = num_blocks
        self.free_blocks: List[int] = list(range(num_blocks)) if free_list is None else list(free_list)

    def allocate(self) -> int:
        if not self.free_blocks:
            raise ValueError(OOM_MESSAGE)
        return self.free_blocks.pop()

    def free(self, block: int) -> None:
        self.free_blocks.append(block)

    def num_free(self) -> int:
        return len(self.free_blocks)


def allocate_table(alloc: BlockAllocator, n: int) -> List[int]:
    """BaseBlockSpaceManager.allocate: n successive pops
    (base_block_space_manager.py:89-97)."""
    return [alloc.allocate() for _ in range(n)]


def free_table(alloc: BlockAllocator, table: Sequence[int]) -> None:
    """BaseBlockSpaceManager._free_block_table frees each distinct page once
    (base_block_space_manager.py:119-121).  The reference iterates a set of
    block objects, whose order follows object addresses and is not fixed;
    this oracle frees distinct pages in first-occurrence order."""
    seen = set()
    for b in table:
        if b not in seen:
            seen.add(b)
            alloc.free(b)


def remap_dst_table(dst_table: Sequence[int], n_src: int) -> Optional[List[int]]:
    """Destination ids for n_src packed pages
    (BaseWorker._insert_kv_cache, paceserve/worker/base_worker.py:264-277):
    a table of n_src pages is used whole; one of n_src + 1 pages (the first
    generated token opened a new page) drops its last page, which stays
    untouched; any other length makes the reference's insert fail (torch
    raises on the shape mismatch), returned here as None."""
    if len(dst_table) == n_src:
        return list(dst_table)
    if len(dst_table) == n_src + 1:
        return list(dst_table[:-1])
    return None


# --------------------------------------------------------------------------
# The reference CPU path timed as the CPU baseline
# --------------------------------------------------------------------------

def torch_cpu_pack_unpack(src_layers, src_idx, dst_layers, dst_idx, buf=None):
    """The reference's per-layer CPU path on host tensors:
    buf[l] = index_select(src[l], 0, src_idx); dst[l].index_copy_(0, dst_idx, buf[l])
    (paceserve/kv_transfer/kv_utils.py:44-46 and :51-52 on host tensors)."""
    import torch

    n = src_idx.numel()
    if buf is None:
        buf = torch.empty((len(src_layers), n) + tuple(src_layers[0].shape[1:]), dtype=src_layers[0].dtype)
    for i, (s, d) in enumerate(zip(src_layers, dst_layers)):
        torch.index_select(s, 0, src_idx, out=buf[i])
        d.index_copy_(0, dst_idx, buf[i])
    return buf


# --------------------------------------------------------------------------
# Paged append (the producer of page contents)
# --------------------------------------------------------------------------
# The reference calls FlashInfer (flashinfer==0.2.0, requirements.txt:40; not
# vendored) at paceserve/model_executor/attention/flashinfer_attention_wrapper.py:
# 241-255.  Its published semantics are restated here; the known answer is the
# reference's own example, examples/flashinfer_example.py:76-114.

def get_seq_lens(kv_indptr: Sequence[int], kv_last_page_len: Sequence[int], page_size: int) -> np.ndarray:
    """Tokens per request: max(pages - 1, 0) * page_size + last_page_len."""
    ip = np.asarray(kv_indptr, dtype=np.int64)
    pages = ip[1:] - ip[:-1]
    return np.maximum(pages - 1, 0) * page_size + np.asarray(kv_last_page_len, dtype=np.int64)


def get_batch_indices_positions(append_indptr: Sequence[int], seq_lens: Sequence[int], nnz: int):
    """(batch_indices, positions): appended token t of request b is the
    request's token seq_lens[b] - append_len[b] + t."""
    bi = np.full(nnz, -1, dtype=np.int64)
    pos = np.full(nnz, -1, dtype=np.int64)
    for b in range(len(append_indptr) - 1):
        a0, a1 = int(append_indptr[b]), int(append_indptr[b + 1])
        for t in range(a1 - a0):
            if a0 + t < nnz:
                bi[a0 + t] = b
                pos[a0 + t] = int(seq_lens[b]) - (a1 - a0) + t
    return bi, pos


def append_paged_kv_cache(key: np.ndarray, value: np.ndarray, batch_indices, positions, cache: np.ndarray,
                          kv_indices, kv_indptr, page_size: int) -> np.ndarray:
    """Returns a copy of one layer's cache [pages, 2, P, H, D] with token i's K
    and V rows written to page kv_indices[kv_indptr[b] + pos // P], slot
    pos % P (K at index 0, V at index 1)."""
    out = cache.copy()
    for i in range(key.shape[0]):
        b, p = int(batch_indices[i]), int(positions[i])
        if b < 0 or p < 0:
            continue
        it = int(kv_indptr[b]) + p // page_size
        if it >= int(kv_indptr[b + 1]):
            continue
        page = int(kv_indices[it])
        out[page, 0, p % page_size] = key[i]
        out[page, 1, p % page_size] = value[i]
    return out
