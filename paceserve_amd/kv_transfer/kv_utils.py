"""KVhelper: drop-in for paceserve.kv_transfer.kv_utils.KVhelper
(paceserve/kv_transfer/kv_utils.py:8-56) with its page movement in HIP.

Same constructor, methods, return values and error behaviour:
  - __init__ reads only get_num_q_heads / get_num_kv_heads(parallel_config),
    get_head_size(), dtype, get_num_layers(parallel_config) and
    cache_config.block_size (kv_utils.py:10-24);
  - get_kv_cache(seq, seq_manager) -> (host tensor [L, n, 2, P, H, D], ids),
    or (zeros [L, 1, ...], [0]) when the sequence has no block table
    (kv_utils.py:33-47); out-of-range ids raise IndexError as torch indexing does;
  - insert_kv_cache(cached_content, kv_indices, device) -> bool, never raises:
    any error prints "error during insert kv cache: ..." and returns False
    (kv_utils.py:49-56);
  - reset_kv_cache(num_gpu_blocks) replaces every layer with a zero tensor
    (kv_utils.py:29-31).

What changes underneath: the reference gathers each layer with torch
advanced indexing into a temporary device tensor and copies it to *pageable*
host memory synchronously, L times; here one kernel per layer chunk packs the
pages into a device slot while the previous chunk streams to *pinned* host
memory on a side stream (pace_kv_pack_to_host), and insert is the mirror
(pace_kv_unpack_from_host).  Device-resident transfer buffers skip the host
leg (pack_pages / unpack_pages).
"""
from __future__ import annotations

import threading
from typing import List, Optional, Sequence

import torch

from . import ops

# One-way host legs (pack to host, unpack from host): chunks of >= 64 MiB keep
# the DMA engine at its full rate (measured on MI355X: 53-56 GB/s from 32 MiB
# up), and packing or unpacking a chunk takes ~1% of its copy, so splitting a
# request into more chunks gains nothing.
STAGE_CHUNK_BYTES = 64 << 20
STAGE_SLOTS = 3
# Round trip (pack, D2H, H2D, unpack): device slots per direction.  Measured on
# MI355X on stagers created once and kept (none freed during the measurement),
# 3 and 4 slots ran within 2% of each other at every request size from 256 to
# 8192 tokens, with no size favouring either, so the round trip takes 3,
# which holds less device memory.
ROUNDTRIP_SLOTS = 3
MiB = 1 << 20
STAGE_GROWTH_CAP = 256 * MiB


def grown_slot_bytes(needed: int, current: int = 0) -> int:
    """Slot bytes for a stager that must hold `needed` bytes per slot and
    replaces one of `current` bytes (0: no stager yet), a multiple of 256.
    Freeing a stager's device rings makes the driver scrub that memory with
    the DMA engines the host-to-device copies use (round trips started
    meanwhile measured up to 30% slower), so a stager that must grow at least
    doubles, by at most STAGE_GROWTH_CAP beyond what is needed: a run of
    growing requests replaces it a few times, not once per new size."""
    grown = needed if current <= 0 else max(needed, min(2 * current, needed + STAGE_GROWTH_CAP))
    return -(-grown // 256) * 256


def normalize_page_ids(ids: Sequence[int], num_pages: int) -> List[int]:
    """torch advanced-indexing semantics for a list of page ids: negative ids
    count from the end, anything outside [-num_pages, num_pages) raises
    IndexError."""
    out = []
    for i in ids:
        i = int(i)
        if i < -num_pages or i >= num_pages:
            raise IndexError(f"index {i} is out of bounds for dimension 0 with size {num_pages}")
        out.append(i + num_pages if i < 0 else i)
    return out


def dedup_keep_last(ids: List[int]) -> List[int]:
    """Positions of `ids` that survive when repeated pages are written in
    order (the last write wins, as in a sequential index_put_)."""
    last = {}
    for pos, pid in enumerate(ids):
        last[pid] = pos
    return sorted(last.values())


def chunk_layers(num_layers: int, layer_bytes: int) -> int:
    """Layers per chunk of a one-way host leg (pack_to_host or
    unpack_from_host) for a request of layer_bytes per layer: the fewest
    layers that reach STAGE_CHUNK_BYTES."""
    if layer_bytes <= 0:
        return max(1, num_layers)
    return max(1, min(num_layers, -(-STAGE_CHUNK_BYTES // layer_bytes)))


def roundtrip_chunk_layers(num_layers: int, layer_bytes: int) -> int:
    """Layers per chunk of the device->host->device round trip: the fewest
    layers giving chunks of 8 MiB and more when a request has at most 8 of
    them, 32 MiB and more up to 16 of them, or 128 MiB and more at any count,
    which keeps the pipeline out of the regime where many small chunks stall
    it (16 chunks of 4-8 MiB, or 32 chunks, ran at 5-37 GB/s per direction);
    then as few layers as keep that many chunks, so that the chunks are as
    even as whole layers allow.  Measured on MI355X on stagers created once
    and kept (32 layers, 64 KiB pages): for 256-1024-token requests the chosen
    8-16 MiB chunks ran 2-5% faster than chunks twice as large (32-41 GB/s),
    and for 2048-8192 tokens the choice was the fastest measured or within
    1.4% of it (42-46 GB/s).  Evening out the chunks matters where the first
    count leaves a short last chunk: a 10 MiB request in chunks of 26 and 6
    layers took 562 us, in two of 16 layers 437 us (the first chunk's D2H copy
    and the last one's H2D copy each run alone), and 18-20 MiB requests in
    three chunks ran 3-5% faster as 11 + 11 + 10 layers than as 15 + 15 + 2."""
    if layer_bytes <= 0:
        return max(1, num_layers)
    for k in range(1, num_layers + 1):
        chunk, count = k * layer_bytes, -(-num_layers // k)
        if chunk >= 128 * MiB or (chunk >= 32 * MiB and count <= 16) or (chunk >= 8 * MiB and count <= 8):
            return -(-num_layers // count)
    return max(1, num_layers)


class KVhelper:
    def __init__(self, rank: int, model_config, cache_config, parallel_config):
        self.rank = rank
        self.num_q_heads = model_config.get_num_q_heads(parallel_config)
        self.num_kv_heads = model_config.get_num_kv_heads(parallel_config)
        self.head_dim = model_config.get_head_size()
        self.dtype = model_config.dtype
        self.block_size = cache_config.block_size
        self.num_layers = model_config.get_num_layers(parallel_config)
        self.model_runner = None
        self._pool: Optional[ops.PagedPool] = None
        self._stager: Optional[ops.Stager] = None
        # The reference calls get_kv_cache / insert_kv_cache from several
        # threads of one worker at once (Ray max_concurrency=8,
        # paceserve/engine/base_llm_engine.py:32,166-177; 4+4 insertion
        # threads, paceserve/disutil/decode_instance.py:50-51).  The staging
        # pipeline and the pool table are shared, so a call holds this lock
        # until its copies have finished.
        self._lock = threading.RLock()
        print(f"kv helper initialized on worker: {self.rank}")

    # ---------------------------------------------------------------- pools

    def add_model_runner(self, model_runner) -> None:
        self.model_runner = model_runner

    def _gpu_cache(self) -> List[torch.Tensor]:
        return self.model_runner.attention_backend_wrapper.gpu_cache

    def pool(self) -> ops.PagedPool:
        """The bound cache as a PagedPool (rebuilt when its tensors change)."""
        with self._lock:
            cache = self._gpu_cache()
            if self._pool is None or not self._pool.holds(cache):
                self._pool = ops.PagedPool(cache[: self.num_layers])
            return self._pool

    def _stager_for(self, pool: ops.PagedPool, slot_bytes: int) -> ops.Stager:
        st = self._stager
        current = 0
        if st is not None and (st.slot_bytes < slot_bytes or st.device != pool.device):
            current = st.slot_bytes if st.device == pool.device else 0
            torch.cuda.current_stream(st.device).synchronize()
            st.close()
            st = None
        if st is None:
            st = ops.Stager(grown_slot_bytes(slot_bytes, current), STAGE_SLOTS, pool.device)
            self._stager = st
        return st

    def page_shape(self):
        return (2, self.block_size, self.num_kv_heads, self.head_dim)

    def reset_kv_cache(self, num_gpu_blocks: int) -> None:
        with self._lock:
            cache = self._gpu_cache()
            for i in range(self.num_layers):
                cache[i] = torch.zeros(num_gpu_blocks, *self.page_shape(), dtype=self.dtype, device="cuda")
            self._pool = None

    # ------------------------------------------------------- reference API

    def get_kv_cache(self, seq, seq_manager):
        try:
            kv_page_indices = seq_manager._get_block_table(seq)
        except Exception:
            print(f"seq {seq.seq_id} was not allocated any memory")
            kv_page_indices = None

        if not kv_page_indices:
            return torch.zeros(self.num_layers, 1, *self.page_shape(), dtype=self.dtype), [0]

        with self._lock:
            pool = self.pool()
            ids = normalize_page_ids(kv_page_indices, pool.num_pages)
            n = len(ids)
            host = torch.empty((self.num_layers, n) + pool.page_shape, dtype=pool.dtype, pin_memory=True)
            layer_bytes = n * pool.page_bytes
            k = chunk_layers(self.num_layers, layer_bytes)
            with torch.cuda.device(pool.device):
                stager = self._stager_for(pool, k * layer_bytes)
                stager.pack_to_host(pool, ids, host, k)
                torch.cuda.current_stream(pool.device).synchronize()
        return host, kv_page_indices

    def insert_kv_cache(self, cached_content, kv_indices, device) -> bool:
        try:
            with self._lock:
                self._insert(cached_content, kv_indices, device)
            return True
        except Exception as e:  # the reference's convention: report, never raise
            print(f"error during insert kv cache: {e}")
            return False

    # ------------------------------------------------------ additive API

    def send_kv_cache(self, seq, seq_manager, channel, left_prefill=None, kv_transfer_start=None,
                      timeout: float = 60.0):
        """get_kv_cache through a KVChannel: packs the sequence's pages out of
        this cache into the channel (the zero-page fallback travels as one
        zero page, as get_kv_cache returns it) and returns the KVref that
        replaces the KVobj on the control plane.  Raises like get_kv_cache,
        plus PaceKVError from the channel."""
        from .channel import KVref, kv_size_mb

        try:
            kv_page_indices = seq_manager._get_block_table(seq)
        except Exception:
            print(f"seq {seq.seq_id} was not allocated any memory")
            kv_page_indices = None
        shape = self.page_shape()
        if not kv_page_indices:
            zeros = torch.zeros(self.num_layers, 1, *shape, dtype=self.dtype)
            ref = KVref(seq.seq_id, [0], kv_size_mb(self.num_layers, 1, zeros[0, 0].numel() * zeros.element_size()),
                        left_prefill, kv_transfer_start)
            ref.msg_id = channel.send_host(zeros, ref.meta(), timeout)
            return ref
        pool = self.pool()
        ids = normalize_page_ids(kv_page_indices, pool.num_pages)
        ref = KVref(seq.seq_id, list(kv_page_indices), kv_size_mb(self.num_layers, len(ids), pool.page_bytes),
                    left_prefill, kv_transfer_start)
        with torch.cuda.device(pool.device):
            ref.msg_id = channel.send(pool, ids, ref.meta(), timeout)
        return ref

    def recv_kv_cache(self, channel, kv_indices, device, timeout: float = 60.0) -> bool:
        """insert_kv_cache of the channel message whose header was just
        received: writes its pages to kv_indices of this cache.  Returns
        False on any error (printed, as insert_kv_cache does), after draining
        the message so that the channel stays usable."""
        try:
            self._recv(channel, kv_indices, device, timeout)
            return True
        except Exception as e:
            print(f"error during insert kv cache: {e}")
            try:
                channel.discard(timeout)
            except Exception:
                pass
            return False

    def _recv(self, channel, kv_indices, device, timeout: float) -> None:
        h = channel._current()
        dev = torch.device(device) if not isinstance(device, int) else torch.device("cuda", device)
        if dev.type != "cuda":
            raise RuntimeError(f"cannot insert into a device cache from device {dev}")
        pool = self.pool()
        ids_in = list(kv_indices)
        ids = normalize_page_ids(ids_in, pool.num_pages) if ids_in else []
        if h.num_layers < self.num_layers or h.page_bytes != pool.page_bytes:
            raise RuntimeError(f"message {h.msg_id} holds {h.num_layers} layers of {h.page_bytes}-byte pages; "
                               f"the cache has {self.num_layers} layers of {pool.page_bytes}-byte pages")
        if h.num_layers == self.num_layers and ids and len(ids) == h.n_pages and len(set(ids)) == len(ids):
            with torch.cuda.device(pool.device):
                channel.recv(pool, ids, timeout)
                torch.cuda.current_stream(pool.device).synchronize()
            return
        # Repeated ids (the last write wins), a one-page broadcast, surplus
        # layers or an empty id list: take the payload to host memory and
        # insert it with insert_kv_cache's rules.
        host = torch.empty((h.num_layers, h.n_pages) + pool.page_shape, dtype=pool.dtype, pin_memory=True)
        channel.recv_host(host, timeout)
        with self._lock:                 # the insert uses the shared stager
            self._insert(host, ids_in, device)

    def pack_pages(self, page_ids, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Device-resident pack of this cache's pages: [L, n, 2, P, H, D]."""
        pool = self.pool()
        ids = normalize_page_ids(page_ids, pool.num_pages)
        return ops.pack(pool, ids, out)

    def unpack_pages(self, buf: torch.Tensor, page_ids) -> None:
        """Device-resident unpack into this cache (ids must be distinct)."""
        pool = self.pool()
        ids = normalize_page_ids(page_ids, pool.num_pages)
        if len(set(ids)) != len(ids):
            raise ValueError("destination page ids repeat a page")
        ops.unpack(buf, pool, ids)

    # ------------------------------------------------------------ internals

    def _insert(self, cached_content, kv_indices, device) -> None:
        dev = torch.device(device) if not isinstance(device, int) else torch.device("cuda", device)
        if dev.type != "cuda":
            raise RuntimeError(f"cannot insert into a device cache from device {dev}")
        ids_in = list(kv_indices)
        if not ids_in:
            # torch.tensor([]) is a float tensor, which cannot index.
            raise IndexError("tensors used as indices must be long, int, byte or bool tensors")
        pool = self.pool()
        ids = normalize_page_ids(ids_in, pool.num_pages)
        if not isinstance(cached_content, torch.Tensor):
            raise TypeError("cached_content must be a tensor")
        if cached_content.dim() != 2 + len(pool.page_shape) or cached_content.shape[0] < self.num_layers:
            raise IndexError(f"cached_content of shape {tuple(cached_content.shape)} does not hold "
                             f"{self.num_layers} layers of pages {pool.page_shape}")
        if tuple(cached_content.shape[2:]) != pool.page_shape:
            raise RuntimeError(f"page shape {tuple(cached_content.shape[2:])} != cache page shape {pool.page_shape}")
        if cached_content.dtype != pool.dtype:
            raise RuntimeError(f"Index put requires the source and destination dtypes match, "
                               f"got {pool.dtype} for the destination and {cached_content.dtype} for the source.")
        content = cached_content[: self.num_layers]
        n = content.shape[1]
        if n != len(ids):
            if n != 1:
                raise RuntimeError(f"shape mismatch: value tensor of shape {tuple(content.shape[1:])} "
                                   f"cannot be broadcast to indexing result of shape "
                                   f"{(len(ids),) + pool.page_shape}")
            content = content.expand((self.num_layers, len(ids)) + pool.page_shape)
        keep = dedup_keep_last(ids)
        if len(keep) != len(ids):
            ids = [ids[p] for p in keep]
            content = content[:, keep]
        with torch.cuda.device(pool.device):
            stream = torch.cuda.current_stream(pool.device)
            if content.device.type == "cuda":
                ops.unpack(content.contiguous(), pool, ids)
            else:
                content = content.contiguous()
                layer_bytes = len(ids) * pool.page_bytes
                k = chunk_layers(self.num_layers, layer_bytes)
                stager = self._stager_for(pool, k * layer_bytes)
                stager.unpack_from_host(content, pool, ids, k)
            stream.synchronize()
