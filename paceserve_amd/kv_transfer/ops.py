"""Tensor-level KV page movement over libpace_kv (HIP kernels for gfx950).

A *pool* is the per-layer paged KV cache of one instance: a list of L device
tensors, each contiguous with shape [num_pages, 2, page_size, num_kv_heads,
head_dim] (the layout of FlashinferAttentionWrapper.gpu_cache,
paceserve/model_executor/attention/flashinfer_attention_wrapper.py:53-73).
A *transfer buffer* is one contiguous tensor [L, n, 2, page_size, H, D]: the
layout KVhelper.get_kv_cache returns (paceserve/kv_transfer/kv_utils.py:44).

Everything here enqueues work on the caller's current HIP stream and returns
without waiting, like a torch op.  Page ids may be given as a device int32
tensor (used as is) or as host data (copied to the device on the current
stream through pinned memory).  Ids outside [0, num_pages) are never
dereferenced by the kernels; the host-side entry points above this module
validate ids before they reach the device.
"""
from __future__ import annotations

import ctypes
from array import array
from typing import List, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from .. import _native

IdsLike = Union[torch.Tensor, Sequence[int]]


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(device: torch.device) -> int:
    """The hipStream_t of torch's current stream on `device`, read without
    building a Stream object where torch offers that (a few microseconds less
    per call, which counts against launches of 20 us)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is None:
        return torch.cuda.current_stream(index).cuda_stream
    return _raw_stream(index)


def _addr(a) -> int:
    """Address of a contiguous numpy array's or array.array's first element."""
    if isinstance(a, array):
        return a.buffer_info()[0]
    return a.__array_interface__["data"][0]


class PagedPool:
    """Per-layer paged KV tensors of one cache, plus their cached layer table.
    host=True builds a host-resident pool of pinned tensors (see HostPagePool)."""

    def __init__(self, layers: Sequence[torch.Tensor], host: bool = False):
        layers = list(layers)
        if not layers:
            raise ValueError("a pool needs at least one layer tensor")
        first = layers[0]
        if first.dim() != 5 or first.shape[1] != 2:
            raise ValueError(
                f"layer tensors must be [num_pages, 2, page_size, num_kv_heads, head_dim], got {tuple(first.shape)}")
        for i, t in enumerate(layers):
            if t.shape != first.shape or t.dtype != first.dtype or t.device != first.device:
                raise ValueError(f"layer {i} differs in shape/dtype/device from layer 0")
            if not t.is_contiguous():
                raise ValueError(f"layer {i} is not contiguous")
        if host:
            if first.device.type != "cpu" or not all(t.is_pinned() for t in layers):
                raise ValueError("host pool layers must be pinned CPU tensors")
        elif first.device.type != "cuda":
            raise ValueError("pool layers must be device tensors")
        self.host = host
        self.layers: List[torch.Tensor] = layers
        self.num_layers = len(layers)
        self.num_pages = int(first.shape[0])
        self.page_shape: Tuple[int, ...] = tuple(int(s) for s in first.shape[1:])
        self.dtype = first.dtype
        self.device = first.device
        self.page_bytes = int(first[0].numel()) * first.element_size()
        if self.page_bytes % 16:
            raise ValueError(f"page bytes ({self.page_bytes}) must be a multiple of 16")
        self._table = _native.pointer_array([t.data_ptr() for t in layers])
        self._table_addr = ctypes.addressof(self._table)

    def table(self, layer_begin: int = 0) -> int:
        """Address of the layer table entry for layer `layer_begin`."""
        return self._table_addr + layer_begin * ctypes.sizeof(ctypes.c_void_p)

    def holds(self, layers: Sequence[torch.Tensor]) -> bool:
        """True if `layers` are exactly the tensors this pool was built from."""
        return len(layers) == self.num_layers and all(a is b for a, b in zip(layers, self.layers))

    def compatible(self, other: "PagedPool") -> bool:
        return (self.page_shape == other.page_shape and self.dtype == other.dtype
                and self.device == other.device)

    def layer_range(self, layer_begin: int, layer_end: Optional[int]) -> Tuple[int, int]:
        end = self.num_layers if layer_end is None else layer_end
        if not (0 <= layer_begin <= end <= self.num_layers):
            raise ValueError(f"layer range [{layer_begin}, {end}) outside [0, {self.num_layers})")
        return layer_begin, end


class HostPagePool(PagedPool):
    """A host-resident pool of pages in pinned memory with the device pool's
    layout: where a preempted request's pages wait until they are swapped back."""

    def __init__(self, num_layers: int, num_pages: int, page_shape: Tuple[int, ...], dtype: torch.dtype):
        layers = [torch.empty((num_pages,) + tuple(page_shape), dtype=dtype, pin_memory=True)
                  for _ in range(num_layers)]
        super().__init__(layers, host=True)

    @classmethod
    def like(cls, pool: PagedPool, num_pages: int) -> "HostPagePool":
        return cls(pool.num_layers, num_pages, pool.page_shape, pool.dtype)


def as_pool(pool_or_layers) -> PagedPool:
    return pool_or_layers if isinstance(pool_or_layers, PagedPool) else PagedPool(pool_or_layers)


def device_ids(ids: IdsLike, device: torch.device, distinct: bool = False) -> torch.Tensor:
    """Page ids as a contiguous int32 device tensor (host data is copied
    asynchronously on the current stream through pinned memory).

    distinct=True (destination ids: two waves copying into one page race,
    so the page would hold either source) rejects host data that repeats a
    page with ValueError; device tensors are used as they are, and a caller
    passing them is responsible for distinct ids."""
    if isinstance(ids, torch.Tensor):
        if ids.device.type == "cuda":
            if ids.dtype != torch.int32 or not ids.is_contiguous() or ids.dim() != 1:
                raise ValueError("device page ids must be a contiguous 1-D int32 tensor")
            if ids.device != device:
                raise ValueError(f"page ids on {ids.device}, pool on {device}")
            return ids
        host = ids.to(torch.int32).contiguous().view(-1)
        if host.numel() == 0:
            return torch.empty(0, dtype=torch.int32, device=device)
        if distinct:
            _check_distinct(host.numpy())
        if not host.is_pinned():
            host = host.pin_memory()
    else:
        ids = list(ids)
        if not ids:
            return torch.empty(0, dtype=torch.int32, device=device)
        if distinct:
            _check_distinct(np.asarray(ids))
        host = torch.tensor(ids, dtype=torch.int32, pin_memory=True)
    return host.to(device, non_blocking=True)


def _check_distinct(ids: np.ndarray) -> None:
    if ids.size > 1:
        u, c = np.unique(ids, return_counts=True)
        if (c > 1).any():
            raise ValueError(f"destination page {int(u[c > 1][0])} appears more than once; destination page "
                             "ids must be distinct")


def _err_ptr(err: Optional[torch.Tensor]) -> Optional[int]:
    if err is None:
        return None
    if err.dtype != torch.int32 or err.device.type != "cuda" or err.numel() < 1:
        raise ValueError("err must be an int32 device tensor with at least one element")
    return err.data_ptr()


def _check_buffer(buf: torch.Tensor, pool: PagedPool, n_layers: int, n_pages: int, what: str) -> int:
    """Validates a transfer buffer [n_layers, >= n_pages, *page_shape]; returns
    its layer stride in bytes."""
    if buf.device != pool.device or buf.dtype != pool.dtype:
        raise ValueError(f"{what}: buffer dtype/device ({buf.dtype}, {buf.device}) "
                         f"differ from the pool's ({pool.dtype}, {pool.device})")
    if not buf.is_contiguous() or buf.dim() != 2 + len(pool.page_shape):
        raise ValueError(f"{what}: buffer must be a contiguous [L, n, *page_shape] tensor")
    if tuple(buf.shape[2:]) != pool.page_shape:
        raise ValueError(f"{what}: buffer page shape {tuple(buf.shape[2:])} != pool page shape {pool.page_shape}")
    if buf.shape[0] < n_layers or buf.shape[1] < n_pages:
        raise ValueError(f"{what}: buffer {tuple(buf.shape[:2])} holds fewer than "
                         f"({n_layers}, {n_pages}) layer pages")
    return buf.stride(0) * buf.element_size()


def pack(src, page_ids: IdsLike, out: Optional[torch.Tensor] = None, *,
         layer_begin: int = 0, layer_end: Optional[int] = None,
         err: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[l - layer_begin, j] = src.layers[l][page_ids[j]] (whole pages, bit-exact).

    Returns the [layers, n, *page_shape] transfer buffer (`out` if given)."""
    pool = as_pool(src)
    lb, le = pool.layer_range(layer_begin, layer_end)
    ids = device_ids(page_ids, pool.device)
    n = ids.numel()
    if out is None:
        out = torch.empty((le - lb, n) + pool.page_shape, dtype=pool.dtype, device=pool.device)
    stride = _check_buffer(out, pool, le - lb, n, "pack")
    _native.check(_native.load().pace_kv_pack(
        pool.table(lb), le - lb, pool.num_pages, ids.data_ptr() if n else None, n,
        pool.page_bytes, out.data_ptr(), stride, _err_ptr(err), _stream_handle(pool.device)))
    return out


def unpack(buf: torch.Tensor, dst, page_ids: IdsLike, *, layer_begin: int = 0,
           layer_end: Optional[int] = None, err: Optional[torch.Tensor] = None) -> None:
    """dst.layers[l][page_ids[j]] = buf[l - layer_begin, j]; other pages untouched.

    page_ids must not repeat a page: host ids that do are rejected
    (ValueError), device ids are the caller's to keep distinct (KVhelper
    removes repeats on the host, keeping the last write)."""
    pool = as_pool(dst)
    lb, le = pool.layer_range(layer_begin, layer_end)
    ids = device_ids(page_ids, pool.device, distinct=True)
    n = ids.numel()
    stride = _check_buffer(buf, pool, le - lb, n, "unpack")
    _native.check(_native.load().pace_kv_unpack(
        buf.data_ptr(), stride, pool.table(lb), le - lb, pool.num_pages,
        ids.data_ptr() if n else None, n, pool.page_bytes, _err_ptr(err),
        _stream_handle(pool.device)))


def move(src, src_ids: IdsLike, dst, dst_ids: IdsLike, *, layer_begin: int = 0,
         layer_end: Optional[int] = None, err: Optional[torch.Tensor] = None) -> None:
    """dst.layers[l][dst_ids[j]] = src.layers[l][src_ids[j]], one fused pass with
    no transfer buffer (same destination bytes as pack followed by unpack).
    dst_ids must be distinct, as for unpack."""
    sp, dp = as_pool(src), as_pool(dst)
    if not sp.compatible(dp) or sp.num_layers != dp.num_layers:
        raise ValueError("source and destination pools differ in layout, layers, dtype or device")
    lb, le = sp.layer_range(layer_begin, layer_end)
    s_ids = device_ids(src_ids, sp.device)
    d_ids = device_ids(dst_ids, dp.device, distinct=True)
    if s_ids.numel() != d_ids.numel():
        raise ValueError(f"{s_ids.numel()} source ids but {d_ids.numel()} destination ids")
    n = s_ids.numel()
    if n == 0 or le == lb:
        return
    _native.check(_native.load().pace_kv_move(
        sp.table(lb), sp.num_pages, s_ids.data_ptr(), dp.table(lb), dp.num_pages,
        d_ids.data_ptr(), le - lb, n, sp.page_bytes, _err_ptr(err), _stream_handle(sp.device)))


def _swap_args(dev: PagedPool, host: PagedPool, dev_ids: IdsLike, host_ids: IdsLike, into_host: bool):
    if not host.host or dev.host:
        raise ValueError("swap needs one device pool and one host pool")
    if dev.page_shape != host.page_shape or dev.dtype != host.dtype or dev.num_layers != host.num_layers:
        raise ValueError("device and host pools differ in layout, layers or dtype")
    d_ids = device_ids(dev_ids, dev.device, distinct=not into_host)
    h_ids = device_ids(host_ids, dev.device, distinct=into_host)
    if d_ids.numel() != h_ids.numel():
        raise ValueError(f"{d_ids.numel()} device ids but {h_ids.numel()} host ids")
    return d_ids, h_ids


def swap_out(dev_pool, dev_ids: IdsLike, host_pool: PagedPool, host_ids: IdsLike, *,
             err: Optional[torch.Tensor] = None) -> None:
    """host_pool.layers[l][host_ids[j]] = dev_pool.layers[l][dev_ids[j]], one
    kernel writing the pinned host pages across PCIe."""
    dev = as_pool(dev_pool)
    d_ids, h_ids = _swap_args(dev, host_pool, dev_ids, host_ids, into_host=True)
    n = d_ids.numel()
    if n == 0:
        return
    _native.check(_native.load().pace_kv_swap_out(
        dev.table(), dev.num_pages, d_ids.data_ptr(), host_pool.table(), host_pool.num_pages,
        h_ids.data_ptr(), dev.num_layers, n, dev.page_bytes, _err_ptr(err), _stream_handle(dev.device)))


def swap_in(host_pool: PagedPool, host_ids: IdsLike, dev_pool, dev_ids: IdsLike, *,
            err: Optional[torch.Tensor] = None) -> None:
    """dev_pool.layers[l][dev_ids[j]] = host_pool.layers[l][host_ids[j]], one
    kernel reading the pinned host pages across PCIe."""
    dev = as_pool(dev_pool)
    d_ids, h_ids = _swap_args(dev, host_pool, dev_ids, host_ids, into_host=False)
    n = d_ids.numel()
    if n == 0:
        return
    _native.check(_native.load().pace_kv_swap_in(
        host_pool.table(), host_pool.num_pages, h_ids.data_ptr(), dev.table(), dev.num_pages,
        d_ids.data_ptr(), dev.num_layers, n, dev.page_bytes, _err_ptr(err), _stream_handle(dev.device)))


class Promoter:
    """pace_kv_promoter: plans a batch on a NativeBlockAllocator, uploads both
    id lists with one copy and moves the pages, all in one library call."""

    def __init__(self, device: Optional[torch.device] = None):
        self.device = torch.device(device) if device is not None else torch.device(
            "cuda", torch.cuda.current_device())
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            _native.check(_native.load().pace_kv_promoter_create(ctypes.byref(handle)))
        self._handle = handle.value

    def promote(self, src, dst, allocator, src_ids, indptr, dst_pages=None,
                buffer: Optional[torch.Tensor] = None, err: Optional[torch.Tensor] = None):
        """Returns every request's destination table, concatenated (int32
        numpy array; request r owns dst_pages[r] entries)."""
        sp, dp = as_pool(src), as_pool(dst)
        if sp is not dp and (not sp.compatible(dp) or sp.num_layers != dp.num_layers):
            raise ValueError("source and destination pools differ in layout, layers, dtype or device")
        src_ids = np.ascontiguousarray(src_ids, dtype=np.int32)
        indptr = np.ascontiguousarray(indptr, dtype=np.int64)
        counts = None if dst_pages is None else np.ascontiguousarray(dst_pages, dtype=np.int32)
        buf_ptr, stride, blayers = None, 0, 0
        if buffer is not None:
            stride = _check_buffer(buffer, sp, 1, src_ids.size, "promote")
            buf_ptr, blayers = buffer.data_ptr(), int(buffer.shape[0])
        tables, total = self._launch(sp, dp, allocator, src_ids, indptr, counts, buf_ptr, stride, blayers, err,
                                     _stream_handle(sp.device))
        return np.frombuffer(tables, dtype=np.int32, count=total).copy()

    def _launch(self, sp: PagedPool, dp: PagedPool, allocator, src_ids, indptr, counts,
                buf_ptr: Optional[int], stride: int, blayers: int, err: Optional[torch.Tensor], stream: int,
                source_range_ok: bool = False):
        """The library call with arguments already checked.  src_ids (int32),
        indptr (int64) and counts (int32, or None) are contiguous numpy arrays
        or array.array objects; the buffer comes as pointer / layer stride /
        layers (or None, 0, 0).  Returns (array('i') of destination tables,
        their total).  With source_range_ok, a source id outside [0,
        num_pages) returns (None, 0) instead of raising (nothing was
        allocated): the caller normalises the ids and calls again."""
        if self._handle is None:
            raise RuntimeError("promoter is closed")
        n_req = len(indptr) - 1
        if counts is None:
            total = int(indptr[-1])
        else:
            total = int(counts.sum()) if isinstance(counts, np.ndarray) else sum(counts)
        tables = array("i", bytes(4 * max(total, 1)))
        rc = _native.load().pace_kv_promote(
            self._handle, allocator.handle, sp.table(), sp.num_pages, dp.table(), dp.num_pages,
            sp.num_layers, sp.page_bytes, n_req, _addr(indptr),
            _addr(src_ids) if len(src_ids) else None,
            None if counts is None else _addr(counts), buf_ptr, stride, blayers,
            tables.buffer_info()[0], _err_ptr(err), stream)
        if rc == _native.PACE_KV_ENOMEM:
            from ..core.block_manager import OOM_MESSAGE
            raise ValueError(OOM_MESSAGE)
        if rc == _native.PACE_KV_ERANGE and source_range_ok and \
                _native.load().pace_kv_last_error().startswith(b"source ids"):
            return None, 0
        _native.check(rc)
        return tables, total

    def close(self) -> None:
        if self._handle is not None:
            handle, self._handle = self._handle, None
            with torch.cuda.device(self.device):
                _native.check(_native.load().pace_kv_promoter_destroy(handle))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Stager:
    """Pinned-host staging pipeline (pace_kv_stager): device slot rings, side
    streams for the round trip's packs and unpacks, D2H copies and H2D copies,
    and the events that order them.

    Host tensors handed to a call are kept alive until the caller's stream has
    passed the point where the call's copies finish.  One host thread at a
    time may drive a stager.  Two slots are the minimum; three (the default,
    kv_utils.ROUNDTRIP_SLOTS) measured as fast as four."""

    def __init__(self, slot_bytes: int, num_slots: int = 3, device: Optional[torch.device] = None):
        self.device = torch.device(device) if device is not None else torch.device(
            "cuda", torch.cuda.current_device())
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            _native.check(_native.load().pace_kv_stager_create(int(slot_bytes), int(num_slots),
                                                               ctypes.byref(handle)))
        self._handle = handle.value
        self.slot_bytes = int(slot_bytes)
        self.num_slots = int(num_slots)
        self._inflight: list = []
        self._spare: list = []  # events of finished calls, recorded again

    def _keep(self, *objs) -> None:
        live = []
        for e, o in self._inflight:
            if e.query():
                self._spare.append(e)
            else:
                live.append((e, o))
        ev = self._spare.pop() if self._spare else torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        live.append((ev, objs))
        self._inflight = live

    def _require(self):
        if self._handle is None:
            raise RuntimeError("stager is closed")
        return self._handle

    @staticmethod
    def _host(t: torch.Tensor, pool: PagedPool, n_layers: int, n: int, what: str) -> None:
        if t.device.type != "cpu" or not t.is_contiguous() or t.dtype != pool.dtype:
            raise ValueError(f"{what}: host buffer must be a contiguous CPU tensor of {pool.dtype}")
        need = n_layers * n * pool.page_bytes
        if t.numel() * t.element_size() < need:
            raise ValueError(f"{what}: host buffer holds {t.numel() * t.element_size()} bytes, needs {need}")

    def pack_to_host(self, src, page_ids: IdsLike, host_out: torch.Tensor, layers_per_chunk: int,
                     *, layer_begin: int = 0, layer_end: Optional[int] = None,
                     err: Optional[torch.Tensor] = None) -> torch.Tensor:
        pool = as_pool(src)
        lb, le = pool.layer_range(layer_begin, layer_end)
        ids = device_ids(page_ids, pool.device)
        n = ids.numel()
        self._host(host_out, pool, le - lb, n, "pack_to_host")
        try:
            _native.check(_native.load().pace_kv_pack_to_host(
                self._require(), pool.table(lb), le - lb, pool.num_pages, ids.data_ptr() if n else None,
                n, pool.page_bytes, int(layers_per_chunk), host_out.data_ptr(), _err_ptr(err),
                _stream_handle(pool.device)))
        finally:  # a call failing part-way leaves copies in flight too
            self._keep(host_out, ids)
        return host_out

    def unpack_from_host(self, host_in: torch.Tensor, dst, page_ids: IdsLike, layers_per_chunk: int,
                         *, layer_begin: int = 0, layer_end: Optional[int] = None,
                         err: Optional[torch.Tensor] = None) -> None:
        pool = as_pool(dst)
        lb, le = pool.layer_range(layer_begin, layer_end)
        ids = device_ids(page_ids, pool.device, distinct=True)
        n = ids.numel()
        self._host(host_in, pool, le - lb, n, "unpack_from_host")
        try:
            _native.check(_native.load().pace_kv_unpack_from_host(
                self._require(), host_in.data_ptr(), pool.table(lb), le - lb, pool.num_pages,
                ids.data_ptr() if n else None, n, pool.page_bytes, int(layers_per_chunk), _err_ptr(err),
                _stream_handle(pool.device)))
        finally:
            self._keep(host_in, ids)

    def roundtrip(self, src, src_ids: IdsLike, dst, dst_ids: IdsLike, host_buf: torch.Tensor,
                  layers_per_chunk: int, *, err: Optional[torch.Tensor] = None) -> None:
        sp, dp = as_pool(src), as_pool(dst)
        if not sp.compatible(dp) or sp.num_layers != dp.num_layers:
            raise ValueError("source and destination pools differ in layout, layers, dtype or device")
        s_ids = device_ids(src_ids, sp.device)
        d_ids = device_ids(dst_ids, dp.device, distinct=True)
        if s_ids.numel() != d_ids.numel():
            raise ValueError(f"{s_ids.numel()} source ids but {d_ids.numel()} destination ids")
        n = s_ids.numel()
        if host_buf.device.type != "cpu" or not host_buf.is_contiguous():
            raise ValueError("roundtrip: host buffer must be a contiguous CPU tensor")
        try:
            _native.check(_native.load().pace_kv_roundtrip(
                self._require(), sp.table(), sp.num_pages, s_ids.data_ptr() if n else None, dp.table(),
                dp.num_pages, d_ids.data_ptr() if n else None, sp.num_layers, n, sp.page_bytes,
                int(layers_per_chunk), host_buf.data_ptr(), host_buf.numel() * host_buf.element_size(),
                _err_ptr(err), _stream_handle(sp.device)))
        finally:
            self._keep(host_buf, s_ids, d_ids)

    def close(self) -> None:
        if self._handle is not None:
            handle, self._handle = self._handle, None
            with torch.cuda.device(self.device):
                _native.check(_native.load().pace_kv_stager_destroy(handle))
            self._inflight.clear()
            self._spare.clear()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
