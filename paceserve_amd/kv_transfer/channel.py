"""Cross-process KV channel over libpace_kv (pace_kv_channel_*).

The reference hands a finished prefill from one instance process to another
by returning a KVobj, whose host tensor Ray pickles through its object store
(paceserve/disutil/prefill_instance.py:96-107 transfer_kv_cache;
paceserve/disutil/decode_instance.py:165-171 ray.get and insert;
paceserve/core/datatypes/kv_cache_obj.py:7-21 KVobj).  A KVChannel carries
the pages instead through a named shared-memory ring: the sending process
packs them straight out of its device pool into the ring, the receiving
process unpacks them straight into its own, and only a small KVref (the
KVobj's fields without the tensor) needs to cross the control plane.

One process creates the channel, the other opens it by name; one side sends,
the other receives.  A message larger than the ring streams through it, so
the receiver must be receiving while the sender sends (in the reference's
pull model the decode side asks for a sequence and then receives it).
"""
from __future__ import annotations

import contextlib
import ctypes
import json
import threading
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

from .. import _native
from . import ops

MiB = 1 << 20


@dataclass
class MessageHeader:
    """A received message's header: its id, metadata and payload shape."""
    msg_id: int
    meta: bytes
    num_layers: int
    n_pages: int
    page_bytes: int

    @property
    def payload_bytes(self) -> int:
        return self.num_layers * self.n_pages * self.page_bytes


def _ms(timeout: float) -> int:
    return max(0, min(int(timeout * 1000), 2**31 - 1))


# Most page ids a send or receive passes in host memory: the library carries
# them in each launch's kernel arguments, so no upload precedes the copies.
HOST_IDS_MAX = 512


def _ids(page_ids: ops.IdsLike, device: torch.device, distinct: bool = False):
    """The page ids as the library takes them: a device tensor is used as it
    is; host data of at most HOST_IDS_MAX ids becomes an int32 numpy array
    (range-checked by the kernels, like device ids); longer host data is
    uploaded (ops.device_ids).  distinct=True rejects repeated host ids."""
    if isinstance(page_ids, torch.Tensor):
        if page_ids.device.type == "cuda" or page_ids.numel() > HOST_IDS_MAX:
            return ops.device_ids(page_ids, device, distinct)
        arr = page_ids.to(torch.int32).contiguous().view(-1).numpy()
    else:
        if len(page_ids) > HOST_IDS_MAX:
            return ops.device_ids(page_ids, device, distinct)
        try:
            arr = np.ascontiguousarray(page_ids, dtype=np.int32).reshape(-1)
        except OverflowError as e:
            raise ValueError("page ids outside the int32 range") from e
    if distinct and arr.size > 1:
        u, c = np.unique(arr, return_counts=True)
        if (c > 1).any():
            raise ValueError(f"destination page {int(u[c > 1][0])} appears more than once; destination page "
                             "ids must be distinct")
    return arr


def _count(ids) -> int:
    return int(ids.numel()) if isinstance(ids, torch.Tensor) else int(ids.size)


def _ptr(ids) -> int:
    return ids.data_ptr() if isinstance(ids, torch.Tensor) else ids.ctypes.data


class KVChannel:
    """One endpoint of a channel (create() on one side, open() on the other).

    Messages arrive in the order they were sent, and a message is received in
    two calls (recv_header, then recv / recv_host / discard).  Threads that
    share an endpoint take whole messages with message(), which holds the
    endpoint's receive lock from the header to the end of the payload;
    threads that each pull their own sequences take a channel each."""

    def __init__(self, handle: int, name: str):
        self._handle = handle
        self.name = name
        slot = ctypes.c_int64()
        slots = ctypes.c_int()
        _native.check(_native.load().pace_kv_channel_info(handle, ctypes.byref(slot), ctypes.byref(slots)))
        self.slot_bytes = slot.value
        self.num_slots = slots.value
        self._header: Optional[MessageHeader] = None
        self._inflight: list = []
        self._rx_lock = threading.Lock()

    @classmethod
    def create(cls, name: str, slot_bytes: int = 32 * MiB, num_slots: int = 4,
               copy_threads: int = 4, device_slot_bytes: int = 0) -> "KVChannel":
        """Creates the ring (num_slots: a power of two in [2, 64]; slot_bytes:
        a multiple of 4096) and returns the creating endpoint.  With
        device_slot_bytes > 0 (a multiple of 4096, at most 1 GiB over all
        slots) it also allocates a ring of device slots on the current GPU,
        through which sends made on that GPU pass without leaving HBM."""
        handle = ctypes.c_void_p()
        lib = _native.load()
        if device_slot_bytes:
            _native.check(lib.pace_kv_channel_create_device(name.encode(), int(slot_bytes), int(num_slots),
                                                            int(copy_threads), int(device_slot_bytes),
                                                            ctypes.byref(handle)))
        else:
            _native.check(lib.pace_kv_channel_create(name.encode(), int(slot_bytes), int(num_slots),
                                                     int(copy_threads), ctypes.byref(handle)))
        return cls(handle.value, name)

    def device_ring(self):
        """(device slot bytes, 0 when the channel has no device ring; whether
        the ring is on the current GPU, so that sends from here use it)."""
        dsb = ctypes.c_int64()
        here = ctypes.c_int()
        _native.check(_native.load().pace_kv_channel_device_info(self._require(), ctypes.byref(dsb),
                                                                 ctypes.byref(here)))
        return dsb.value, bool(here.value)

    @classmethod
    def open(cls, name: str, copy_threads: int = 4, timeout: float = 30.0) -> "KVChannel":
        handle = ctypes.c_void_p()
        _native.check(_native.load().pace_kv_channel_open(name.encode(), int(copy_threads), _ms(timeout),
                                                          ctypes.byref(handle)))
        return cls(handle.value, name)

    @staticmethod
    def unlink(name: str) -> None:
        """Removes a channel name left behind by a creator that died without
        closing it (open endpoints keep working)."""
        _native.check(_native.load().pace_kv_channel_unlink(name.encode()))

    def _require(self) -> int:
        if self._handle is None:
            raise RuntimeError(f"channel {self.name} is closed")
        return self._handle

    # ------------------------------------------------------------- sending

    def send(self, src, page_ids: ops.IdsLike, meta: bytes = b"", timeout: float = 60.0) -> int:
        """Sends pool pages src[l][page_ids[j]] as one message; returns its id.
        Packs run on the current stream after its earlier work; the call
        returns when the whole payload is in the ring."""
        pool = ops.as_pool(src)
        ids = _ids(page_ids, pool.device)
        n = _count(ids)
        out = ctypes.c_uint64()
        meta = bytes(meta)
        with torch.cuda.device(pool.device):
            _native.check(_native.load().pace_kv_channel_send(
                self._require(), pool.table(), pool.num_layers, pool.num_pages, _ptr(ids) if n else None,
                n, pool.page_bytes, meta, len(meta), _ms(timeout), ctypes.byref(out),
                ops._stream_handle(pool.device)))
        return out.value

    def send_host(self, payload: torch.Tensor, meta: bytes = b"", timeout: float = 60.0) -> int:
        """Sends a host payload [L, n, *page_shape] (a KVobj's kv_cache) as one
        message; returns its id."""
        if payload.device.type != "cpu" or not payload.is_contiguous() or payload.dim() < 3:
            raise ValueError("send_host: payload must be a contiguous CPU tensor [L, n, *page_shape]")
        L, n = int(payload.shape[0]), int(payload.shape[1])
        page_bytes = int(payload[0, 0].numel()) * payload.element_size() if L and n else 16
        out = ctypes.c_uint64()
        meta = bytes(meta)
        _native.check(_native.load().pace_kv_channel_send_host(
            self._require(), payload.data_ptr() if L and n else None, L, n, page_bytes, meta, len(meta),
            _ms(timeout), ctypes.byref(out)))
        return out.value

    # ----------------------------------------------------------- receiving

    def recv_header(self, timeout: float = 60.0) -> MessageHeader:
        """Waits for the next message and returns its header; its payload
        must be received (recv / recv_host / discard) before the next one."""
        lib = self._require()
        cap = 64 << 10
        while True:
            buf = ctypes.create_string_buffer(cap)
            meta_len = ctypes.c_int64()
            layers = ctypes.c_int()
            n = ctypes.c_int64()
            pb = ctypes.c_int64()
            msg = ctypes.c_uint64()
            rc = _native.load().pace_kv_channel_recv_header(
                lib, buf, cap, ctypes.byref(meta_len), ctypes.byref(layers), ctypes.byref(n), ctypes.byref(pb),
                ctypes.byref(msg), _ms(timeout))
            if rc == _native.PACE_KV_ERANGE and meta_len.value > cap:
                cap = meta_len.value
                continue
            _native.check(rc)
            h = MessageHeader(msg.value, buf.raw[:meta_len.value], layers.value, n.value, pb.value)
            self._header = h if h.payload_bytes else None
            return h

    @contextlib.contextmanager
    def message(self, timeout: float = 60.0):
        """Receives the next message's header under the endpoint's receive
        lock and yields it; the body receives the payload (recv / recv_host),
        and a payload left unreceived is drained on exit, so that several
        threads can take whole messages from one endpoint."""
        with self._rx_lock:
            h = self.recv_header(timeout)
            try:
                yield h
            finally:
                if self._header is not None:
                    self.discard(timeout)

    def recv(self, dst, page_ids: ops.IdsLike, timeout: float = 60.0,
             err: Optional[torch.Tensor] = None) -> None:
        """Receives the current message's payload into pool pages
        dst[l][page_ids[j]] (distinct ids).  Unpacks run on the current
        stream; the last ones are still enqueued when the call returns."""
        h = self._current()
        pool = ops.as_pool(dst)
        ids = _ids(page_ids, pool.device, distinct=True)
        n = _count(ids)
        if (pool.num_layers, n, pool.page_bytes) != (h.num_layers, h.n_pages, h.page_bytes):
            raise ValueError(f"message {h.msg_id} holds {h.num_layers} layers x {h.n_pages} pages x "
                             f"{h.page_bytes} B; the destination is {pool.num_layers} x {n} x {pool.page_bytes} B")
        with torch.cuda.device(pool.device):
            _native.check(_native.load().pace_kv_channel_recv(
                self._require(), pool.table(), pool.num_layers, pool.num_pages, _ptr(ids), n,
                pool.page_bytes, ops._err_ptr(err), _ms(timeout), ops._stream_handle(pool.device)))
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(pool.device))
        self._inflight = [(e, o) for e, o in self._inflight if not e.query()]
        self._inflight.append((ev, ids))
        self._header = None

    def recv_host(self, out: torch.Tensor, timeout: float = 60.0) -> torch.Tensor:
        """Receives the current message's payload into a contiguous CPU tensor
        of exactly the payload's size; returns it."""
        h = self._current()
        if out.device.type != "cpu" or not out.is_contiguous():
            raise ValueError("recv_host: out must be a contiguous CPU tensor")
        size = out.numel() * out.element_size()
        _native.check(_native.load().pace_kv_channel_recv_host(self._require(), out.data_ptr(), size, _ms(timeout)))
        self._header = None
        return out

    def discard(self, timeout: float = 60.0) -> None:
        """Drains the current message's payload without keeping it.  A message
        whose receive the library already gave up (the sender abandoned it, or
        a device step failed) has nothing left to drain: its leftover chunks
        are skipped before the next header.  Other failures (a timeout) keep
        the message pending, so that the drain can be retried."""
        if self._header is None:
            return
        rc = _native.load().pace_kv_channel_recv_host(self._require(), None, 0, _ms(timeout))
        if rc != _native.PACE_KV_ESTATE:
            _native.check(rc)
        self._header = None

    def _current(self) -> MessageHeader:
        if self._header is None:
            raise RuntimeError(f"channel {self.name}: no message payload pending (call recv_header first)")
        return self._header

    # ------------------------------------------------------------- closing

    def close(self) -> None:
        if self._handle is not None:
            handle, self._handle = self._handle, None
            _native.check(_native.load().pace_kv_channel_close(handle))
            self._inflight.clear()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class KVref:
    """What crosses the control plane in place of a KVobj: the KVobj's fields
    (paceserve/core/datatypes/kv_cache_obj.py:7-21) without the tensor, plus
    the id of the channel message that carries the pages."""
    seq_id: object
    kv_indices: List[int]
    size: float                     # MB, as KVobj.size
    left_prefill: Optional[float] = None
    kv_transfer_start: Optional[float] = None
    msg_id: int = 0

    def meta(self) -> bytes:
        return json.dumps({"seq_id": self.seq_id, "kv_indices": list(self.kv_indices), "size": self.size,
                           "left_prefill": self.left_prefill,
                           "kv_transfer_start": self.kv_transfer_start}).encode()

    @classmethod
    def from_header(cls, h: MessageHeader) -> "KVref":
        d = json.loads(h.meta.decode())
        return cls(d["seq_id"], d["kv_indices"], d["size"], d.get("left_prefill"), d.get("kv_transfer_start"),
                   h.msg_id)


def kv_size_mb(num_layers: int, n_pages: int, page_bytes: int) -> float:
    """KVobj.size for a payload of this shape (bytes / 1e6)."""
    return num_layers * n_pages * page_bytes / 10**6


def page_ids_of(ids: Sequence[int]) -> List[int]:
    return [int(i) for i in ids]
