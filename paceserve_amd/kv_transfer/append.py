"""Paged KV append on the HIP path: the producer of the pages the migration
path moves.

Drop-in for the three FlashInfer calls of the reference's attention wrapper
(paceserve/model_executor/attention/flashinfer_attention_wrapper.py:241-255):
get_seq_lens, get_batch_indices_positions and append_paged_kv_cache, with the
same arguments and the NHD layout [num_pages, 2, page_size, H, D] per layer.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import _native
from .ops import _err_ptr, _stream_handle


def _i32(t: torch.Tensor, name: str, device: torch.device) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or t.dim() != 1:
        raise ValueError(f"{name} must be a 1-D tensor")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, the cache on {device}")
    if t.dtype is torch.int32 and t.is_contiguous():
        return t
    return t.to(torch.int32).contiguous()


def get_seq_lens(kv_indptr: torch.Tensor, kv_last_page_len: torch.Tensor, page_size: int) -> torch.Tensor:
    """max(pages - 1, 0) * page_size + last_page_len per request (int32)."""
    pages = kv_indptr[1:] - kv_indptr[:-1]
    return (torch.clamp(pages - 1, min=0) * page_size + kv_last_page_len).to(torch.int32)


def get_batch_indices_positions(append_indptr: torch.Tensor, seq_lens: torch.Tensor,
                                nnz: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Request index and sequence position of each appended token (HIP)."""
    dev = append_indptr.device
    ai = _i32(append_indptr, "append_indptr", dev)
    sl = _i32(seq_lens, "seq_lens", dev)
    batch = ai.numel() - 1
    if sl.numel() != batch:
        raise ValueError(f"{sl.numel()} sequence lengths for {batch} requests")
    bi = torch.empty(nnz, dtype=torch.int32, device=dev)
    pos = torch.empty(nnz, dtype=torch.int32, device=dev)
    if nnz:
        _native.check(_native.load().pace_kv_batch_indices_positions(
            ai.data_ptr(), sl.data_ptr(), batch, nnz, bi.data_ptr(), pos.data_ptr(), _stream_handle(dev)))
    return bi, pos


def _check_append(append_key: torch.Tensor, append_value: torch.Tensor, paged_kv_cache: torch.Tensor,
                  kv_layout: str):
    """Validates the key/value rows and the cache; returns (P, H, D)."""
    if kv_layout != "NHD":
        raise ValueError("only the NHD layout [num_pages, 2, page_size, H, D] is supported")
    cache = paged_kv_cache
    if cache.dim() != 5 or cache.shape[1] != 2 or not cache.is_contiguous() or cache.device.type != "cuda":
        raise ValueError("paged_kv_cache must be a contiguous device tensor [num_pages, 2, P, H, D]")
    _, _, P, H, D = cache.shape
    dev, dtype = cache.device, cache.dtype
    for name, t in (("append_key", append_key), ("append_value", append_value)):
        if t.dim() != 3 or t.shape[1] != H or t.shape[2] != D or t.dtype != dtype or t.device != dev:
            raise ValueError(f"{name} must be [nnz, {H}, {D}] {dtype} on {dev}")
        if t.stride(2) != 1 or t.stride(1) != D:
            raise ValueError(f"{name} rows must be contiguous [H, D] blocks")
    if append_key.shape[0] != append_value.shape[0] or append_key.stride(0) != append_value.stride(0):
        raise ValueError("append_key and append_value differ in length or token stride")
    return P, H, D


def append_paged_kv_cache(append_key: torch.Tensor, append_value: torch.Tensor,
                          batch_indices: torch.Tensor, positions: torch.Tensor,
                          paged_kv_cache: torch.Tensor, kv_indices: torch.Tensor,
                          kv_indptr: torch.Tensor, kv_last_page_len: torch.Tensor,
                          kv_layout: str = "NHD", err: Optional[torch.Tensor] = None) -> None:
    """Writes append_key[i] / append_value[i] ([nnz, H, D]) into
    paged_kv_cache[kv_indices[kv_indptr[b] + pos // P], 0 / 1, pos % P]."""
    P, H, D = _check_append(append_key, append_value, paged_kv_cache, kv_layout)
    cache = paged_kv_cache
    dev = cache.device
    nnz = append_key.shape[0]
    bi = _i32(batch_indices, "batch_indices", dev)
    pos = _i32(positions, "positions", dev)
    idx = _i32(kv_indices, "kv_indices", dev)
    ip = _i32(kv_indptr, "kv_indptr", dev)
    _i32(kv_last_page_len, "kv_last_page_len", dev)
    if bi.numel() < nnz or pos.numel() < nnz:
        raise ValueError("batch_indices and positions need one entry per appended token")
    if nnz == 0:
        return
    elem = cache.element_size()
    _native.check(_native.load().pace_kv_append(
        append_key.data_ptr(), append_value.data_ptr(), append_key.stride(0) * elem, nnz,
        bi.data_ptr(), pos.data_ptr(), ip.numel() - 1, cache.data_ptr(), cache.shape[0],
        idx.data_ptr(), idx.numel(), ip.data_ptr(), P, H * D * elem, _err_ptr(err),
        _stream_handle(dev)))


def append_paged_kv_cache_indptr(append_key: torch.Tensor, append_value: torch.Tensor,
                                 append_indptr: torch.Tensor, paged_kv_cache: torch.Tensor,
                                 kv_indices: torch.Tensor, kv_indptr: torch.Tensor,
                                 kv_last_page_len: torch.Tensor, kv_layout: str = "NHD",
                                 err: Optional[torch.Tensor] = None) -> None:
    """get_seq_lens + get_batch_indices_positions + append_paged_kv_cache in
    one launch: each token's request and position come from append_indptr
    (the request offsets of the appended tokens), kv_indptr and
    kv_last_page_len, as the reference computes them for every layer
    (paceserve/model_executor/attention/flashinfer_attention_wrapper.py:241-255)."""
    P, H, D = _check_append(append_key, append_value, paged_kv_cache, kv_layout)
    cache = paged_kv_cache
    dev = cache.device
    nnz = append_key.shape[0]
    ai = _i32(append_indptr, "append_indptr", dev)
    idx = _i32(kv_indices, "kv_indices", dev)
    ip = _i32(kv_indptr, "kv_indptr", dev)
    last = _i32(kv_last_page_len, "kv_last_page_len", dev)
    batch = ai.numel() - 1
    if ip.numel() != batch + 1 or last.numel() != batch:
        raise ValueError(f"kv_indptr needs {batch + 1} entries and kv_last_page_len {batch} "
                         f"for {batch} requests")
    if nnz == 0:
        return
    elem = cache.element_size()
    _native.check(_native.load().pace_kv_append_indptr(
        append_key.data_ptr(), append_value.data_ptr(), append_key.stride(0) * elem, nnz, ai.data_ptr(),
        batch, cache.data_ptr(), cache.shape[0], idx.data_ptr(), idx.numel(), ip.data_ptr(), last.data_ptr(),
        P, H * D * elem, _err_ptr(err), _stream_handle(dev)))
