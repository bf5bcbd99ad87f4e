"""Wire containers of a migrated request's KV cache.

Mirror paceserve/core/datatypes/kv_cache_obj.py:7-31: KVobj carries the packed
pages [L, n, 2, P, H, D] (on the host after get_kv_cache), the *source* page
ids, and size in MB (bytes / 1e6); KVmetadata announces a transfer.
"""
from __future__ import annotations

from typing import List, Optional


class KVobj:
    def __init__(self, seq_id, kv_cache, kv_indices: List[int], left_prefill=None,
                 kv_transfer_start: Optional[float] = None):
        self.seq_id = seq_id
        self.kv_cache = kv_cache
        self.kv_indices = kv_indices
        self.size = (kv_cache.element_size() * kv_cache.numel()) / (10 ** 6)
        self.left_prefill = left_prefill
        self.kv_transfer_start = kv_transfer_start


class KVmetadata:
    def __init__(self, seq, kv_size: int):
        self.seq = seq
        self.kv_size = kv_size
        self.start_time = 0
        self._prefill_instance = None
        self._transfer_ref = None
