"""Seeded synthetic migration workloads at the reference's KV shapes.

Each workload fixes the cache shape, the source/destination pool sizes, the
request lengths and how the source pool's free list is fragmented, so that the
benchmark and the tests build identical source block tables and pages:

  llama3-8b-512tok-fp16      Llama-3-8B KV (32 layers, 8 KV heads, head_dim
                             128, page 16), fp16: one 512-token request (32
                             pages) at seeded random pages of a 2048-page pool,
                             values N(0,1).  Seed 1001.
  llama3-8b-16req-bf16       same shape, bf16: 16 requests, lengths
                             lognormal(median 1024, sigma 1.0) clipped to
                             [128, 8192]; 16384-page pools; the source free
                             list is a seeded permutation; separate fresh
                             destination pool.  Seed 1002.
  llama2-7b-8x4095tok-fp16   Llama-2-7B KV (32 KV heads), fp16: 8 requests of
                             4095 tokens (256 pages each, last page 15/16
                             full); 4096-page pools, permuted; migrated through
                             pinned host memory, one layer per chunk.  Seed 1003.
  llama3-8b-32768tok-bf16    Llama-3-8B KV, bf16, values uniform[-4, 4]: one
                             32768-token request filling a 2048-page pool in
                             permuted order; on-device and pinned-host
                             variants.  Seed 1004.
  llama3-70b-256req-bf16     Llama-3-70B KV (80 layers, 8 KV heads), bf16: 256
                             requests of U{64..2048} tokens; 20480-page pools;
                             a seeded permutation of the source pool dealt to
                             requests round-robin one page at a time; moved in
                             8-layer chunks.  Seed 1005.
  llama3-8b-4096tok-bf16     Llama-3-8B KV, bf16: one 4096-token request (256
                             pages) in a 2048-page pool (the promote-latency
                             workload).  Seed 1100.
  llama3-70b-256req-bf16-tp8 one GPU's share of llama3-70b-256req-bf16 under
                             tensor parallelism 8: the same requests and block
                             tables, with the 8 KV heads split one per GPU, so
                             each page is 8 KiB (2 x 16 x 1 x 128 x 2 B);
                             moved in 40-layer chunks.  Seed 1005.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Iterable, Iterator, List, Optional, Sequence

import numpy as np
import torch


@dataclass(frozen=True)
class KVShape:
    num_layers: int
    num_kv_heads: int
    head_dim: int
    page_size: int
    dtype: torch.dtype

    @property
    def page_shape(self):
        return (2, self.page_size, self.num_kv_heads, self.head_dim)

    @property
    def dtype_name(self) -> str:
        return str(self.dtype).replace("torch.", "")

    @property
    def page_bytes(self) -> int:
        return 2 * self.page_size * self.num_kv_heads * self.head_dim * torch.empty(0, dtype=self.dtype).element_size()


@dataclass
class Workload:
    name: str
    description: str
    shape: KVShape
    src_pool_pages: int
    dst_pool_pages: int
    lengths: List[int]
    src_tables: List[List[int]]
    seed: int
    init: str = "normal"             # "normal" = N(0,1), "uniform4" = U[-4, 4]
    staging: str = "device"          # "device", "pinned" or "both"
    layers_per_chunk: Optional[int] = None         # host-leg (staging) chunk
    device_layers_per_chunk: Optional[int] = None  # transfer-buffer chunk on device
    dst_free: Optional[List[int]] = None
    notes: dict = field(default_factory=dict)

    @property
    def n_pages(self) -> int:
        return sum(len(t) for t in self.src_tables)

    @property
    def payload_bytes(self) -> int:
        return self.shape.num_layers * self.n_pages * self.shape.page_bytes

    # The source pool is drawn from `seed`, the destination pool from seed + 50.
    def src_pool(self, device) -> List[torch.Tensor]:
        return fill_pool(self.src_pool_pages, self.shape, self.seed, self.init, device)

    def dst_pool(self, device) -> List[torch.Tensor]:
        return fill_pool(self.dst_pool_pages, self.shape, self.seed + DST_SEED_OFFSET, self.init, device)

    def src_before(self, device) -> Iterator[torch.Tensor]:
        """src_pool's layers, regenerated one at a time (pool_layers)."""
        return pool_layers(self.src_pool_pages, self.shape, self.seed, self.init, device)

    def dst_before(self, device) -> Iterator[torch.Tensor]:
        """dst_pool's layers, regenerated one at a time (pool_layers)."""
        return pool_layers(self.dst_pool_pages, self.shape, self.seed + DST_SEED_OFFSET, self.init, device)

    def summary(self) -> dict:
        return {
            "workload": self.name,
            "description": self.description,
            "layers": self.shape.num_layers,
            "kv_heads": self.shape.num_kv_heads,
            "head_dim": self.shape.head_dim,
            "page_size": self.shape.page_size,
            "cache_dtype": str(self.shape.dtype).replace("torch.", ""),
            "requests": len(self.src_tables),
            "pages": self.n_pages,
            "src_pool_pages": self.src_pool_pages,
            "dst_pool_pages": self.dst_pool_pages,
            "payload_bytes": self.payload_bytes,
            "seed": self.seed,
        }


DST_SEED_OFFSET = 50
LLAMA3_8B = dict(num_layers=32, num_kv_heads=8, head_dim=128, page_size=16)


def _pages(tokens: int, page_size: int) -> int:
    return -(-tokens // page_size)


def _lifo_tables(free_list: List[int], lengths: List[int], page_size: int) -> List[List[int]]:
    """Requests allocate in order, each popping its pages from the end of the
    free list (the reference allocator's order)."""
    free = list(free_list)
    tables = []
    for n_tok in lengths:
        n = _pages(n_tok, page_size)
        if n > len(free):
            raise ValueError("pool too small for the workload")
        got = free[-n:]
        del free[-n:]
        got.reverse()
        tables.append(got)
    return tables


# The migration workloads, smallest first.  The default benchmark workload is
# the largest one that fits one GPU: 256 requests at the Llama-3-70B KV shape.
NAMES = ("llama3-8b-512tok-fp16", "llama3-8b-16req-bf16", "llama2-7b-8x4095tok-fp16",
         "llama3-8b-32768tok-bf16", "llama3-70b-256req-bf16")
DEFAULT = "llama3-70b-256req-bf16"
PROMOTE = "llama3-8b-4096tok-bf16"
# One GPU's share of a sharded migration, at its real shape (each GPU of a
# tensor-parallel group moves its own head slice of the same pages).
SHARDS = ("llama3-70b-256req-bf16-tp8",)


def get(name: str) -> Workload:
    """The workload called `name` (one of NAMES or PROMOTE)."""
    if name == "llama3-8b-512tok-fp16":
        seed = 1001
        rng = np.random.default_rng(seed)
        shape = KVShape(**LLAMA3_8B, dtype=torch.float16)
        lengths = [512]
        tables = [rng.permutation(2048)[:32].tolist()]
        return Workload(name, "1 x 512-token request, Llama-3-8B KV, fp16, 2048-page pool",
                        shape, 2048, 2048, lengths, tables, seed)
    if name == "llama3-8b-16req-bf16":
        seed = 1002
        rng = np.random.default_rng(seed)
        shape = KVShape(**LLAMA3_8B, dtype=torch.bfloat16)
        raw = rng.lognormal(mean=np.log(1024.0), sigma=1.0, size=16)
        lengths = np.clip(np.rint(raw), 128, 8192).astype(int).tolist()
        free = rng.permutation(16384).tolist()
        tables = _lifo_tables(free, lengths, 16)
        return Workload(name, "16 requests, lognormal(median 1024, sigma 1.0) tokens clipped "
                        "[128, 8192], Llama-3-8B KV, bf16, 16384-page pools, fragmented source free list",
                        shape, 16384, 16384, lengths, tables, seed)
    if name == "llama2-7b-8x4095tok-fp16":
        seed = 1003
        rng = np.random.default_rng(seed)
        shape = KVShape(num_layers=32, num_kv_heads=32, head_dim=128, page_size=16, dtype=torch.float16)
        lengths = [4095] * 8
        free = rng.permutation(4096).tolist()
        tables = _lifo_tables(free, lengths, 16)
        return Workload(name, "8 x 4095-token requests (partial last page), Llama-2-7B KV, fp16, "
                        "4096-page pools, pinned-host round trip per layer",
                        shape, 4096, 4096, lengths, tables, seed, staging="pinned", layers_per_chunk=1)
    if name == "llama3-8b-32768tok-bf16":
        seed = 1004
        rng = np.random.default_rng(seed)
        shape = KVShape(**LLAMA3_8B, dtype=torch.bfloat16)
        lengths = [32768]
        tables = [rng.permutation(2048).tolist()]
        return Workload(name, "1 x 32768-token request, Llama-3-8B KV, bf16, values U[-4,4], "
                        "2048-page pool in permuted order, on-device and pinned-host",
                        shape, 2048, 2048, lengths, tables, seed, init="uniform4", staging="both")
    if name in ("llama3-70b-256req-bf16", "llama3-70b-256req-bf16-tp8"):
        tp8 = name.endswith("-tp8")
        seed = 1005
        rng = np.random.default_rng(seed)
        shape = KVShape(num_layers=80, num_kv_heads=1 if tp8 else 8, head_dim=128, page_size=16,
                        dtype=torch.bfloat16)
        lengths = rng.integers(64, 2049, size=256).tolist()
        need = [_pages(n, 16) for n in lengths]
        perm = rng.permutation(20480).tolist()
        tables: List[List[int]] = [[] for _ in lengths]
        k = 0
        while any(len(t) < n for t, n in zip(tables, need)):
            for r in range(len(lengths)):
                if len(tables[r]) < need[r]:
                    tables[r].append(perm[k])
                    k += 1
        if tp8:
            return Workload(name, "one GPU's share at tensor parallelism 8 of 256 requests U{64..2048} tokens, "
                            "Llama-3-70B KV (80 layers, 1 of 8 KV heads: 8 KiB pages), bf16, 20480-page pools "
                            "dealt round-robin (heavily fragmented), 40-layer chunks",
                            shape, 20480, 20480, lengths, tables, seed, device_layers_per_chunk=40)
        return Workload(name, "256 requests U{64..2048} tokens, Llama-3-70B KV (80 layers), bf16, "
                        "20480-page pools dealt round-robin (heavily fragmented), 8-layer chunks",
                        shape, 20480, 20480, lengths, tables, seed, device_layers_per_chunk=8)
    if name == PROMOTE:
        seed = 1100
        rng = np.random.default_rng(seed)
        shape = KVShape(**LLAMA3_8B, dtype=torch.bfloat16)
        lengths = [4096]
        tables = [rng.permutation(2048)[:256].tolist()]
        return Workload(name, "1 x 4096-token request, Llama-3-8B KV, bf16, 2048-page pools",
                        shape, 2048, 2048, lengths, tables, seed)
    raise ValueError(f"unknown workload {name!r} (known: {', '.join(NAMES + SHARDS + (PROMOTE,))})")


def _fill_layer(t: torch.Tensor, g: torch.Generator, init: str) -> None:
    if init == "normal":
        t.normal_(generator=g)
    elif init == "uniform4":
        t.uniform_(-4.0, 4.0, generator=g)
    else:
        raise ValueError(init)


def fill_pool(layers_pages: int, shape: KVShape, seed: int, init: str, device) -> List[torch.Tensor]:
    """Per-layer pool tensors with seeded values (generated on `device`)."""
    g = torch.Generator(device=device).manual_seed(seed)
    out = []
    for _ in range(shape.num_layers):
        t = torch.empty((layers_pages,) + shape.page_shape, dtype=shape.dtype, device=device)
        _fill_layer(t, g, init)
        out.append(t)
    return out


def pool_layers(layers_pages: int, shape: KVShape, seed: int, init: str, device) -> Iterator[torch.Tensor]:
    """The layers fill_pool(layers_pages, shape, seed, init, device) returns,
    regenerated one at a time into one reused tensor: the same generator
    draws in the same order give the same values, so a pool's content before
    a migration can be rebuilt layer by layer without a second pool's memory."""
    g = torch.Generator(device=device).manual_seed(seed)
    t = torch.empty((layers_pages,) + shape.page_shape, dtype=shape.dtype, device=device)
    for _ in range(shape.num_layers):
        _fill_layer(t, g, init)
        yield t


def migration_mismatch(src_layers: Sequence[torch.Tensor], dst_layers: Sequence[torch.Tensor],
                       src_ids: torch.Tensor, dst_ids: torch.Tensor,
                       dst_before: Iterable[torch.Tensor],
                       src_before: Optional[Iterable[torch.Tensor]] = None) -> Optional[str]:
    """Exact whole-layer check of a migration, compared as raw bytes.

    For every layer l the destination must equal its content before the
    migration (dst_before, an iterable of layers; it is modified) with the
    source's selected pages put in by torch's own indexing,
        before.index_copy_(0, dst_ids, src_layers[l].index_select(0, src_ids)),
    which is the reference's gather then scatter (paceserve/kv_transfer/
    kv_utils.py:44-46,51-52), so a page written twice, swapped, missed or
    written where no id points fails.  With src_before the source layers must
    also equal their content before.  Returns None, or a message naming the
    first layer and the first pages that differ."""
    si, di = src_ids.long(), dst_ids.long()
    befores = [dst_before] + ([src_before] if src_before is not None else [])
    for l, olds in enumerate(zip(*befores)):
        if l >= len(dst_layers):
            break
        want = olds[0]
        want.index_copy_(0, di, src_layers[l].index_select(0, si))
        checks = [("destination", dst_layers[l], want)]
        if src_before is not None:
            checks.append(("source", src_layers[l], olds[1]))
        for what, got, exp in checks:
            a, b = got.view(torch.uint8), exp.view(torch.uint8)
            if not torch.equal(a, b):
                bad = (a != b).reshape(a.shape[0], -1).any(1).nonzero().flatten()[:4].tolist()
                return f"layer {l}: {what} pages {bad} differ"
    return None
