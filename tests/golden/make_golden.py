"""Writes the golden fixtures of the KV migration path (tests/golden/*.npz).

The expected outputs are computed here by element-by-element loops over
(layer, page, K/V, slot, head, dim) that restate the reference's semantics
directly, independently of oracle/kv_oracle.py, so that the fixtures can pin
the oracle:
  - pack:   out[l][j] = src[l][src_table[j]]      (paceserve/kv_transfer/kv_utils.py:44-46)
  - unpack: dst[l][dst_ids[j]] = buf[l][j]        (paceserve/kv_transfer/kv_utils.py:49-52)
  - dst_ids from the worker's LIFO allocation and the n / n+1 rule
    (paceserve/worker/base_worker.py:255-277,
     paceserve/core/block_space_manager/base_block_space_manager.py:29-39,89-97)
  - the zero-page fallback (paceserve/kv_transfer/kv_utils.py:34-42)
  - token t of a request sits at page t // P, slot t % P, K at index 0 and V at
    index 1 of the page (the layout asserted in examples/flashinfer_example.py:
    76-114: request lengths [3, 7], page_size 4, pages [0] and [1, 2]).

Values are raw 16-bit words (fp16 or bf16 bit patterns of N(0,1) samples);
the path copies bytes, so words are what the tests compare.

Run: python tests/golden/make_golden.py   (rewrites the .npz files)
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

L, H, D, P = 2, 2, 8, 4
POOL = 6


def words(rng: np.random.Generator, shape, kind: str) -> np.ndarray:
    x = rng.standard_normal(shape).astype(np.float32)
    if kind == "fp16":
        return x.astype(np.float16).view(np.uint16)
    # bf16: the upper half of the float32 bit pattern
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def brute_pack(src, table):
    n = len(table)
    out = np.zeros((L, n, 2, P, H, D), dtype=np.uint16)
    for l in range(L):
        for j in range(n):
            for kv in range(2):
                for s in range(P):
                    for h in range(H):
                        for d in range(D):
                            out[l, j, kv, s, h, d] = src[l][table[j], kv, s, h, d]
    return out


def brute_unpack(buf, dst, ids):
    res = [layer.copy() for layer in dst]
    for l in range(L):
        for j, pid in enumerate(ids):
            for kv in range(2):
                for s in range(P):
                    for h in range(H):
                        for d in range(D):
                            res[l][pid, kv, s, h, d] = buf[l, j, kv, s, h, d]
    return res


def lifo(free_list, n):
    free = list(free_list)
    got = []
    for _ in range(n):
        got.append(free[-1])
        free = free[:-1]
    return got, free


def case(name, kind, seed, src_table, dst_tokens, dst_free=None, indptr=None):
    """One migration: pack src_table, allocate ceil(dst_tokens/P) pages from the
    destination's free list, remap (n or n+1), unpack."""
    rng = np.random.default_rng(seed)
    src = words(rng, (L, POOL, 2, P, H, D), kind)
    dst = words(rng, (L, POOL, 2, P, H, D), kind)
    free = list(range(POOL)) if dst_free is None else list(dst_free)
    m = -(-dst_tokens // P)
    dst_table, free_after = lifo(free, m)
    n = len(src_table)
    if m == n:
        ids = dst_table
    elif m == n + 1:
        ids = dst_table[:-1]
    else:
        raise ValueError("fixture cases use the n or n+1 rule only")
    buf = brute_pack(src, src_table)
    dst_after = brute_unpack(buf, dst, ids)
    np.savez(HERE / f"case_{name}.npz", kind=np.array(kind), src=src, dst_before=dst,
             src_table=np.array(src_table, dtype=np.int32), dst_free=np.array(free, dtype=np.int32),
             dst_tokens=np.array(dst_tokens), dst_table=np.array(dst_table, dtype=np.int32),
             dst_ids=np.array(ids, dtype=np.int32), free_after=np.array(free_after, dtype=np.int32),
             packed=buf, dst_after=np.stack(dst_after),
             indptr=np.array(indptr if indptr is not None else [0, n], dtype=np.int32))


def flashinfer_layout():
    """Token placement of examples/flashinfer_example.py:76-114 (lengths [3, 7],
    page_size 4, pages [0] and [1, 2], one head): token t of request r is in page
    table_r[t // 4], slot t % 4; K at index 0, V at index 1."""
    rng = np.random.default_rng(7)
    lens = [3, 7]
    tables = [[0], [1, 2]]
    k = words(rng, (10, 1, 128), "fp16")
    v = words(rng, (10, 1, 128), "fp16")
    cache = np.zeros((3, 2, 4, 1, 128), dtype=np.uint16)
    tok = 0
    for r, n_tok in enumerate(lens):
        for t in range(n_tok):
            page = tables[r][t // 4]
            for d in range(128):
                cache[page, 0, t % 4, 0, d] = k[tok, 0, d]
                cache[page, 1, t % 4, 0, d] = v[tok, 0, d]
            tok += 1
    np.savez(HERE / "layout_flashinfer_example.npz", k=k, v=v, cache=cache,
             lens=np.array(lens), table0=np.array(tables[0], dtype=np.int32),
             table1=np.array(tables[1], dtype=np.int32))


def main():
    # 13 tokens -> 4 pages, last page 1 slot valid; src pages from a fragmented pool.
    case("fp16_partial", "fp16", 11, src_table=[4, 1, 5, 2], dst_tokens=13)
    # 8 prompt tokens + the first generated token: src 2 pages, dst 3 (n+1 rule).
    case("bf16_nplus1", "bf16", 12, src_table=[3, 0], dst_tokens=9)
    # Zero-page fallback inserted into a 1-page destination.
    rng = np.random.default_rng(13)
    dst = words(rng, (L, POOL, 2, P, H, D), "fp16")
    zeros = np.zeros((L, 1, 2, P, H, D), dtype=np.uint16)
    table, _ = lifo(range(POOL), 1)
    after = brute_unpack(zeros, dst, table)
    np.savez(HERE / "case_zero_fallback.npz", kind=np.array("fp16"), dst_before=dst,
             packed=zeros, src_table=np.array([0], dtype=np.int32),
             dst_ids=np.array(table, dtype=np.int32), dst_after=np.stack(after))
    # Two requests batched (CSR concatenation) into a destination whose free
    # list was fragmented by earlier frees.
    case("fp16_batch2", "fp16", 14, src_table=[5, 0, 3, 1, 2], dst_tokens=20,
         dst_free=[2, 0, 5, 1, 4, 3], indptr=[0, 3, 5])
    flashinfer_layout()


if __name__ == "__main__":
    main()
