"""Pins the CPU oracle (oracle/kv_oracle.py) before its answers are trusted.

Checks: the committed golden fixtures (written by element-by-element loops in
tests/golden/make_golden.py), the library routines the reference's indexing
reduces to (torch.index_select / Tensor.index_copy_ for unique ids, numpy
take), invariants of the copy, and closed forms of the allocator.  A set of
deliberately wrong oracles (each a plausible slip: layers and pages
transposed, K and V swapped, partial last page truncated, source and
destination tables swapped, extra page overwritten) must fail the fixtures.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import kv_oracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = ["fp16_partial", "bf16_nplus1", "fp16_batch2"]


def load(name):
    with np.load(GOLDEN / f"case_{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", CASES)
def test_pack_matches_golden(name):
    c = load(name)
    got = orc.pack(list(c["src"]), c["src_table"].tolist())
    assert got.dtype == np.uint16
    np.testing.assert_array_equal(got, c["packed"])


@pytest.mark.parametrize("name", CASES)
def test_allocation_and_remap_match_golden(name):
    c = load(name)
    alloc = orc.BlockAllocator(len(c["dst_free"]), c["dst_free"].tolist())
    table = orc.allocate_table(alloc, orc.pages_for_tokens(int(c["dst_tokens"]), 4))
    assert table == c["dst_table"].tolist()
    assert alloc.free_blocks == c["free_after"].tolist()
    assert orc.remap_dst_table(table, len(c["src_table"])) == c["dst_ids"].tolist()


@pytest.mark.parametrize("name", CASES)
def test_unpack_matches_golden(name):
    c = load(name)
    got = orc.unpack(c["packed"], list(c["dst_before"]), c["dst_ids"].tolist())
    np.testing.assert_array_equal(np.stack(got), c["dst_after"])


def test_zero_fallback_matches_golden():
    c = load("zero_fallback")
    zeros, ids = orc.zero_page_fallback(2, c["packed"].shape[2:], np.uint16)
    assert ids == [0]
    np.testing.assert_array_equal(zeros, c["packed"])
    got = orc.unpack(zeros, list(c["dst_before"]), c["dst_ids"].tolist())
    np.testing.assert_array_equal(np.stack(got), c["dst_after"])


def test_batch_request_slices_equal_single_requests():
    c = load("fp16_batch2")
    ip = c["indptr"].tolist()
    src = list(c["src"])
    table = c["src_table"].tolist()
    for r in range(len(ip) - 1):
        single = orc.pack(src, table[ip[r]:ip[r + 1]])
        np.testing.assert_array_equal(c["packed"][:, ip[r]:ip[r + 1]], single)


def test_flashinfer_layout_known_answer():
    """examples/flashinfer_example.py:107,114 asserts K of request 0's tokens
    0..2 in page 0 slots 0..2 and request 1's tokens in pages 1, 2; packing a
    request's pages therefore yields its tokens in order at [:, j, 0, slot]."""
    with np.load(GOLDEN / "layout_flashinfer_example.npz", allow_pickle=False) as z:
        k, v, cache = z["k"], z["v"], z["cache"]
        t0, t1 = z["table0"].tolist(), z["table1"].tolist()
    packed = orc.pack([cache], t1)[0]          # request 1: 7 tokens in 2 pages
    k_tokens = packed[:, 0].reshape(-1, 1, 128)[:7]
    v_tokens = packed[:, 1].reshape(-1, 1, 128)[:7]
    np.testing.assert_array_equal(k_tokens, k[3:10])
    np.testing.assert_array_equal(v_tokens, v[3:10])
    packed0 = orc.pack([cache], t0)[0]
    np.testing.assert_array_equal(packed0[0, 0, :3], k[0:3])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_oracle_equals_torch_index_routines(dtype):
    g = torch.Generator().manual_seed(3)
    L, N = 3, 17
    src = [torch.randn(N, 2, 4, 2, 8, generator=g).to(dtype) for _ in range(L)]
    dst = [torch.randn(N, 2, 4, 2, 8, generator=g).to(dtype) for _ in range(L)]
    s_ids = torch.randperm(N, generator=g)[:9]
    d_ids = torch.randperm(N, generator=g)[:9]
    ref_buf = torch.stack([torch.index_select(s, 0, s_ids) for s in src])
    ref_dst = [d.clone().index_copy_(0, d_ids, ref_buf[i]) for i, d in enumerate(dst)]
    wv = torch.int16 if dtype != torch.float32 else torch.int32
    np_src = [s.view(wv).numpy() for s in src]
    np_dst = [d.view(wv).numpy() for d in dst]
    buf = orc.pack(np_src, s_ids.tolist())
    np.testing.assert_array_equal(buf, ref_buf.view(wv).numpy())
    out = orc.unpack(buf, np_dst, d_ids.tolist())
    for a, b in zip(out, ref_dst):
        np.testing.assert_array_equal(a, b.view(wv).numpy())
    # the timed CPU baseline path computes the same bytes
    dst2 = [d.clone() for d in dst]
    buf2 = orc.torch_cpu_pack_unpack(src, s_ids, dst2, d_ids)
    assert torch.equal(buf2.view(wv), ref_buf.view(wv))
    for a, b in zip(dst2, ref_dst):
        assert torch.equal(a.view(wv), b.view(wv))


def test_copy_invariants():
    rng = np.random.default_rng(5)
    src = [rng.integers(0, 2 ** 16, (20, 2, 4, 1, 8), dtype=np.uint16) for _ in range(2)]
    dst = [rng.integers(0, 2 ** 16, (20, 2, 4, 1, 8), dtype=np.uint16) for _ in range(2)]
    s_ids = rng.permutation(20)[:7].tolist()
    d_ids = rng.permutation(20)[:7].tolist()
    src_before = [s.copy() for s in src]
    out = orc.move(src, s_ids, dst, d_ids)
    for l in range(2):
        np.testing.assert_array_equal(src[l], src_before[l])      # source never written
        untouched = sorted(set(range(20)) - set(d_ids))
        np.testing.assert_array_equal(out[l][untouched], dst[l][untouched])
        np.testing.assert_array_equal(out[l][d_ids], src[l][s_ids])
    # unpack(pack) at the same ids restores the pages
    back = orc.unpack(orc.pack(src, s_ids), [np.zeros_like(s) for s in src], s_ids)
    for l in range(2):
        np.testing.assert_array_equal(back[l][s_ids], src[l][s_ids])


def test_repeated_destination_pages_keep_last_write():
    layer = np.zeros((4, 2, 1, 1, 1), dtype=np.uint16)
    buf = np.arange(3 * 2, dtype=np.uint16).reshape(1, 3, 2, 1, 1, 1) + 1
    out = orc.unpack(buf, [layer], [2, 0, 2])
    np.testing.assert_array_equal(out[0][2], buf[0, 2])
    np.testing.assert_array_equal(out[0][0], buf[0, 1])
    # torch's CPU index_put_ (sequential) agrees
    t = torch.zeros(4, 2, 1, 1, 1, dtype=torch.int16)
    t[torch.tensor([2, 0, 2])] = torch.from_numpy(buf[0].astype(np.int16))
    np.testing.assert_array_equal(out[0].astype(np.int16), t.numpy())


def test_negative_and_out_of_range_ids_follow_torch_indexing():
    layer = np.arange(5 * 2, dtype=np.uint16).reshape(5, 2, 1, 1, 1)
    np.testing.assert_array_equal(orc.pack([layer], [-1])[0, 0], layer[4])
    with pytest.raises(IndexError):
        orc.pack([layer], [5])
    with pytest.raises(IndexError):
        orc.pack([layer], [-6])


# ------------------------------------------------------------ allocator


def test_fresh_allocator_hands_out_descending_pages():
    a = orc.BlockAllocator(10)
    assert orc.allocate_table(a, 4) == [9, 8, 7, 6]
    assert a.num_free() == 6


def test_free_then_allocate_returns_freed_pages_lifo():
    a = orc.BlockAllocator(8)
    t = orc.allocate_table(a, 3)                 # [7, 6, 5]
    orc.free_table(a, t + [t[0]])                # repeats freed once
    assert a.num_free() == 8
    assert orc.allocate_table(a, 3) == list(reversed(t))


def test_exhaustion_raises_reference_message():
    a = orc.BlockAllocator(2)
    orc.allocate_table(a, 2)
    with pytest.raises(ValueError, match="Out of memory! No free blocks are available."):
        a.allocate()


def test_remap_rule_cases():
    assert orc.remap_dst_table([5, 4, 3], 3) == [5, 4, 3]
    assert orc.remap_dst_table([5, 4, 3, 2], 3) == [5, 4, 3]
    assert orc.remap_dst_table([5, 4, 3, 2, 1], 3) is None
    assert orc.remap_dst_table([5, 4], 3) is None


@pytest.mark.parametrize("tokens", [1, 15, 16, 17, 4095, 4096, 32768])
def test_pages_for_tokens_brute_force(tokens):
    P = 16
    pages, fill = 0, P
    for _ in range(tokens):          # fill slots one token at a time
        if fill == P:
            pages, fill = pages + 1, 0
        fill += 1
    assert orc.pages_for_tokens(tokens, P) == pages
    assert orc.last_page_len(tokens, P) == fill


# ------------------------------------------------------ planted mistakes


def _bad_transposed(layers, ids):
    good = orc.pack(layers, ids)
    return good.reshape(good.shape[1], good.shape[0], *good.shape[2:]).copy()


def _bad_kv_swapped(layers, ids):
    return orc.pack(layers, ids)[:, :, ::-1].copy()


def _bad_partial_page(layers, ids):
    out = orc.pack(layers, ids)
    out[:, -1, :, 1:] = 0            # only the first slot of the last page
    return out


def _bad_off_by_one(layers, ids):
    return orc.pack(layers, [(i + 1) % layers[0].shape[0] for i in ids])


@pytest.mark.parametrize("bad", [_bad_transposed, _bad_kv_swapped, _bad_partial_page, _bad_off_by_one])
def test_planted_pack_mistakes_fail_the_fixtures(bad):
    c = load("fp16_partial")
    got = bad(list(c["src"]), c["src_table"].tolist())
    assert got.shape != c["packed"].shape or not np.array_equal(got, c["packed"])


def test_planted_unpack_mistakes_fail_the_fixtures():
    c = load("bf16_nplus1")
    # using the full n+1 table writes into the page that must stay untouched
    wrong_ids = c["dst_table"].tolist()
    buf = np.concatenate([c["packed"], c["packed"][:, :1]], axis=1)
    got = orc.unpack(buf, list(c["dst_before"]), wrong_ids)
    assert not np.array_equal(np.stack(got), c["dst_after"])
    # swapping source and destination tables
    c2 = load("fp16_partial")
    got2 = orc.unpack(c2["packed"], list(c2["dst_before"]), c2["src_table"].tolist())
    assert not np.array_equal(np.stack(got2), c2["dst_after"])


# ------------------------------------------------------------ paged append


def flashinfer_example():
    with np.load(GOLDEN / "layout_flashinfer_example.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_append_oracle_reproduces_flashinfer_example():
    """examples/flashinfer_example.py:76-114: lengths [3, 7], page_size 4,
    page indptr [0, 1, 3], indices [0, 1, 2], last page lengths [3, 3]."""
    z = flashinfer_example()
    kv_indptr, kv_indices, last = [0, 1, 3], [0, 1, 2], [3, 3]
    seq = orc.get_seq_lens(kv_indptr, last, 4)
    assert seq.tolist() == [3, 7]
    bi, pos = orc.get_batch_indices_positions([0, 3, 10], seq, 10)
    assert bi.tolist() == [0] * 3 + [1] * 7
    assert pos.tolist() == [0, 1, 2, 0, 1, 2, 3, 4, 5, 6]
    cache = np.zeros((3, 2, 4, 1, 128), dtype=np.uint16)
    got = orc.append_paged_kv_cache(z["k"], z["v"], bi, pos, cache, kv_indices, kv_indptr, 4)
    np.testing.assert_array_equal(got, z["cache"])


@pytest.mark.parametrize("chunks", [[10], [1] * 10, [4, 3, 3], [7, 1, 1, 1]])
def test_append_in_chunks_equals_append_at_once(chunks):
    rng = np.random.default_rng(sum(chunks) * len(chunks))
    P, pages = 4, [5, 2, 7]
    k = rng.integers(0, 2 ** 16, (10, 2, 8), dtype=np.uint16)
    v = rng.integers(0, 2 ** 16, (10, 2, 8), dtype=np.uint16)
    cache0 = rng.integers(0, 2 ** 16, (8, 2, P, 2, 8), dtype=np.uint16)
    once_bi, once_pos = orc.get_batch_indices_positions([0, 10], [10], 10)
    once = orc.append_paged_kv_cache(k, v, once_bi, once_pos, cache0, pages, [0, 3], P)
    cache, done = cache0, 0
    for c in chunks:                      # the sequence grows chunk by chunk
        total = done + c
        n_pages = -(-total // P)
        seq = orc.get_seq_lens([0, n_pages], [total % P or P], P)
        bi, pos = orc.get_batch_indices_positions([0, c], seq, c)
        cache = orc.append_paged_kv_cache(k[done:total], v[done:total], bi, pos, cache, pages, [0, n_pages], P)
        done = total
    np.testing.assert_array_equal(cache, once)
