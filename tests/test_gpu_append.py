"""Paged append on the HIP path (pace_kv_append, pace_kv_batch_indices_positions,
and pace_kv_append_indptr, which derives positions in the same launch) against
the reference's FlashInfer example and the oracle, and the producer ->
migration -> producer sequence a partially prefilled promotion needs."""
import numpy as np
import pytest
import torch

from oracle import kv_oracle as orc
from paceserve_amd.kv_transfer import append as ap
from paceserve_amd.kv_transfer import ops

pytestmark = pytest.mark.gpu

WORD = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32,
        torch.float8_e4m3fn: torch.uint8}


def words(t):
    return t.view(WORD[t.dtype])


def i32(x, dev):
    return torch.tensor(x, dtype=torch.int32, device=dev)


def test_flashinfer_example_known_answer(gpu):
    with np.load("tests/golden/layout_flashinfer_example.npz", allow_pickle=False) as z:
        k, v, want = z["k"], z["v"], z["cache"]
    kk = torch.from_numpy(k.astype(np.int16)).to(gpu).view(torch.float16)
    vv = torch.from_numpy(v.astype(np.int16)).to(gpu).view(torch.float16)
    cache = torch.zeros(3, 2, 4, 1, 128, dtype=torch.float16, device=gpu)
    kv_indptr, kv_indices, last = i32([0, 1, 3], gpu), i32([0, 1, 2], gpu), i32([3, 3], gpu)
    seq = ap.get_seq_lens(kv_indptr, last, 4)
    bi, pos = ap.get_batch_indices_positions(i32([0, 3, 10], gpu), seq, 10)
    assert seq.tolist() == [3, 7] and bi.tolist() == [0] * 3 + [1] * 7
    assert pos.tolist() == [0, 1, 2, 0, 1, 2, 3, 4, 5, 6]
    ap.append_paged_kv_cache(kk, vv, bi, pos, cache, kv_indices, kv_indptr, last)
    torch.cuda.synchronize()
    assert np.array_equal(words(cache).cpu().numpy().astype(np.uint16), want)
    fused = torch.zeros_like(cache)
    ap.append_paged_kv_cache_indptr(kk, vv, i32([0, 3, 10], gpu), fused, kv_indices, kv_indptr, last)
    torch.cuda.synchronize()
    assert np.array_equal(words(fused).cpu().numpy().astype(np.uint16), want)


# Rows of 2 KiB (two vectors per lane), 8 KiB (eight), 128 B and 32 B (part of
# one lane set), 1 KiB, 10 KiB (sixteen, guarded), 32 KiB and 24 KiB (two
# chunks of 16 KiB, the second guarded); R requests, more than one wave's 64
# for the fused form's request search.
@pytest.mark.parametrize("dtype,H,D,P,R", [
    (torch.bfloat16, 8, 128, 16, 6), (torch.float16, 32, 128, 16, 6), (torch.float16, 1, 64, 4, 6),
    (torch.float32, 4, 64, 16, 6), (torch.float8_e4m3fn, 8, 128, 16, 6), (torch.bfloat16, 2, 8, 16, 6),
    (torch.float16, 40, 128, 16, 5), (torch.bfloat16, 64, 256, 16, 4), (torch.bfloat16, 96, 128, 16, 3),
    (torch.bfloat16, 8, 128, 16, 130)])
def test_mixed_prefill_and_decode_batch_matches_oracle(gpu, dtype, H, D, P, R):
    print(f"append case {dtype} H={H} D={D} P={P} R={R}", flush=True)
    rng = np.random.default_rng(H * D + P + R)
    prior = rng.integers(0, 40, R)                 # tokens already in each request
    app = rng.integers(1, 25, R)                   # tokens appended now
    app[::2] = 1                                   # decode requests append one token
    if R > 6:
        app[3::7] = 0                              # requests appending nothing
    total = prior + app
    pages = -(-total // P)
    NP = int(pages.sum()) + 5
    perm = rng.permutation(NP)
    kv_indptr = np.concatenate([[0], np.cumsum(pages)])
    kv_indices = perm[: kv_indptr[-1]]
    last = np.where(total % P == 0, P, total % P)
    append_indptr = np.concatenate([[0], np.cumsum(app)])
    nnz = int(append_indptr[-1])
    wt = WORD[dtype]
    # int8 words of each tensor, copied into a fresh tensor so that an empty
    # batch (no new tokens) still has the strides a dtype view needs
    raw = lambda shape: torch.empty(shape, dtype=torch.int8, device=gpu).copy_(
        torch.from_numpy(rng.integers(-2 ** 7, 2 ** 7, shape).astype(np.int8)))
    k = raw((nnz, H, D * torch.empty(0, dtype=dtype).element_size())).view(dtype).view(nnz, H, D)
    v = raw((nnz, H, D * torch.empty(0, dtype=dtype).element_size())).view(dtype).view(nnz, H, D)
    cache = raw((NP, 2, P, H, D * torch.empty(0, dtype=dtype).element_size())).view(dtype).view(NP, 2, P, H, D)
    want = orc.append_paged_kv_cache(
        words(k).cpu().numpy(), words(v).cpu().numpy(),
        *orc.get_batch_indices_positions(append_indptr, orc.get_seq_lens(kv_indptr, last, P), nnz),
        words(cache).cpu().numpy(), kv_indices, kv_indptr, P)
    fused = cache.clone()
    seq = ap.get_seq_lens(i32(kv_indptr, gpu), i32(last, gpu), P)
    bi, pos = ap.get_batch_indices_positions(i32(append_indptr, gpu), seq, nnz)
    ap.append_paged_kv_cache(k, v, bi, pos, cache, i32(kv_indices, gpu), i32(kv_indptr, gpu), i32(last, gpu))
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    ap.append_paged_kv_cache_indptr(k, v, i32(append_indptr, gpu), fused, i32(kv_indices, gpu), i32(kv_indptr, gpu),
                                    i32(last, gpu), err=err)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(words(cache).cpu().numpy(), want)
    np.testing.assert_array_equal(words(fused).cpu().numpy(), want)
    assert int(err.item()) == 0


def test_out_of_range_tokens_are_skipped_and_counted(gpu):
    cache = torch.zeros(4, 2, 4, 1, 64, dtype=torch.float16, device=gpu)
    k = torch.ones(4, 1, 64, dtype=torch.float16, device=gpu)
    kv_indptr, kv_indices = i32([0, 1, 2], gpu), i32([3, 7], gpu)     # page 7 does not exist
    bi = i32([0, 1, 5, 0], gpu)          # request 5 does not exist
    pos = i32([1, 0, 0, 4], gpu)         # position 4 is past request 0's single page
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    ap.append_paged_kv_cache(k, k, bi, pos, cache, kv_indices, kv_indptr, i32([2, 1], gpu), err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 3
    assert (cache[3, :, 1] == 1).all() and int((cache != 0).sum()) == 2 * 64


def test_fused_append_skips_and_counts_tokens_out_of_range(gpu):
    """Tokens past the last request's offsets, a request whose last-page
    length puts its tokens before position 0, and a page id past the cache
    are skipped and counted once per token; the other tokens land."""
    cache = torch.zeros(4, 2, 4, 1, 64, dtype=torch.float16, device=gpu)
    k = torch.ones(6, 1, 64, dtype=torch.float16, device=gpu)
    # request 0: 2 tokens into page 3 (one page, last_len 2: positions 0, 1)
    # request 1: 2 tokens with last_len 1 on one page -> positions -1, 0
    # request 2: 1 token into page 9 (past the cache)
    # tokens 5: beyond append_indptr[-1]
    ai = i32([0, 2, 4, 5], gpu)
    kv_indptr, kv_indices, last = i32([0, 1, 2, 3], gpu), i32([3, 1, 9], gpu), i32([2, 1, 1], gpu)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    ap.append_paged_kv_cache_indptr(k, k, ai, cache, kv_indices, kv_indptr, last, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 3                    # request 1's first token, request 2's, token 5
    assert (cache[3, :, :2] == 1).all() and (cache[1, :, 0] == 1).all()
    assert int((cache != 0).sum()) == 3 * 2 * 64


def test_partially_prefilled_request_promoted_then_continued(gpu):
    """Chunk 1 of a prompt is appended into the low-priority pool, the request
    is promoted (pages moved to the high-priority pool), chunk 2 is appended
    there: the result equals appending the whole prompt on the high-priority
    pool directly."""
    L, H, D, P, NP = 3, 8, 128, 16, 64
    rng = np.random.default_rng(9)
    n1, n2 = 37, 50
    k = torch.randn(L, n1 + n2, H, D, device=gpu).to(torch.bfloat16)
    v = torch.randn(L, n1 + n2, H, D, device=gpu).to(torch.bfloat16)
    lp = [torch.zeros(NP, 2, P, H, D, dtype=torch.bfloat16, device=gpu) for _ in range(L)]
    hp = [torch.zeros(NP, 2, P, H, D, dtype=torch.bfloat16, device=gpu) for _ in range(L)]
    ref = [torch.zeros(NP, 2, P, H, D, dtype=torch.bfloat16, device=gpu) for _ in range(L)]

    def append(pool, l, table, done, k_new, v_new):
        total = done + k_new.shape[0]
        pages = -(-total // P)
        ip = i32([0, pages], gpu)
        last = i32([total % P or P], gpu)
        seq = ap.get_seq_lens(ip, last, P)
        bi, pos = ap.get_batch_indices_positions(i32([0, k_new.shape[0]], gpu), seq, k_new.shape[0])
        ap.append_paged_kv_cache(k_new, v_new, bi, pos, pool[l], i32(table[:pages], gpu), ip, last)

    lp_table = rng.permutation(NP)[:6].tolist()         # room for 87 tokens
    for l in range(L):
        append(lp, l, lp_table, 0, k[l, :n1], v[l, :n1])
    n_lp = -(-n1 // P)
    hp_table = rng.permutation(NP)[:6].tolist()
    ops.move(lp, lp_table[:n_lp], hp, hp_table[:n_lp])   # promotion of the prefilled pages
    for l in range(L):
        append(hp, l, hp_table, n1, k[l, n1:], v[l, n1:])
        append(ref, l, hp_table, 0, k[l], v[l])
    torch.cuda.synchronize()
    for l in range(L):
        assert torch.equal(words(hp[l]), words(ref[l])), f"layer {l}"


def test_append_of_70000_tokens(gpu):
    # 70 000 tokens of two requests (one prefill, one continued) in one launch
    # of 140 000 workgroups.
    P, H, D, pages = 16, 1, 8, 5000
    g = torch.Generator(device=gpu).manual_seed(31)
    cache = torch.randn((pages, 2, P, H, D), generator=g, device=gpu).half()
    seq_lens = [60000, 10005]                 # request 1 already held 5 tokens
    new = [60000, 10000]
    npages = [-(-n // P) for n in seq_lens]
    kv_indptr = i32([0, npages[0], npages[0] + npages[1]], gpu)
    kv_indices = torch.randperm(pages, generator=torch.Generator().manual_seed(32))[:sum(npages)].to(torch.int32).to(gpu)
    last = i32([n - (k - 1) * P for n, k in zip(seq_lens, npages)], gpu)
    append_indptr = i32([0, new[0], new[0] + new[1]], gpu)
    nnz = sum(new)
    key = torch.randn((nnz, H, D), generator=g, device=gpu).half()
    value = torch.randn((nnz, H, D), generator=g, device=gpu).half()
    bi, pos = ap.get_batch_indices_positions(append_indptr, ap.get_seq_lens(kv_indptr, last, P), nnz)
    before = cache.clone()
    ap.append_paged_kv_cache(key, value, bi, pos, cache, kv_indices, kv_indptr, last)
    torch.cuda.synchronize()
    b_l, p_l = bi.long(), pos.long()
    page_t = kv_indices.long()[kv_indptr.long()[b_l] + p_l // P]
    assert torch.equal(words(cache[page_t, 0, p_l % P]), words(key))
    assert torch.equal(words(cache[page_t, 1, p_l % P]), words(value))
    # the 5 tokens request 1 held before the append are untouched
    first = kv_indices.long()[npages[0]]
    assert torch.equal(words(cache[first, :, :5]), words(before[first, :, :5]))


@pytest.mark.parametrize("seed", list(range(6)) + [283])   # seed 283: one request, no new tokens
def test_random_appends_match_numpy(gpu, seed):
    """Seeded random batches through both forms: 1-1000 requests (the fused
    form's request search takes more than one round of 256 past 256
    requests), prior lengths 0-99, 0-40 new tokens per request, random row
    shapes and element types.  Expected: every appended row placed by numpy at
    kv_indices[kv_indptr[b] + pos // P], slot pos % P, pos counted from the end
    of the request's tokens; every other slot unchanged."""
    rng = np.random.default_rng(7000 + seed)
    R = int(rng.choice([1, 7, 64, 257, 600, 1000]))
    P = int(rng.choice([1, 4, 16]))
    H, D = int(rng.choice([1, 2, 8])), int(rng.choice([16, 64, 128]))
    dtype = [torch.float16, torch.bfloat16, torch.float32, torch.float8_e4m3fn][int(rng.integers(0, 4))]
    esz = torch.empty(0, dtype=dtype).element_size()
    prior = rng.integers(0, 100, R)
    app = rng.integers(0, 41, R)
    total = prior + app
    pages = -(-total // P)
    NP = int(pages.sum()) + 3
    kv_indptr = np.concatenate([[0], np.cumsum(pages)])
    kv_indices = rng.permutation(NP)[: kv_indptr[-1]]
    last = np.where(total == 0, 0, np.where(total % P == 0, P, total % P))
    append_indptr = np.concatenate([[0], np.cumsum(app)])
    nnz = int(append_indptr[-1])
    print(f"random append seed {seed}: R={R} P={P} H={H} D={D} {dtype} nnz={nnz} pages={NP}", flush=True)
    # int8 words of each tensor, copied into a fresh tensor so that an empty
    # batch (no new tokens) still has the strides a dtype view needs
    raw = lambda shape: torch.empty(shape, dtype=torch.int8, device=gpu).copy_(
        torch.from_numpy(rng.integers(-2 ** 7, 2 ** 7, shape).astype(np.int8)))
    k = raw((nnz, H, D * esz)).view(dtype).view(nnz, H, D)
    v = raw((nnz, H, D * esz)).view(dtype).view(nnz, H, D)
    cache = raw((NP, 2, P, H, D * esz)).view(dtype).view(NP, 2, P, H, D)
    # numpy placement of every appended token
    want = words(cache).cpu().numpy().copy()
    kw, vw = words(k).cpu().numpy(), words(v).cpu().numpy()
    b = np.repeat(np.arange(R), app)
    pos = total[b] - app[b] + (np.arange(nnz) - append_indptr[b])
    page = kv_indices[kv_indptr[b] + pos // P]
    want[page, 0, pos % P] = kw
    want[page, 1, pos % P] = vw
    two = cache.clone()
    seq = ap.get_seq_lens(i32(kv_indptr, gpu), i32(last, gpu), P)
    bi, ps = ap.get_batch_indices_positions(i32(append_indptr, gpu), seq, nnz)
    ap.append_paged_kv_cache(k, v, bi, ps, two, i32(kv_indices, gpu), i32(kv_indptr, gpu), i32(last, gpu))
    fused = cache.clone()
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    ap.append_paged_kv_cache_indptr(k, v, i32(append_indptr, gpu), fused, i32(kv_indices, gpu),
                                    i32(kv_indptr, gpu), i32(last, gpu), err=err)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(words(two).cpu().numpy(), want)
    np.testing.assert_array_equal(words(fused).cpu().numpy(), want)
    assert int(err.item()) == 0


@pytest.mark.parametrize("pattern", ["one-each", "uneven", "sparse"])
@pytest.mark.parametrize("R", [7, 300])
def test_decode_shaped_batches_match_numpy(gpu, pattern, R):
    """Batches with no more tokens than requests, where the fused form first
    tries request i for token i: one token per request (every guess right),
    as many tokens as requests but spread 0/1/2 (some guesses wrong), and
    fewer tokens than requests; 7 and 300 requests (the fallback search then
    takes two rounds).  Both forms place every row where numpy does and leave
    every other slot unchanged."""
    rng = np.random.default_rng({"one-each": 1, "uneven": 2, "sparse": 3}[pattern] * 1000 + R)
    P, H, D, dtype = 16, 8, 128, torch.bfloat16
    if pattern == "one-each":
        app = np.ones(R, dtype=np.int64)
    elif pattern == "uneven":
        app = rng.permutation(np.resize([0, 1, 2], R))       # sums to about R
        app[-1] += R - int(app.sum())                         # exactly R tokens
        assert app.min() >= 0
    else:
        app = (rng.random(R) < 0.6).astype(np.int64)          # 0 or 1, fewer tokens than requests
    prior = rng.integers(0, 70, R)
    total = prior + app
    pages = -(-total // P)
    NP = int(pages.sum()) + 3
    kv_indptr = np.concatenate([[0], np.cumsum(pages)])
    kv_indices = rng.permutation(NP)[: kv_indptr[-1]]
    last = np.where(total == 0, 0, np.where(total % P == 0, P, total % P))
    append_indptr = np.concatenate([[0], np.cumsum(app)])
    nnz = int(append_indptr[-1])
    assert nnz <= R
    print(f"decode-shaped append {pattern} R={R} nnz={nnz}", flush=True)
    raw = lambda shape: torch.empty(shape, dtype=torch.int8, device=gpu).copy_(
        torch.from_numpy(rng.integers(-2 ** 7, 2 ** 7, shape).astype(np.int8)))
    k = raw((nnz, H, D * 2)).view(dtype).view(nnz, H, D)
    v = raw((nnz, H, D * 2)).view(dtype).view(nnz, H, D)
    cache = raw((NP, 2, P, H, D * 2)).view(dtype).view(NP, 2, P, H, D)
    want = words(cache).cpu().numpy().copy()
    b = np.repeat(np.arange(R), app)
    pos = total[b] - app[b] + (np.arange(nnz) - append_indptr[b])
    page = kv_indices[kv_indptr[b] + pos // P]
    want[page, 0, pos % P] = words(k).cpu().numpy()
    want[page, 1, pos % P] = words(v).cpu().numpy()
    two = cache.clone()
    seq = ap.get_seq_lens(i32(kv_indptr, gpu), i32(last, gpu), P)
    bi, ps = ap.get_batch_indices_positions(i32(append_indptr, gpu), seq, nnz)
    ap.append_paged_kv_cache(k, v, bi, ps, two, i32(kv_indices, gpu), i32(kv_indptr, gpu), i32(last, gpu))
    fused = cache.clone()
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    ap.append_paged_kv_cache_indptr(k, v, i32(append_indptr, gpu), fused, i32(kv_indices, gpu),
                                    i32(kv_indptr, gpu), i32(last, gpu), err=err)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(words(two).cpu().numpy(), want)
    np.testing.assert_array_equal(words(fused).cpu().numpy(), want)
    assert int(err.item()) == 0


def test_fused_decode_batch_skips_and_counts_tokens_out_of_range(gpu):
    """The same rules when the fused form first tries request i for token i
    (5 tokens, 5 requests): request 1's last-page length puts its token
    before position 0, request 2's page id is past the cache, request 4
    appends nothing so token 4 is beyond the last request's offsets; those
    three are skipped and counted, requests 0 and 3 land."""
    cache = torch.zeros(4, 2, 4, 1, 64, dtype=torch.float16, device=gpu)
    k = torch.ones(5, 1, 64, dtype=torch.float16, device=gpu)
    ai = i32([0, 1, 2, 3, 4, 4], gpu)
    kv_indptr, kv_indices, last = i32([0, 1, 2, 3, 4, 5], gpu), i32([3, 1, 9, 2, 0], gpu), i32([1, 0, 1, 3, 1], gpu)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    ap.append_paged_kv_cache_indptr(k, k, ai, cache, kv_indices, kv_indptr, last, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 3
    assert (cache[3, :, 0] == 1).all() and (cache[2, :, 2] == 1).all()
    assert int((cache != 0).sum()) == 2 * 2 * 64
