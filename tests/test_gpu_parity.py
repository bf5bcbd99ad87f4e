"""Parity of the HIP path (libpace_kv.so through its C ABI) with the oracle,
the golden fixtures and torch's own device gather/scatter.  Bit-exact: the
path copies bytes, so every comparison is on raw integer words."""
import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import kv_oracle as orc
from paceserve_amd import _native, workloads
from paceserve_amd.kv_transfer import ops

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"

WORD = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32,
        torch.float8_e4m3fn: torch.uint8, torch.uint8: torch.uint8}


def words(t):
    return t.view(WORD[t.dtype])


def same(a, b):
    return a.shape == b.shape and torch.equal(words(a), words(b))


def load(name):
    with np.load(GOLDEN / f"case_{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def to_dev(arr, kind, gpu):
    dt = torch.float16 if kind == "fp16" else torch.bfloat16
    return torch.from_numpy(arr.astype(np.int16)).to(gpu).view(dt)


def rand_pool(L, pages, shape, dtype, gpu, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    if dtype in (torch.float16, torch.bfloat16, torch.float32):
        return [torch.randn((pages,) + shape, generator=g, device=gpu, dtype=torch.float32).to(dtype)
                for _ in range(L)]
    return [torch.randint(0, 256, (pages,) + shape, generator=g, device=gpu, dtype=torch.uint8).view(dtype)
            for _ in range(L)]


@pytest.mark.parametrize("name", ["fp16_partial", "bf16_nplus1", "fp16_batch2"])
def test_golden_cases(gpu, name):
    c = load(name)
    kind = str(c["kind"])
    src = [to_dev(s, kind, gpu) for s in c["src"]]
    dst = [to_dev(d, kind, gpu) for d in c["dst_before"]]
    buf = ops.pack(src, c["src_table"].tolist())
    torch.cuda.synchronize()
    assert np.array_equal(words(buf).cpu().numpy().astype(np.uint16), c["packed"])
    ops.unpack(buf, dst, c["dst_ids"].tolist())
    torch.cuda.synchronize()
    got = np.stack([words(d).cpu().numpy().astype(np.uint16) for d in dst])
    assert np.array_equal(got, c["dst_after"])
    # fused move leaves the same destination bytes
    dst2 = [to_dev(d, kind, gpu) for d in c["dst_before"]]
    ops.move(src, c["src_table"].tolist(), dst2, c["dst_ids"].tolist())
    torch.cuda.synchronize()
    got2 = np.stack([words(d).cpu().numpy().astype(np.uint16) for d in dst2])
    assert np.array_equal(got2, c["dst_after"])


def test_zero_fallback_insert(gpu):
    c = load("zero_fallback")
    dst = [to_dev(d, "fp16", gpu) for d in c["dst_before"]]
    ops.unpack(to_dev(c["packed"], "fp16", gpu), dst, c["dst_ids"].tolist())
    torch.cuda.synchronize()
    got = np.stack([words(d).cpu().numpy().astype(np.uint16) for d in dst])
    assert np.array_equal(got, c["dst_after"])


SHAPES = [
    # (L, pool pages, page shape [2, P, H, D], dtype, n)
    (1, 8, (2, 16, 8, 128), torch.float16, 3),
    (3, 40, (2, 16, 8, 128), torch.bfloat16, 17),
    (32, 64, (2, 16, 8, 128), torch.float16, 32),
    (2, 16, (2, 16, 32, 128), torch.float16, 9),     # Llama-2-7B page (256 KiB)
    (4, 33, (2, 16, 1, 128), torch.bfloat16, 20),    # TP=8 slice: 8 KiB page
    (3, 12, (2, 16, 4, 64), torch.float32, 7),       # 32 KiB page, fp32
    (2, 20, (2, 16, 8, 128), torch.float8_e4m3fn, 11),  # fp8 page (32 KiB)
    (2, 9, (2, 4, 2, 8), torch.float16, 5),          # 256 B page: guarded kernel
    (2, 9, (2, 3, 1, 8), torch.bfloat16, 6),         # 96 B page: guarded kernel
    (80, 10, (2, 16, 1, 64), torch.bfloat16, 6),     # > 64 layers: two launches
]


@pytest.mark.parametrize("L,pages,shape,dtype,n", SHAPES)
def test_pack_unpack_move_match_torch_and_oracle(gpu, L, pages, shape, dtype, n):
    src = rand_pool(L, pages, shape, dtype, gpu, seed=L * 1000 + pages)
    dst = rand_pool(L, pages, shape, dtype, gpu, seed=L * 1000 + pages + 1)
    g = torch.Generator().manual_seed(pages)
    s_ids = torch.randperm(pages, generator=g)[:n]
    d_ids = torch.randperm(pages, generator=g)[:n]
    s_dev, d_dev = s_ids.to(gpu), d_ids.to(gpu)
    ref_buf = torch.stack([torch.index_select(words(s), 0, s_dev) for s in src])
    ref_dst = [words(d).clone().index_copy_(0, d_dev, ref_buf[i]) for i, d in enumerate(dst)]
    src_before = [words(s).clone() for s in src]

    buf = ops.pack(src, s_ids.tolist())
    torch.cuda.synchronize()
    assert torch.equal(words(buf), ref_buf)
    dst_a = [d.clone() for d in dst]
    ops.unpack(buf, dst_a, d_ids.int().to(gpu))
    dst_b = [d.clone() for d in dst]
    ops.move(src, s_ids.tolist(), dst_b, d_ids.tolist())
    torch.cuda.synchronize()
    for l in range(L):
        assert torch.equal(words(dst_a[l]), ref_dst[l]), f"unpack layer {l}"
        assert torch.equal(words(dst_b[l]), ref_dst[l]), f"move layer {l}"
        assert torch.equal(words(src[l]), src_before[l]), f"source layer {l} written"
    if L * pages * np.prod(shape) <= 1 << 22:     # oracle on the CPU for small cases
        np_src = [words(s).cpu().numpy() for s in src]
        np.testing.assert_array_equal(words(buf).cpu().numpy(), orc.pack(np_src, s_ids.tolist()))


def test_layer_ranges_and_preallocated_buffer(gpu):
    L, pages, shape = 6, 30, (2, 16, 8, 128)
    src = rand_pool(L, pages, shape, torch.bfloat16, gpu, 1)
    ids = [29, 0, 13, 7]
    big = torch.full((3, 10) + shape, 7.0, dtype=torch.bfloat16, device=gpu)   # room for 10 pages
    ops.pack(src, ids, big, layer_begin=2, layer_end=5)
    torch.cuda.synchronize()
    for i, l in enumerate(range(2, 5)):
        assert same(big[i, :4], src[l][torch.tensor(ids, device=gpu)])
        assert (big[i, 4:] == 7.0).all()


def test_out_of_range_ids_are_skipped_and_counted(gpu):
    L, pages, shape = 3, 8, (2, 16, 8, 128)
    src = rand_pool(L, pages, shape, torch.float16, gpu, 2)
    ids = torch.tensor([1, 8, -1, 5], dtype=torch.int32, device=gpu)   # 8 and -1 are invalid
    out = torch.full((L, 4) + shape, 3.0, dtype=torch.float16, device=gpu)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    ops.pack(src, ids, out, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 2 * L
    for l in range(L):
        assert same(out[l, 0], src[l][1]) and same(out[l, 3], src[l][5])
        assert (out[l, 1] == 3.0).all() and (out[l, 2] == 3.0).all()
    dst = rand_pool(L, pages, shape, torch.float16, gpu, 3)
    before = [d.clone() for d in dst]
    err.zero_()
    ops.unpack(out, dst, torch.tensor([2, 100, 4, -7], dtype=torch.int32, device=gpu), err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 2 * L
    for l in range(L):
        assert same(dst[l][2], out[l, 0]) and same(dst[l][4], out[l, 2])
        keep = [0, 1, 3, 5, 6, 7]
        assert same(dst[l][keep], before[l][keep])


def check_large_batch(gpu, L, pages, shape, n, seed):
    src = rand_pool(L, pages, shape, torch.float16, gpu, seed)
    dst = rand_pool(L, pages, shape, torch.float16, gpu, seed + 1)
    g = torch.Generator(device=gpu).manual_seed(seed + 2)
    s_ids = torch.randperm(pages, generator=g, device=gpu)[:n].to(torch.int32)
    d_ids = torch.randperm(pages, generator=g, device=gpu)[:n].to(torch.int32)
    want = [d.clone() for d in dst]
    for l in range(L):
        words(want[l]).index_copy_(0, d_ids.long(), words(src[l]).index_select(0, s_ids.long()))
    buf = ops.pack(src, s_ids)
    fused = [d.clone() for d in dst]
    ops.unpack(buf, dst, d_ids)
    ops.move(src, s_ids, fused, d_ids)
    torch.cuda.synchronize()
    for l in range(L):
        assert same(buf[l], src[l].index_select(0, s_ids.long()))
        assert same(dst[l], want[l]) and same(fused[l], want[l])


def test_batches_of_more_than_65535_pages(gpu):
    # 128-byte pages (a partial 1 KiB row each): 131 073 pages in one launch
    # of 131 073 x 2 workgroups.
    check_large_batch(gpu, 2, 140_000, (2, 4, 1, 8), 131_073, 11)


def test_batches_over_2_pow_25_workgroups_split_across_launches(gpu):
    # 16-byte pages (one workgroup each): 2^24 + 7 pages of 2 layers are
    # 2^25 + 14 workgroups, more than one launch takes, so the pages split
    # over two launches.
    check_large_batch(gpu, 2, (1 << 24) + 100, (2, 1, 1, 4), (1 << 24) + 7, 21)


def test_empty_batch_is_a_no_op(gpu):
    src = rand_pool(2, 4, (2, 16, 8, 128), torch.float16, gpu, 4)
    buf = ops.pack(src, [])
    assert buf.shape == (2, 0, 2, 16, 8, 128)
    ops.unpack(buf, src, [])
    ops.move(src, [], src, [])
    torch.cuda.synchronize()


@pytest.mark.parametrize("n,layers_per_chunk", [(5, 1), (12, 3), (12, 8), (1, 2)])
def test_staging_pack_to_host_and_back(gpu, n, layers_per_chunk):
    L, pages, shape = 7, 16, (2, 16, 8, 128)
    src = rand_pool(L, pages, shape, torch.bfloat16, gpu, 10 + n)
    dst = rand_pool(L, pages, shape, torch.bfloat16, gpu, 20 + n)
    g = torch.Generator().manual_seed(n)
    s_ids = torch.randperm(pages, generator=g)[:n].tolist()
    d_ids = torch.randperm(pages, generator=g)[:n].tolist()
    page_bytes = int(np.prod(shape)) * 2
    with ops.Stager(layers_per_chunk * n * page_bytes, 2) as st:
        host = torch.empty((L, n) + shape, dtype=torch.bfloat16, pin_memory=True)
        st.pack_to_host(src, s_ids, host, layers_per_chunk)
        torch.cuda.current_stream().synchronize()
        ref = torch.stack([s[torch.tensor(s_ids, device=gpu)] for s in src]).cpu()
        assert same(host, ref)
        expect = [words(d).clone() for d in dst]
        for l in range(L):
            expect[l][torch.tensor(d_ids, device=gpu)] = words(ref[l]).to(gpu)
        st.unpack_from_host(host, dst, d_ids, layers_per_chunk)
        torch.cuda.current_stream().synchronize()
        for l in range(L):
            assert torch.equal(words(dst[l]), expect[l]), f"layer {l}"
        # pageable host memory goes through the same pipeline
        pageable = ref.clone()
        dst2 = rand_pool(L, pages, shape, torch.bfloat16, gpu, 20 + n)
        st.unpack_from_host(pageable, dst2, d_ids, layers_per_chunk)
        torch.cuda.current_stream().synchronize()
        for l in range(L):
            assert torch.equal(words(dst2[l]), expect[l]), f"pageable layer {l}"


@pytest.mark.parametrize("slots,host_chunks,layers_per_chunk", [(2, None, 1), (3, 1, 2), (2, 2, 3), (4, None, 5)])
def test_roundtrip_matches_move(gpu, slots, host_chunks, layers_per_chunk):
    L, pages, shape, n = 9, 24, (2, 16, 8, 128), 10
    src = rand_pool(L, pages, shape, torch.float16, gpu, 30)
    dst = rand_pool(L, pages, shape, torch.float16, gpu, 31)
    ref = [d.clone() for d in dst]
    g = torch.Generator().manual_seed(5)
    s_ids = torch.randperm(pages, generator=g)[:n].tolist()
    d_ids = torch.randperm(pages, generator=g)[:n].tolist()
    ops.move(src, s_ids, ref, d_ids)
    page_bytes = int(np.prod(shape)) * 2
    chunk = layers_per_chunk * n * page_bytes
    host_bytes = L * n * page_bytes if host_chunks is None else host_chunks * chunk
    host = torch.empty(host_bytes, dtype=torch.uint8, pin_memory=True)
    with ops.Stager(chunk, slots) as st:
        for rep in range(2):              # back-to-back calls reuse slots and events
            out = [d.clone() for d in dst]
            st.roundtrip(src, s_ids, out, d_ids, host, layers_per_chunk)
            torch.cuda.current_stream().synchronize()
            for l in range(L):
                assert same(out[l], ref[l]), f"rep {rep} layer {l}"


def test_stager_rejects_oversized_chunks(gpu):
    src = rand_pool(2, 8, (2, 16, 8, 128), torch.float16, gpu, 40)
    host = torch.empty((2, 4, 2, 16, 8, 128), dtype=torch.float16, pin_memory=True)
    with ops.Stager(65536 * 3, 2) as st:         # one layer of 4 pages needs 4 * 65536
        with pytest.raises(_native.PaceKVError, match="slot holds"):
            st.pack_to_host(src, [0, 1, 2, 3], host, 1)


def test_concurrent_host_threads_on_their_own_streams(gpu):
    # The reference inserts from several Ray threads at once; the entry points
    # hold no global state, so threads driving their own streams interleave
    # freely.  Each thread moves its own disjoint set of pages.
    import threading

    L, pages, shape, threads, rounds = 4, 256, (2, 16, 8, 128), 4, 25
    src = rand_pool(L, pages, shape, torch.bfloat16, gpu, 21)
    dst = rand_pool(L, pages, shape, torch.bfloat16, gpu, 22)
    src_pool, dst_pool = ops.PagedPool(src), ops.PagedPool(dst)
    perm = torch.randperm(pages, generator=torch.Generator().manual_seed(23))
    share = pages // threads
    sets = [(perm[t * share:(t + 1) * share].tolist(), perm.flip(0)[t * share:(t + 1) * share].tolist())
            for t in range(threads)]
    errors = []
    # The pools were filled on the default stream, which the workers' streams
    # (torch's pooled streams are non-blocking) do not wait for.
    torch.cuda.synchronize()

    def worker(t):
        try:
            s_ids, d_ids = sets[t]
            stream = torch.cuda.Stream(gpu)
            with torch.cuda.stream(stream):
                s_dev = torch.tensor(s_ids, dtype=torch.int32, device=gpu)
                d_dev = torch.tensor(d_ids, dtype=torch.int32, device=gpu)
                for r in range(rounds):
                    if r % 2:
                        ops.move(src_pool, s_dev, dst_pool, d_dev)
                    else:
                        buf = ops.pack(src_pool, s_dev)
                        ops.unpack(buf, dst_pool, d_dev)
            stream.synchronize()
        except Exception as e:          # reported by the main thread
            errors.append((t, repr(e)))

    ts = [threading.Thread(target=worker, args=(t,)) for t in range(threads)]
    for th in ts:
        th.start()
    for th in ts:
        th.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for s_ids, d_ids in sets:
        si = torch.tensor(s_ids, device=gpu)
        di = torch.tensor(d_ids, device=gpu)
        for l in range(L):
            assert same(dst[l].index_select(0, di), src[l].index_select(0, si))


# (slots, host ring regions, layers, layers per chunk): the round trip's
# enqueue order needs two slots and two regions, and runs one chunk at a time
# with a one-region ring; a two-slot stager with many chunks exercises every
# wait of the order at its tightest.
ROUNDTRIP_EDGES = [(2, 2, 12, 1), (2, 12, 12, 1), (3, 1, 6, 1), (5, 3, 13, 2), (2, 2, 2, 1), (4, 1, 1, 1)]


@pytest.mark.parametrize("slots,regions,L,k", ROUNDTRIP_EDGES)
def test_roundtrip_enqueue_order_edges(gpu, slots, regions, L, k):
    """pace_kv_roundtrip at the edges of its enqueue order, three calls in a
    row on one stager (the later calls wait on events the earlier ones
    recorded) with a different host ring and batch each time: every layer of
    the destination equals torch's scatter of torch's gather."""
    print(f"roundtrip edges: slots={slots} regions={regions} L={L} k={k}", flush=True)
    shape, pages = (2, 16, 2, 64), 40
    page_bytes = int(np.prod(shape)) * 2
    src = rand_pool(L, pages, shape, torch.bfloat16, gpu, 300 + L)
    rng = np.random.default_rng(300 + slots * 10 + regions)
    with ops.Stager(-(-(k * pages * page_bytes) // 256) * 256, slots) as st:
        for rep in range(3):
            n = int(rng.integers(1, pages + 1))
            s_ids = rng.permutation(pages)[:n].tolist()
            d_ids = rng.permutation(pages)[:n].tolist()
            dst = rand_pool(L, pages, shape, torch.bfloat16, gpu, 400 + rep)
            before = [d.clone() for d in dst]
            ring = torch.empty(regions * k * n * page_bytes, dtype=torch.uint8, pin_memory=True)
            st.roundtrip(src, s_ids, dst, d_ids, ring, k)
            torch.cuda.current_stream().synchronize()
            bad = workloads.migration_mismatch(src, dst, torch.tensor(s_ids, device=gpu),
                                               torch.tensor(d_ids, device=gpu), before)
            assert bad is None, f"rep {rep}: {bad}"


def test_roundtrips_on_two_streams_share_one_host_buffer(gpu):
    """Two round trips through one stager and one pinned host buffer,
    enqueued back to back on two streams with no synchronisation between
    them and with different chunk sizes (so their host regions overlap
    differently): the second call's device-to-host copies wait for the
    first call's host-to-device copies, and both destinations are exact."""
    L, pages, shape = 8, 48, (2, 16, 2, 64)
    page_bytes = int(np.prod(shape)) * 2
    src = rand_pool(L, pages, shape, torch.bfloat16, gpu, 500)
    dsts = [rand_pool(L, pages, shape, torch.bfloat16, gpu, 501 + i) for i in range(2)]
    befores = [[d.clone() for d in dst] for dst in dsts]
    rng = np.random.default_rng(500)
    n = 40
    s_ids = [rng.permutation(pages)[:n].tolist() for _ in range(2)]
    d_ids = [rng.permutation(pages)[:n].tolist() for _ in range(2)]
    host = torch.empty(4 * n * page_bytes, dtype=torch.uint8, pin_memory=True)   # 4 one-layer regions, 2 two-layer
    streams = [torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)]
    torch.cuda.synchronize()
    with ops.Stager(2 * n * page_bytes, 3) as st:
        for i, k in enumerate((1, 2)):
            with torch.cuda.stream(streams[i]):
                st.roundtrip(src, s_ids[i], dsts[i], d_ids[i], host, k)
        torch.cuda.synchronize()
    for i in range(2):
        bad = workloads.migration_mismatch(src, dsts[i], torch.tensor(s_ids[i], device=gpu),
                                           torch.tensor(d_ids[i], device=gpu), befores[i])
        assert bad is None, f"call {i}: {bad}"


@pytest.mark.parametrize("side", [False, True], ids=["null-stream", "side-stream"])
def test_roundtrip_orders_against_the_callers_stream(gpu, side):
    """The round trip's kernels run on a stream of the stager's own; the
    caller's stream orders them all the same.  With no synchronisation
    anywhere: the caller's stream spins (~20 ms), then writes new contents
    into the source pool, then calls the round trip, then snapshots the
    destination.  The snapshot holds the new contents at every moved page
    (the packs waited for the write; the snapshot waited for the unpacks)."""
    L, pages, shape = 6, 64, (2, 16, 2, 64)
    page_bytes = int(np.prod(shape)) * 2
    src = rand_pool(L, pages, shape, torch.bfloat16, gpu, 700)
    new = rand_pool(L, pages, shape, torch.bfloat16, gpu, 701)
    dst = rand_pool(L, pages, shape, torch.bfloat16, gpu, 702)
    before = [d.clone() for d in dst]
    rng = np.random.default_rng(700)
    n = 48
    s_ids = rng.permutation(pages)[:n].tolist()
    d_ids = rng.permutation(pages)[:n].tolist()
    host = torch.empty(L * n * page_bytes, dtype=torch.uint8, pin_memory=True)
    stream = torch.cuda.Stream(gpu) if side else torch.cuda.current_stream(gpu)
    with ops.Stager(2 * n * page_bytes, 3) as st:
        # the first call creates the host-ring events outside the timed order
        st.roundtrip(src, s_ids, dst, d_ids, host, 2)
        for d, b in zip(dst, before):
            d.copy_(b)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            torch.cuda._sleep(50_000_000)
            for s, w in zip(src, new):
                s.copy_(w)
            st.roundtrip(src, s_ids, dst, d_ids, host, 2)
            snap = [d.clone() for d in dst]
        torch.cuda.synchronize()
    bad = workloads.migration_mismatch(new, snap, torch.tensor(s_ids, device=gpu),
                                       torch.tensor(d_ids, device=gpu), before)
    assert bad is None, bad


@pytest.mark.parametrize("ks", [(2, 2, 2, 2), (6, 2, 6, 2), (2, 6, 2, 6)],
                         ids=["all-chunked", "one-chunk-first", "one-chunk-second"])
def test_mixed_stager_calls_on_two_streams_without_synchronisation(gpu, ks):
    """One stager's slots and events order every kind of call against the
    others: a round trip on stream A, a pack to host on stream B, an unpack
    from host on stream A and a round trip on stream B, enqueued back to back
    with no synchronisation (the four calls move independent data), all end
    exact, also when some calls are one chunk (whose stages all run on the
    caller's stream) and the others three."""
    L, pages, shape, n, k = 6, 48, (2, 16, 2, 64), 40, 2
    page_bytes = int(np.prod(shape)) * 2
    rng = np.random.default_rng(950)
    srcs = [rand_pool(L, pages, shape, torch.bfloat16, gpu, 950 + i) for i in range(4)]
    dsts = [rand_pool(L, pages, shape, torch.bfloat16, gpu, 960 + i) for i in range(4)]
    befores = [[d.clone() for d in dst] for dst in dsts]
    s_ids = [rng.permutation(pages)[:n].tolist() for _ in range(4)]
    d_ids = [rng.permutation(pages)[:n].tolist() for _ in range(4)]
    ring = [torch.empty(3 * k * n * page_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    host_out = torch.empty((L, n) + shape, dtype=torch.bfloat16, pin_memory=True)
    # the unpack's input: call 2's source pages, gathered by torch
    host_in = torch.stack([s[torch.tensor(s_ids[2], device=gpu)] for s in srcs[2]]).cpu().pin_memory()
    streams = [torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)]
    torch.cuda.synchronize()
    with ops.Stager(L * n * page_bytes, 4) as st:
        with torch.cuda.stream(streams[0]):
            st.roundtrip(srcs[0], s_ids[0], dsts[0], d_ids[0], ring[0], ks[0])
        with torch.cuda.stream(streams[1]):
            st.pack_to_host(srcs[1], s_ids[1], host_out, ks[1])
        with torch.cuda.stream(streams[0]):
            st.unpack_from_host(host_in, dsts[2], d_ids[2], ks[2])
        with torch.cuda.stream(streams[1]):
            st.roundtrip(srcs[3], s_ids[3], dsts[3], d_ids[3], ring[1], ks[3])
        torch.cuda.synchronize()
    for i in (0, 2, 3):
        bad = workloads.migration_mismatch(srcs[i], dsts[i], torch.tensor(s_ids[i], device=gpu),
                                           torch.tensor(d_ids[i], device=gpu), befores[i])
        assert bad is None, f"call {i}: {bad}"
    want = torch.stack([s[torch.tensor(s_ids[1], device=gpu)] for s in srcs[1]]).cpu()
    assert torch.equal(words(host_out), words(want)), "call 1: pack to host"


@pytest.mark.parametrize("ks", [(2, 6, 2, 6), (6, 2, 6, 2), (2, 2, 2, 2), (6, 6, 6, 6)],
                         ids=["chunked-first", "one-chunk-first", "all-chunked", "all-one-chunk"])
def test_roundtrips_into_the_same_pages_land_in_call_order(gpu, ks):
    """Round trips on one stager run their unpacks in call order whichever
    stream each names: four calls enqueued back to back with no
    synchronisation, alternating two streams, each writing other source
    pages into the same destination pages, leave the last call's pages, also
    when one-chunk calls (on the caller's stream) and three-chunk calls (on
    the stager's streams) alternate."""
    L, pages, shape, n = 6, 64, (2, 16, 2, 64), 40
    page_bytes = int(np.prod(shape)) * 2
    rng = np.random.default_rng(970)
    srcs = [rand_pool(L, pages, shape, torch.bfloat16, gpu, 970 + i) for i in range(4)]
    dst = rand_pool(L, pages, shape, torch.bfloat16, gpu, 979)
    s_ids = [rng.permutation(pages)[:n].tolist() for _ in range(4)]
    d_ids = rng.permutation(pages)[:n].tolist()
    rings = [torch.empty(L * n * page_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(4)]
    streams = [torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)]
    torch.cuda.synchronize()
    with ops.Stager(L * n * page_bytes, 3) as st:
        for i in range(4):
            with torch.cuda.stream(streams[i % 2]):
                st.roundtrip(srcs[i], s_ids[i], dst, d_ids, rings[i], ks[i])
        torch.cuda.synchronize()
    d_dev = torch.tensor(d_ids, device=gpu)
    s_dev = torch.tensor(s_ids[3], device=gpu)
    for l in range(L):
        assert torch.equal(words(dst[l][d_dev]), words(srcs[3][l][s_dev])), f"layer {l}"


def test_random_call_sequences_on_three_streams(gpu):
    """Seeded random sequences of 3-7 calls on one stager (pack to host,
    unpack from host, round trip; 1, 2, 3 or 6 layers per chunk, so one chunk
    or several) spread over three streams with no synchronisation between
    them.  Every call's bytes are exact, and round trips into one shared
    destination leave the last one's pages."""
    L, pages, shape, n = 6, 64, (2, 16, 2, 64), 24
    page_bytes = int(np.prod(shape)) * 2
    streams = [torch.cuda.Stream(gpu) for _ in range(3)]
    srcs = [rand_pool(L, pages, shape, torch.bfloat16, gpu, 500 + i) for i in range(4)]
    with ops.Stager(L * n * page_bytes, 3) as st:
        for it in range(40):
            rng = np.random.default_rng(it)
            shared = rand_pool(L, pages, shape, torch.bfloat16, gpu, 900 + it)
            shared_ids = rng.permutation(pages)[:n].tolist()
            last, checks, keep = None, [], []
            torch.cuda.synchronize()
            for c in range(int(rng.integers(3, 8))):
                kind = str(rng.choice(["pack", "unpack", "roundtrip", "shared"]))
                k = int(rng.choice([1, 2, 3, 6]))
                src = srcs[int(rng.integers(0, len(srcs)))]
                s_ids = rng.permutation(pages)[:n].tolist()
                d_ids = rng.permutation(pages)[:n].tolist()
                want = torch.stack([words(t)[torch.tensor(s_ids, device=gpu)] for t in src])
                ring = torch.empty(L * n * page_bytes, dtype=torch.uint8, pin_memory=True)
                keep.append(ring)
                with torch.cuda.stream(streams[int(rng.integers(0, 3))]):
                    if kind == "pack":
                        host = torch.zeros((L, n) + shape, dtype=torch.bfloat16, pin_memory=True)
                        st.pack_to_host(src, s_ids, host, k)
                        checks.append((kind, host, None, want))
                    elif kind == "unpack":
                        dst = rand_pool(L, pages, shape, torch.bfloat16, gpu, 700 + c)
                        host = want.view(torch.bfloat16).cpu().pin_memory()
                        keep.append(host)
                        st.unpack_from_host(host, dst, d_ids, k)
                        checks.append((kind, dst, d_ids, want))
                    elif kind == "roundtrip":
                        dst = rand_pool(L, pages, shape, torch.bfloat16, gpu, 800 + c)
                        st.roundtrip(src, s_ids, dst, d_ids, ring, k)
                        checks.append((kind, dst, d_ids, want))
                    else:
                        st.roundtrip(src, s_ids, shared, shared_ids, ring, k)
                        last = want
            torch.cuda.synchronize()
            for kind, out, d_ids, want in checks:
                if kind == "pack":
                    assert torch.equal(words(out), want.cpu()), f"iteration {it}: pack to host"
                else:
                    di = torch.tensor(d_ids, device=gpu)
                    for l in range(L):
                        assert torch.equal(words(out[l])[di], want[l]), f"iteration {it}: {kind} layer {l}"
            if last is not None:
                di = torch.tensor(shared_ids, device=gpu)
                for l in range(L):
                    assert torch.equal(words(shared[l])[di], last[l]), f"iteration {it}: shared destination"


@pytest.mark.parametrize("k", [2, 6], ids=["three-chunks", "one-chunk"])
def test_roundtrip_failing_part_way_leaves_the_stager_usable(gpu, k):
    """A round trip whose destination table has a NULL pointer for the last
    layer fails when it reaches that layer's chunk, on the host, after the
    earlier chunks were packed, copied and unpacked (the NULL pointer never
    reaches a kernel).  The call returns PACE_KV_EINVAL naming the layer, the
    earlier chunks' destination layers are exact, the later ones untouched,
    and the same stager then runs a full round trip exactly.  With one chunk
    (every stage on the caller's stream) no destination layer changes."""
    L, pages, shape, n = 6, 64, (2, 16, 2, 64), 40
    page_bytes = int(np.prod(shape)) * 2
    src = rand_pool(L, pages, shape, torch.bfloat16, gpu, 900)
    dst = rand_pool(L, pages, shape, torch.bfloat16, gpu, 901)
    before = [d.clone() for d in dst]
    rng = np.random.default_rng(900)
    s_ids = rng.permutation(pages)[:n].tolist()
    d_ids = rng.permutation(pages)[:n].tolist()
    s_dev = torch.tensor(s_ids, dtype=torch.int32, device=gpu)
    d_dev = torch.tensor(d_ids, dtype=torch.int32, device=gpu)
    host = torch.empty(L * n * page_bytes, dtype=torch.uint8, pin_memory=True)
    sp = ops.PagedPool(src)
    table = _native.pointer_array([d.data_ptr() for d in dst[:-1]] + [None])
    lib = _native.load()
    with ops.Stager(k * n * page_bytes, 4) as st:
        rc = lib.pace_kv_roundtrip(st._handle, sp.table(), pages, s_dev.data_ptr(), ctypes.addressof(table),
                                   pages, d_dev.data_ptr(), L, n, page_bytes, k, host.data_ptr(),
                                   host.numel(), None, ops._stream_handle(gpu))
        torch.cuda.synchronize()
        assert rc == _native.PACE_KV_EINVAL
        # the last layer's index within its chunk
        assert f"layer {k - 1} pointer is NULL" in lib.pace_kv_last_error().decode()
        want = [words(b).clone() for b in before]
        for l in range(L - k):
            want[l][d_dev.long()] = words(src[l])[s_dev.long()]
        for l in range(L):
            assert torch.equal(words(dst[l]), want[l]), f"layer {l} after the failed call"
        dst2 = rand_pool(L, pages, shape, torch.bfloat16, gpu, 902)
        before2 = [d.clone() for d in dst2]
        st.roundtrip(src, s_ids, dst2, d_ids, host, k)
        torch.cuda.synchronize()
        bad = workloads.migration_mismatch(src, dst2, s_dev, d_dev, before2)
        assert bad is None, bad


@pytest.mark.parametrize("k", [2, 6], ids=["three-chunks", "one-chunk"])
def test_one_way_legs_failing_part_way_leave_the_stager_usable(gpu, k):
    """A pack to host whose source table, and an unpack from host whose
    destination table, has a NULL pointer for the last layer fail with
    PACE_KV_EINVAL when they reach that layer's chunk (c).  What was enqueued
    before it arrives exactly, and nothing else: the pack has copied chunks
    0..c-2 (step i enqueues pack(i+1) before the copy of chunk i), the unpack
    has written chunks 0..c-1.  The caller's stream is ordered after the
    copies already enqueued, and the same stager then runs both legs
    exactly."""
    L, pages, shape, n = 6, 64, (2, 16, 2, 64), 40
    page_bytes = int(np.prod(shape)) * 2
    src = rand_pool(L, pages, shape, torch.bfloat16, gpu, 930)
    dst = rand_pool(L, pages, shape, torch.bfloat16, gpu, 931)
    before = [d.clone() for d in dst]
    rng = np.random.default_rng(930)
    s_dev = torch.tensor(rng.permutation(pages)[:n].tolist(), dtype=torch.int32, device=gpu)
    d_dev = torch.tensor(rng.permutation(pages)[:n].tolist(), dtype=torch.int32, device=gpu)
    want = torch.stack([words(s)[s_dev.long()] for s in src])      # [L, n, ...] int16 words
    host = torch.zeros((L, n) + shape, dtype=torch.bfloat16, pin_memory=True)
    host_in = want.view(torch.bfloat16).cpu().pin_memory()
    bad_src = _native.pointer_array([t.data_ptr() for t in src[:-1]] + [None])
    bad_dst = _native.pointer_array([t.data_ptr() for t in dst[:-1]] + [None])
    lib = _native.load()
    stream = ops._stream_handle(gpu)
    with ops.Stager(k * n * page_bytes, 3) as st:
        rc = lib.pace_kv_pack_to_host(st._handle, ctypes.addressof(bad_src), L, pages, s_dev.data_ptr(), n,
                                      page_bytes, k, host.data_ptr(), None, stream)
        torch.cuda.synchronize()
        assert rc == _native.PACE_KV_EINVAL
        assert f"layer {k - 1} pointer is NULL" in lib.pace_kv_last_error().decode()
        c = (L - 1) // k                # the failing chunk
        done = max(0, c - 1) * k         # layers copied to the host
        assert torch.equal(words(host)[:done], want[:done].cpu())
        assert not words(host)[done:].any()
        rc = lib.pace_kv_unpack_from_host(st._handle, host_in.data_ptr(), ctypes.addressof(bad_dst), L, pages,
                                          d_dev.data_ptr(), n, page_bytes, k, None, stream)
        torch.cuda.synchronize()
        assert rc == _native.PACE_KV_EINVAL
        for l in range(L):
            expect = words(before[l]).clone()
            if l < c * k:                # layers unpacked
                expect[d_dev.long()] = want[l]
            assert torch.equal(words(dst[l]), expect), f"layer {l} after the failed unpack"
        out = torch.empty((L, n) + shape, dtype=torch.bfloat16, pin_memory=True)
        st.pack_to_host(src, s_dev, out, k)
        dst2 = rand_pool(L, pages, shape, torch.bfloat16, gpu, 932)
        before2 = [d.clone() for d in dst2]
        st.unpack_from_host(host_in, dst2, d_dev, k)
        torch.cuda.synchronize()
        assert torch.equal(words(out), want.cpu())
        bad = workloads.migration_mismatch(src, dst2, s_dev, d_dev, before2)
        assert bad is None, bad


def _hip_host_alloc(nbytes):
    """hipHostMalloc of exactly nbytes, as (uint8 CPU tensor over it, free):
    the caller synchronises and drops every view before calling free()."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    ptr = ctypes.c_void_p()
    assert hip.hipHostMalloc(ctypes.byref(ptr), ctypes.c_size_t(nbytes), ctypes.c_uint(0)) == 0
    arr = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(ptr.value))
    return torch.from_numpy(arr), lambda: hip.hipHostFree(ptr)


@pytest.mark.parametrize("k", [2, 6], ids=["three-chunks", "one-chunk"])
@pytest.mark.parametrize("kind", ["pageable", "pinned-at-offset", "pinned-to-the-end"])
def test_roundtrip_host_buffer_kinds(gpu, kind, k):
    """The round trip, and a one-chunk pack to host, copy device to host with
    a kernel when the host buffer is pinned memory the device addresses, and
    with hipMemcpyAsync otherwise.  A pageable buffer, a pinned view starting
    4 KiB into its allocation, and a pinned view ending exactly at its
    allocation's end all give the exact destination (and host bytes), two
    calls in a row; the second call's chunks (656 KiB per layer) are not a
    multiple of the kernel's 256 KiB pass, so its remainder loop runs."""
    L, pages, shape = 6, 64, (2, 16, 2, 64)
    page_bytes = int(np.prod(shape)) * 2
    src = rand_pool(L, pages, shape, torch.bfloat16, gpu, 800)
    rng = np.random.default_rng(800)
    with ops.Stager(6 * 48 * page_bytes, 4) as st:
        for rep in range(2):
            n = 48 - rep * 7
            need = L * n * page_bytes
            free = None
            if kind == "pageable":
                host = torch.empty(need, dtype=torch.uint8)
            elif kind == "pinned-at-offset":
                host = torch.empty(need + 4096, dtype=torch.uint8, pin_memory=True)[4096:]
            else:
                # torch's host allocator rounds a block up; hipHostMalloc gives the exact size
                base, free = _hip_host_alloc(need + 16)
                host = base[16:]
            s_ids = rng.permutation(pages)[:n].tolist()
            d_ids = rng.permutation(pages)[:n].tolist()
            dst = rand_pool(L, pages, shape, torch.bfloat16, gpu, 801 + rep)
            before = [d.clone() for d in dst]
            want = torch.stack([words(s)[torch.tensor(s_ids, device=gpu)] for s in src]).cpu()
            try:
                st.roundtrip(src, s_ids, dst, d_ids, host, k)
                torch.cuda.synchronize()   # the round trip reads host until it completes
                host.zero_()
                st.pack_to_host(src, s_ids, host.view(torch.bfloat16).view((L, n) + shape), k)
                torch.cuda.synchronize()
                packed = host.view(torch.int16).view(want.shape).clone()
            finally:
                torch.cuda.synchronize()
                if free is not None:
                    st._inflight.clear()
                    del host, base
                    free()
            bad = workloads.migration_mismatch(src, dst, torch.tensor(s_ids, device=gpu),
                                               torch.tensor(d_ids, device=gpu), before)
            assert bad is None, f"{kind} rep {rep}: {bad}"
            assert torch.equal(packed, want), f"{kind} rep {rep}: pack to host"


@pytest.mark.parametrize("seed", range(16))
def test_random_staging_matches_torch(gpu, seed):
    """Seeded random pinned-host legs through one stager: layer counts on both
    sides of the 64-layer launch split, pages of 64 B to 64 KiB (whole and
    partial 1 KiB rows), four element types, 1 to all layers per chunk, 2-5
    slots, and a host ring of one chunk up to the whole payload; pack to host,
    unpack from host and the round trip, each compared with torch's gather
    and scatter, twice in a row on the same stager with different batches."""
    rng = np.random.default_rng(9000 + seed)
    L = int(rng.choice([1, 3, 8, 33, 70]))
    shape = (2, int(rng.choice([1, 4, 16])), int(rng.choice([1, 2, 8])), int(rng.choice([8, 64, 128])))
    dtype = [torch.float16, torch.bfloat16, torch.float32, torch.uint8][int(rng.integers(0, 4))]
    esz = torch.empty(0, dtype=dtype).element_size()
    page_bytes = int(np.prod(shape)) * esz
    pages = int(rng.integers(1, 200))
    k = int(rng.integers(1, L + 1))                   # layers per chunk
    slots = int(rng.integers(2, 6))
    src = rand_pool(L, pages, shape, dtype, gpu, 100 + seed)
    dst = rand_pool(L, pages, shape, dtype, gpu, 200 + seed)
    chunk = -(-(k * pages * page_bytes) // 256) * 256  # slots hold k layers of up to all pages
    print(f"random staging seed {seed}: L={L} shape={shape} {dtype} pages={pages} k={k} slots={slots}",
          flush=True)
    with ops.Stager(chunk, slots) as st:
        for rep in range(2):
            n = int(rng.integers(1, pages + 1))
            s_ids = rng.permutation(pages)[:n].tolist()
            d_ids = rng.permutation(pages)[:n].tolist()
            si, di = torch.tensor(s_ids, device=gpu), torch.tensor(d_ids, device=gpu)
            ref = torch.stack([words(s)[si] for s in src])                     # [L, n, ...] on the device
            expect = [words(d).clone() for d in dst]
            for l in range(L):
                expect[l][di] = ref[l]
            # pack to host
            host = torch.empty((L, n) + shape, dtype=dtype, pin_memory=True)
            st.pack_to_host(src, s_ids, host, k)
            torch.cuda.current_stream().synchronize()
            assert torch.equal(words(host), ref.cpu()), f"rep {rep}: pack_to_host"
            # unpack from host
            got = [d.clone() for d in dst]
            st.unpack_from_host(host, got, d_ids, k)
            torch.cuda.current_stream().synchronize()
            for l in range(L):
                assert torch.equal(words(got[l]), expect[l]), f"rep {rep}: unpack_from_host layer {l}"
            # round trip through a host ring of one chunk up to the whole payload
            ring_chunks = int(rng.integers(1, -(-L // k) + 1))
            ring = torch.empty(ring_chunks * k * n * page_bytes, dtype=torch.uint8, pin_memory=True)
            got = [d.clone() for d in dst]
            st.roundtrip(src, s_ids, got, d_ids, ring, k)
            torch.cuda.current_stream().synchronize()
            for l in range(L):
                assert torch.equal(words(got[l]), expect[l]), f"rep {rep}: roundtrip layer {l}"
