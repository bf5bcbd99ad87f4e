"""The cross-process channel on the GPU: pages packed out of one pool and
unpacked into another through the shared-memory ring, checked bit-exactly
against torch's own gather; device and host payloads on either side; a
sender in another process; and the worker methods that replace returning a
KVobj through Ray (_send_kv_cache / _recv_kv_cache / _recv_next_kv_cache),
with insertion threads sharing one channel."""
import os
import subprocess
import sys
import threading
from pathlib import Path

import numpy as np
import pytest
import torch

from paceserve_amd import workloads
from paceserve_amd.core.sequence import Sequence
from paceserve_amd.kv_transfer import ops
from paceserve_amd.kv_transfer.channel import KVChannel, KVref
from paceserve_amd.kv_transfer.kv_utils import KVhelper
from paceserve_amd.kv_transfer.worker import KVStatus, KVWorker, WorkerSequenceManager

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
_count = [0]


def name():
    _count[0] += 1
    return f"pace_gpu_test_{os.getpid()}_{_count[0]}"


def words(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.uint8)


def rand_pool(L, pages, shape, dtype, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    return [torch.randn((pages,) + shape, generator=g, device=dev, dtype=torch.float32).to(dtype)
            for _ in range(L)]


# The three requests the cross-process tests send: request r moves source
# pages r, r+3, ... (40 of them) into destination pages 40r .. 40r+39.
PEER_SRC_IDS = [p for r in range(3) for p in list(range(r, 128, 3))[:40]]
PEER_DST_IDS = list(range(120))


def peer_mismatch(src, dst, dev):
    """Whole-layer check of the three requests into a zeroed destination
    (workloads.migration_mismatch: every page of every layer, so a stray
    write into a page no request names fails)."""
    return workloads.migration_mismatch(src, dst, torch.tensor(PEER_SRC_IDS, device=dev),
                                        torch.tensor(PEER_DST_IDS, device=dev),
                                        (torch.zeros_like(s) for s in src))


def run_pair(slot_bytes, num_slots, send, recv, device_slot_bytes=0):
    """Runs send(tx) on a thread and recv(rx) here; returns send's result.
    device_slot_bytes > 0: the channel also has a device ring (same GPU), so
    device payloads go through it."""
    nm = name()
    rx = KVChannel.create(nm, slot_bytes, num_slots, 4, device_slot_bytes=device_slot_bytes)
    tx = KVChannel.open(nm, 4, timeout=10)
    if device_slot_bytes:
        assert tx.device_ring() == (device_slot_bytes, True)
    out, errs = [], []

    def sender():
        try:
            out.append(send(tx))
        except Exception as e:                     # reported below
            errs.append(repr(e))

    t = threading.Thread(target=sender)
    t.start()
    try:
        recv(rx)
    finally:
        t.join(timeout=60)
        tx.close()
        rx.close()
    assert not errs, errs
    return out[0] if out else None


# (layers, pool pages, page shape, pages sent, slot bytes): layer chunks, page
# chunks (a layer larger than a slot), a partial 1 KiB row per page, more
# layers than one launch takes, one page.
CASES = [(32, 64, (2, 16, 8, 128), 20, 4 << 20), (4, 300, (2, 16, 8, 128), 200, 1 << 20),
         (3, 50, (2, 3, 1, 16), 40, 4096), (70, 16, (2, 16, 1, 64), 9, 1 << 20), (2, 8, (2, 16, 8, 128), 1, 1 << 20)]


@pytest.mark.parametrize("L,pages,shape,n,slot", CASES)
def test_device_to_device_through_the_ring(gpu, L, pages, shape, n, slot):
    print(f"channel case L={L} pages={pages} shape={shape} n={n} slot={slot}", flush=True)
    src = rand_pool(L, pages, shape, torch.float16, gpu, 1)
    dst = rand_pool(L, pages, shape, torch.float16, gpu, 2)
    rng = np.random.default_rng(L + n)
    s_ids = rng.permutation(pages)[:n].tolist()
    d_ids = rng.permutation(pages)[:n].tolist()
    before = [words(d).clone() for d in dst]

    def recv(rx):
        h = rx.recv_header(timeout=30)
        assert (h.meta, h.num_layers, h.n_pages) == (b"pages", L, n)
        rx.recv(dst, d_ids, timeout=30)
        torch.cuda.synchronize()

    msg = run_pair(slot, 4, lambda tx: tx.send(src, s_ids, b"pages", timeout=30), recv)
    assert msg >= 1
    si, di = torch.tensor(s_ids, device=gpu), torch.tensor(d_ids, device=gpu)
    keep = torch.tensor(sorted(set(range(pages)) - set(d_ids)), device=gpu, dtype=torch.long)
    for l in range(L):
        assert torch.equal(words(dst[l])[di], words(src[l])[si]), f"layer {l}"
        assert torch.equal(words(dst[l])[keep], before[l][keep]), f"layer {l} untouched pages"


def test_device_sender_host_receiver_and_back(gpu):
    L, pages, shape, n = 5, 40, (2, 16, 8, 128), 17
    src = rand_pool(L, pages, shape, torch.bfloat16, gpu, 3)
    ids = np.random.default_rng(5).permutation(pages)[:n].tolist()
    host = torch.empty((L, n) + shape, dtype=torch.bfloat16)

    def recv(rx):
        rx.recv_header(timeout=30)
        rx.recv_host(host, timeout=30)

    run_pair(1 << 20, 2, lambda tx: tx.send(src, ids, timeout=30), recv)
    want = torch.stack([s[torch.tensor(ids, device=gpu)] for s in src]).cpu()
    assert torch.equal(words(host), words(want))

    dst = rand_pool(L, pages, shape, torch.bfloat16, gpu, 4)
    d_ids = np.random.default_rng(6).permutation(pages)[:n].tolist()

    def recv2(rx):
        rx.recv_header(timeout=30)
        rx.recv(dst, d_ids, timeout=30)
        torch.cuda.synchronize()

    run_pair(1 << 20, 2, lambda tx: tx.send_host(host, timeout=30), recv2)
    for l in range(L):
        assert torch.equal(words(dst[l][torch.tensor(d_ids, device=gpu)]).cpu(), words(host[l]))


SENDER = r"""
import sys, torch
sys.path.insert(0, {root!r})
from paceserve_amd.kv_transfer.channel import KVChannel
dev = torch.device("cuda", 0)
g = torch.Generator(device=dev).manual_seed(77)
src = [torch.randn((128, 2, 16, 8, 128), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
       for _ in range(32)]
ch = KVChannel.open({name!r}, 8, timeout=60)
for r in range(3):
    ids = list(range(r, 128, 3))[:40]
    ch.send(src, ids, ("request %d" % r).encode(), timeout=60)
print("sender done", flush=True)
ch.close()
"""


def test_sender_in_another_process(gpu):
    nm = name()
    rx = KVChannel.create(nm, 16 << 20, 4, 8)
    child = subprocess.Popen([sys.executable, "-c", SENDER.format(root=str(ROOT), name=nm)])
    try:
        g = torch.Generator(device=gpu).manual_seed(77)
        src = [torch.randn((128, 2, 16, 8, 128), generator=g, device=gpu, dtype=torch.float32).to(torch.bfloat16)
               for _ in range(32)]
        dst = [torch.zeros_like(s) for s in src]
        for r in range(3):
            h = rx.recv_header(timeout=120)
            assert h.meta == f"request {r}".encode() and h.n_pages == 40
            d_ids = list(range(40 * r, 40 * r + 40))
            rx.recv(dst, d_ids, timeout=60)
        torch.cuda.synchronize()
        assert child.wait(timeout=60) == 0
    finally:
        if child.poll() is None:
            child.kill()
        rx.close()
    assert peer_mismatch(src, dst, gpu) is None


# ---------------------------------------------------------- worker methods

L, H, D, P, POOL = 4, 8, 128, 16, 64


class ModelConfig:
    dtype = torch.float16

    def get_num_q_heads(self, pc):
        return 32

    def get_num_kv_heads(self, pc):
        return H

    def get_head_size(self):
        return D

    def get_num_layers(self, pc):
        return L


class CacheConfig:
    block_size = P


class _Runner:
    def __init__(self, cache):
        self.attention_backend_wrapper = type("W", (), {"gpu_cache": cache})()


def make_worker(dev, seed, free_list=None):
    g = torch.Generator(device=dev).manual_seed(seed)
    cache = [torch.randn(POOL, 2, P, H, D, generator=g, device=dev, dtype=torch.float32).half() for _ in range(L)]
    h = KVhelper(0, ModelConfig(), CacheConfig(), None)
    h.add_model_runner(_Runner(cache))
    return KVWorker(h, WorkerSequenceManager(P, POOL, free_list=free_list)), cache


# the worker-level tests run over the shared-memory ring and over the device ring
RINGS = {"host": 0, "device": 1 << 20}


@pytest.mark.parametrize("ring", RINGS)
@pytest.mark.parametrize("tokens_src,tokens_dst", [(40, 40), (48, 49)])
def test_worker_send_and_receive(gpu, tokens_src, tokens_dst, ring):
    """prefill side _send_kv_cache (frees the source pages) -> KVref on the
    control plane -> decode side _recv_kv_cache with LIFO allocation and the
    n / n+1 remap; the same destination bytes as _get_kv_cache + KVobj +
    _insert_kv_cache."""
    src_w, src_cache = make_worker(gpu, 4, np.random.default_rng(4).permutation(POOL).tolist())
    dst_w, dst_cache = make_worker(gpu, 5)
    seq = Sequence.of_length("r", tokens_src, P)
    src_w.seq_manager.add_seq(seq)
    src_w.seq_manager.block_manager.allocate(seq)
    src_table = src_w.seq_manager._get_block_table(seq)
    free_before = src_w.seq_manager.block_manager.get_num_free_gpu_blocks()
    # the decode side's sequence holds the prompt and the first generated token(s)
    dst_seq = Sequence.of_length("r", tokens_src, P, tokens_dst - tokens_src)
    before = [words(c).clone() for c in dst_cache]
    got = {}

    def recv(rx):
        got["status"] = dst_w._recv_kv_cache(dst_seq, rx, gpu, timeout=30)

    print(f"worker send/receive over the {ring} ring, {tokens_src} -> {tokens_dst} tokens", flush=True)
    ref, rank = run_pair(1 << 20, 4, lambda tx: src_w._send_kv_cache(seq, tx, 1.0, 2.0), recv, RINGS[ring])
    assert isinstance(ref, KVref) and ref.kv_indices == src_table and rank == 0
    assert ref.size == L * len(src_table) * 2 * P * H * D * 2 / 1e6
    assert src_w.seq_manager.block_manager.get_num_free_gpu_blocks() == free_before + len(src_table)
    st = got["status"]
    assert isinstance(st, KVStatus) and st.status
    dst_table = dst_w.seq_manager._get_block_table(dst_seq)
    n = len(src_table)
    assert dst_table[:n] == list(range(POOL - 1, POOL - 1 - n, -1))
    for l in range(L):
        assert torch.equal(words(dst_cache[l][torch.tensor(dst_table[:n], device=gpu)]),
                           words(src_cache[l][torch.tensor(src_table, device=gpu)]))
        untouched = sorted(set(range(POOL)) - set(dst_table[:n]))
        assert torch.equal(words(dst_cache[l][untouched]), before[l][untouched])


@pytest.mark.parametrize("ring", RINGS)
def test_insertion_threads_share_one_channel(gpu, ring):
    """Four insertion threads take whichever sequence arrives next from one
    channel (_recv_next_kv_cache), as the reference's insertion threads insert
    whichever transfer finishes first; every sequence lands in its own
    destination pages."""
    src_w, src_cache = make_worker(gpu, 10)
    dst_w, dst_cache = make_worker(gpu, 11)
    before = [c.clone() for c in dst_cache]
    src_before = [c.clone() for c in src_cache]
    lengths = [16 * k for k in (3, 1, 4, 2, 5, 2, 3, 1)]
    seqs = [Sequence.of_length(f"s{i}", n, P) for i, n in enumerate(lengths)]
    for s in seqs:
        src_w.seq_manager.add_seq(s)
        src_w.seq_manager.block_manager.allocate(s)
    src_tables = {s.seq_id: src_w.seq_manager._get_block_table(s) for s in seqs}
    want = {s.seq_id: [c[torch.tensor(src_tables[s.seq_id], device=gpu)].clone() for c in src_cache] for s in seqs}
    torch.cuda.synchronize()
    dst_seqs = {s.seq_id: Sequence.of_length(s.seq_id, n, P) for s, n in zip(seqs, lengths)}
    results, errors = {}, []
    lock = threading.Lock()

    def insertion_thread(rx):
        # takes messages until it takes a stop message (the sender sends one
        # per thread after the sequences)
        try:
            while True:
                seq, status = dst_w._recv_next_kv_cache(dst_seqs.get, rx, gpu, timeout=30)
                if isinstance(seq, str) and seq.startswith("stop"):
                    return
                with lock:
                    results[seq.seq_id] = status
        except Exception as e:                         # reported below
            errors.append(repr(e))

    def recv(rx):
        ts = [threading.Thread(target=insertion_thread, args=(rx,)) for _ in range(4)]
        for t in ts:
            t.start()
        for t in ts:
            t.join(timeout=60)
        torch.cuda.synchronize()

    def send(tx):
        for s in seqs:
            src_w._send_kv_cache(s, tx)
        # one empty message per thread still waiting, so that every thread returns
        for i in range(4):
            tx.send_host(torch.empty((0, 0, 2, P, H, D), dtype=torch.float16),
                         KVref(f"stop{i}", [], 0.0).meta(), timeout=30)

    print(f"four insertion threads over the {ring} ring", flush=True)
    run_pair(1 << 20, 4, send, recv, RINGS[ring])
    assert not errors, errors
    for s in seqs:
        st = results[s.seq_id]
        assert isinstance(st, KVStatus) and st.status, s.seq_id
        table = dst_w.seq_manager._get_block_table(dst_seqs[s.seq_id])
        for l in range(L):
            assert torch.equal(words(dst_cache[l][torch.tensor(table, device=gpu)]), words(want[s.seq_id][l])), \
                f"{s.seq_id} layer {l}"
    # every page of every layer of both caches: each sequence's pages where its
    # table points, the pages no sequence received untouched, the source unchanged
    s_ids = torch.tensor([p for s in seqs for p in src_tables[s.seq_id]], device=gpu)
    d_ids = torch.tensor([p for s in seqs for p in dst_w.seq_manager._get_block_table(dst_seqs[s.seq_id])],
                         device=gpu)
    bad = workloads.migration_mismatch(src_cache, dst_cache, s_ids, d_ids, before, src_before)
    assert bad is None, bad


@pytest.mark.parametrize("ring", RINGS)
def test_worker_receive_refusals_drain_the_message(gpu, ring):
    """A destination without room, and a message for another sequence, return
    False and leave the channel ready for the next message."""
    src_w, src_cache = make_worker(gpu, 6)
    dst_w, dst_cache = make_worker(gpu, 7, free_list=list(range(3)))          # room for 3 pages
    seqs = [Sequence.of_length(f"s{i}", 16 * k, P) for i, k in enumerate((5, 2, 2))]
    for s in seqs:
        src_w.seq_manager.add_seq(s)
        src_w.seq_manager.block_manager.allocate(s)
    tables = [src_w.seq_manager._get_block_table(s) for s in seqs]
    results = []

    def send(tx):
        return [src_w._send_kv_cache(s, tx) for s in seqs]

    def recv(rx):
        results.append(dst_w._recv_kv_cache(Sequence.of_length("s0", 80, P), rx, gpu, timeout=30))   # 5 > 3 pages
        results.append(dst_w._recv_kv_cache(Sequence.of_length("other", 32, P), rx, gpu, timeout=30))
        results.append(dst_w._recv_kv_cache(Sequence.of_length("s2", 32, P), rx, gpu, timeout=30))
        torch.cuda.synchronize()

    print(f"worker refusals over the {ring} ring", flush=True)
    run_pair(1 << 20, 2, send, recv, RINGS[ring])
    assert results[0] is False and results[1] is False
    assert isinstance(results[2], KVStatus) and results[2].status
    dst_table = dst_w.seq_manager._get_block_table(Sequence.of_length("s2", 32, P))
    for l in range(L):
        assert torch.equal(words(dst_cache[l][torch.tensor(dst_table, device=gpu)]),
                           words(src_cache[l][torch.tensor(tables[2], device=gpu)]))


@pytest.mark.parametrize("ring", RINGS)
def test_helper_zero_fallback_and_repeated_ids(gpu, ring):
    """A sequence without a block table sends one zero page, as get_kv_cache
    returns it; repeated destination ids keep the last page written, as the
    reference's index_put_ does."""
    src_w, _ = make_worker(gpu, 8)
    dst_w, dst_cache = make_worker(gpu, 9)
    src_cache = src_w.kvhelper._gpu_cache()

    class NoTable:
        def _get_block_table(self, seq):
            raise KeyError(seq.seq_id)

    class Table:
        def _get_block_table(self, seq):
            return [3, 4, 5]

    oks = []

    def send(tx):
        a = src_w.kvhelper.send_kv_cache(Sequence.of_length("z", 16, P), NoTable(), tx)
        b = src_w.kvhelper.send_kv_cache(Sequence.of_length("t", 48, P), Table(), tx)
        return a, b

    def recv(rx):
        h = rx.recv_header(timeout=30)
        assert KVref.from_header(h).kv_indices == [0] and h.n_pages == 1
        oks.append(dst_w.kvhelper.recv_kv_cache(rx, [10], gpu, timeout=30))
        rx.recv_header(timeout=30)
        oks.append(dst_w.kvhelper.recv_kv_cache(rx, [20, 21, 20], gpu, timeout=30))
        torch.cuda.synchronize()

    print(f"zero fallback and repeated ids over the {ring} ring", flush=True)
    run_pair(1 << 20, 2, send, recv, RINGS[ring])
    assert oks == [True, True]
    for l in range(L):
        assert not dst_cache[l][10].any()
        assert torch.equal(words(dst_cache[l][20]), words(src_cache[l][5]))
        assert torch.equal(words(dst_cache[l][21]), words(src_cache[l][4]))


# ------------------------------------------------------- same-GPU device ring

def run_pair_device(dev_slot, send, recv, host_slot=4096, num_slots=4):
    """run_pair over a channel with a device ring; the shared-memory slots are
    4 KiB, so a payload of larger pages can only have taken the device ring."""
    nm = name()
    rx = KVChannel.create(nm, host_slot, num_slots, 2, device_slot_bytes=dev_slot)
    tx = KVChannel.open(nm, 2, timeout=10)
    assert rx.device_ring() == (dev_slot, True) and tx.device_ring() == (dev_slot, True)
    out, errs = [], []

    def sender():
        try:
            out.append(send(tx))
        except Exception as e:                     # reported below
            errs.append(repr(e))

    t = threading.Thread(target=sender)
    t.start()
    recv_err = None
    try:
        recv(rx)
    except Exception as e:                         # reported with the sender's
        recv_err = repr(e)
    finally:
        t.join(timeout=60)
        tx.close()
        rx.close()
    assert not errs and recv_err is None, f"sender: {errs}; receiver: {recv_err}"
    return out[0] if out else None


# (layers, pool pages, page shape, pages sent, device slot bytes): layer chunks,
# page chunks (a layer larger than a slot), more layers than one launch
# takes, one page, a two-slot ring
DEVICE_CASES = [(32, 64, (2, 16, 8, 128), 20, 4 << 20, 4), (4, 300, (2, 16, 8, 128), 200, 1 << 20, 4),
                (70, 16, (2, 16, 1, 64), 9, 1 << 20, 4), (2, 8, (2, 16, 8, 128), 1, 1 << 20, 4),
                (8, 128, (2, 16, 8, 128), 100, 1 << 20, 2), (16, 64, (2, 16, 8, 128), 30, 1 << 20, 8)]


@pytest.mark.parametrize("L,pages,shape,n,slot,slots", DEVICE_CASES)
def test_device_ring_in_one_process(gpu, L, pages, shape, n, slot, slots):
    print(f"device ring case L={L} pages={pages} shape={shape} n={n} slot={slot} slots={slots}", flush=True)
    src = rand_pool(L, pages, shape, torch.float16, gpu, 11)
    dst = rand_pool(L, pages, shape, torch.float16, gpu, 12)
    rng = np.random.default_rng(L + n + 1)
    s_ids = rng.permutation(pages)[:n].tolist()
    d_ids = rng.permutation(pages)[:n].tolist()
    before = [words(d).clone() for d in dst]

    def recv(rx):
        for r in range(2):                          # two messages: the ring's slots are reused
            h = rx.recv_header(timeout=30)
            assert (h.meta, h.num_layers, h.n_pages) == (f"m{r}".encode(), L, n)
            rx.recv(dst, d_ids, timeout=30)

    def send(tx):
        for r in range(2):
            tx.send(src, s_ids, f"m{r}".encode(), timeout=30)

    run_pair_device(slot, send, recv, num_slots=slots)
    torch.cuda.synchronize()
    si, di = torch.tensor(s_ids, device=gpu), torch.tensor(d_ids, device=gpu)
    keep = torch.tensor(sorted(set(range(pages)) - set(d_ids)), device=gpu, dtype=torch.long)
    for l in range(L):
        assert torch.equal(words(dst[l])[di], words(src[l])[si]), f"layer {l}"
        assert torch.equal(words(dst[l])[keep], before[l][keep]), f"layer {l} untouched pages"


def test_device_ring_to_host_discard_and_host_messages(gpu):
    """A device-slot message received into host memory, one discarded, and a
    host payload (shared-memory slots) between them, on one channel."""
    L, pages, shape, n = 5, 40, (2, 16, 8, 128), 17
    src = rand_pool(L, pages, shape, torch.bfloat16, gpu, 13)
    ids = np.random.default_rng(7).permutation(pages)[:n].tolist()
    want = torch.stack([s[torch.tensor(ids, device=gpu)] for s in src]).cpu()
    got = torch.empty((L, n) + shape, dtype=torch.bfloat16)
    back = torch.empty_like(got)

    def send(tx):
        tx.send(src, ids, b"a", timeout=30)        # device slots
        tx.send(src, ids, b"b", timeout=30)        # device slots, discarded
        tx.send_host(want, b"c", timeout=30)       # shared-memory slots

    def recv(rx):
        assert rx.recv_header(timeout=30).meta == b"a"
        rx.recv_host(got, timeout=30)
        assert rx.recv_header(timeout=30).meta == b"b"
        rx.discard(timeout=30)
        assert rx.recv_header(timeout=30).meta == b"c"
        rx.recv_host(back, timeout=30)

    run_pair_device(1 << 20, send, recv, host_slot=1 << 20)
    assert torch.equal(words(got), words(want))
    assert torch.equal(words(back), words(want))


@pytest.mark.parametrize("creator", ["sender", "receiver"])
def test_device_ring_outlives_its_creator_in_one_process(gpu, creator):
    """Two endpoints of one process share the device ring, which is freed
    when the last of them closes.  The creator closes first: as the sender,
    the message it published is still received out of the ring; as the
    receiver, a later send into the closed channel fails with
    PACE_KV_ECLOSED before it packs anything."""
    from paceserve_amd import _native

    print(f"device ring, creator = {creator}, creator closes first", flush=True)
    L, pages, shape = 3, 16, (2, 16, 8, 128)
    src = rand_pool(L, pages, shape, torch.bfloat16, gpu, 40)
    dst = rand_pool(L, pages, shape, torch.bfloat16, gpu, 41)
    before = [d.clone() for d in dst]
    s_ids, d_ids = [3, 9, 0, 15, 7], [12, 1, 4, 8, 2]
    nm = name()
    first = KVChannel.create(nm, 4096, 4, 2, device_slot_bytes=1 << 20)
    second = KVChannel.open(nm, 2, timeout=10)
    tx, rx = (first, second) if creator == "sender" else (second, first)
    try:
        # 3 layers x 5 pages x 64 KiB: one chunk in one 1 MiB device slot, so
        # the send returns once the message is in the ring
        tx.send(src, s_ids, b"m", timeout=30)
        if creator == "sender":
            first.close()
        h = rx.recv_header(timeout=30)
        assert (h.meta, h.num_layers, h.n_pages) == (b"m", L, 5)
        assert rx.device_ring() == (1 << 20, True)
        rx.recv(dst, d_ids, timeout=30)
        torch.cuda.synchronize()
        if creator == "receiver":
            first.close()
            with pytest.raises(_native.PaceKVError) as e:
                tx.send(src, [1, 2], b"late", timeout=30)
            assert e.value.status == _native.PACE_KV_ECLOSED
            torch.cuda.synchronize()
    finally:
        for ch in (first, second):
            ch.close()
    bad = workloads.migration_mismatch(src, dst, torch.tensor(s_ids, device=gpu), torch.tensor(d_ids, device=gpu),
                                       before)
    assert bad is None, bad


DEVICE_PEER = r"""
import sys, torch
sys.path.insert(0, {root!r})
from paceserve_amd import workloads
from paceserve_amd.kv_transfer.channel import KVChannel
dev = torch.device("cuda", 0)
g = torch.Generator(device=dev).manual_seed(78)
src = [torch.randn((128, 2, 16, 8, 128), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
       for _ in range(32)]
ch = KVChannel.open({name!r}, 2, timeout=60)
assert ch.device_ring() == ({dev_slot}, True), ch.device_ring()
if {role!r} == "send":
    for r in range(3):
        ids = list(range(r, 128, 3))[:40]
        ch.send(src, ids, ("request %d" % r).encode(), timeout=60)
else:
    dst = [torch.zeros_like(s) for s in src]
    for r in range(3):
        h = ch.recv_header(timeout=60)
        assert h.meta == ("request %d" % r).encode() and h.n_pages == 40, h
        ch.recv(dst, list(range(40 * r, 40 * r + 40)), timeout=60)
    torch.cuda.synchronize()
    # every page of every layer: the three requests' pages, zeros elsewhere
    bad = workloads.migration_mismatch(src, dst, torch.tensor({src_ids}, device=dev),
                                       torch.tensor({dst_ids}, device=dev), (torch.zeros_like(s) for s in src))
    assert bad is None, bad
print("peer done", flush=True)
ch.close()
"""


@pytest.mark.parametrize("peer", ["send", "recv"])
def test_device_ring_with_a_peer_process(gpu, peer):
    """The ring's creator on one side, a process that opens the exported
    ring on the other: the opener sends (its packs write the creator's
    allocation) or receives (its unpacks read it)."""
    nm = name()
    dev_slot = 4 << 20                                  # 40 pages x 64 KiB: whole layers, 4 MiB slots
    ch = KVChannel.create(nm, 4096, 4, 2, device_slot_bytes=dev_slot)
    child = subprocess.Popen([sys.executable, "-c",
                              DEVICE_PEER.format(root=str(ROOT), name=nm, dev_slot=dev_slot, role=peer,
                                                 src_ids=PEER_SRC_IDS, dst_ids=PEER_DST_IDS)])
    try:
        g = torch.Generator(device=gpu).manual_seed(78)
        src = [torch.randn((128, 2, 16, 8, 128), generator=g, device=gpu, dtype=torch.float32).to(torch.bfloat16)
               for _ in range(32)]
        dst = [torch.zeros_like(s) for s in src]
        for r in range(3):
            if peer == "send":
                h = ch.recv_header(timeout=120)
                assert h.meta == f"request {r}".encode() and h.n_pages == 40
                ch.recv(dst, list(range(40 * r, 40 * r + 40)), timeout=60)
            else:
                ch.send(src, list(range(r, 128, 3))[:40], f"request {r}".encode(), timeout=120)
        torch.cuda.synchronize()
        assert child.wait(timeout=60) == 0
    finally:
        if child.poll() is None:
            child.kill()
        ch.close()
    if peer == "send":
        assert peer_mismatch(src, dst, gpu) is None


# ------------------------------------------------------- seeded random sweep

def random_channel_case(seed):
    """A seeded channel configuration: pool shape, pages sent, slot size and
    count, and the ring (host slots, or a device ring beside 4 KiB host
    slots)."""
    rng = np.random.default_rng(5000 + seed)
    P = int(rng.choice([1, 3, 16]))
    H = int(rng.choice([1, 2, 8]))
    D = int(rng.choice([16, 64, 128]))
    shape = (2, P, H, D)
    page_bytes = 2 * P * H * D * 2
    L = int(rng.integers(1, 81))
    pages = int(rng.integers(1, 301))
    n = int(rng.integers(1, pages + 1))
    slots = int(rng.choice([2, 4, 8]))
    # slot sizes from one page (at most 2000 chunks per message) up to beyond
    # a whole layer, in 4 KiB steps
    lo = max(-(-page_bytes // 4096), -(-(L * n * page_bytes) // (2000 * 4096)))
    hi = max(lo, -(-(2 * n * page_bytes) // 4096))
    slot = 4096 * int(rng.integers(lo, hi + 1))
    slot = min(slot, (1 << 30) // slots)
    ring = "device" if seed % 2 else "host"
    return L, pages, shape, n, slot, slots, ring, rng


@pytest.mark.parametrize("seed", range(16))
def test_random_channel_messages(gpu, seed):
    L, pages, shape, n, slot, slots, ring, rng = random_channel_case(seed)
    print(f"random channel case {seed}: L={L} pages={pages} shape={shape} n={n} slot={slot} x {slots} "
          f"ring={ring}", flush=True)
    src = rand_pool(L, pages, shape, torch.float16, gpu, 30 + seed)
    dst = rand_pool(L, pages, shape, torch.float16, gpu, 60 + seed)
    before = [words(d).clone() for d in dst]
    # three messages of n pages each into disjoint destination pages where
    # the pool has room for them, else into the same ones (the last wins)
    msgs = []
    for m in range(3):
        s_ids = rng.permutation(pages)[:n].tolist()
        d_ids = rng.permutation(pages)[:n].tolist()
        msgs.append((s_ids, d_ids))

    # page ids alternate between host lists (carried in the kernel arguments)
    # and device tensors, on both sides
    def as_ids(ids, i):
        return ids if (i + seed) % 2 == 0 else torch.tensor(ids, dtype=torch.int32, device=gpu)

    def send(tx):
        return [tx.send(src, as_ids(s, i), f"m{i}".encode(), timeout=30) for i, (s, _) in enumerate(msgs)]

    def recv(rx):
        for i, (_, d) in enumerate(msgs):
            h = rx.recv_header(timeout=30)
            assert (h.meta, h.num_layers, h.n_pages) == (f"m{i}".encode(), L, n)
            rx.recv(dst, as_ids(d, i + 1), timeout=30)
        torch.cuda.synchronize()

    if ring == "device":
        run_pair_device(slot, send, recv, num_slots=slots)
    else:
        run_pair(slot, slots, send, recv)
    # the expected destination: torch's scatter of torch's gather, message by message
    want = [b.clone() for b in before]
    for s_ids, d_ids in msgs:
        si, di = torch.tensor(s_ids, device=gpu), torch.tensor(d_ids, device=gpu)
        for l in range(L):
            want[l][di] = words(src[l])[si]
    for l in range(L):
        assert torch.equal(words(dst[l]), want[l]), f"layer {l}"


@pytest.mark.parametrize("ring", RINGS)
def test_host_page_ids_beyond_the_inline_limit(gpu, ring):
    """Through the C ABI, more than 512 page ids in host memory are refused
    with PACE_KV_ERANGE before anything is sent; through KVChannel the same
    ids go up to the device instead, and arrive."""
    from paceserve_amd import _native

    L, pages, shape, n = 2, 700, (2, 16, 1, 64), 600
    src = rand_pool(L, pages, shape, torch.float16, gpu, 50)
    dst = rand_pool(L, pages, shape, torch.float16, gpu, 51)
    before = [d.clone() for d in dst]
    s_ids = np.random.default_rng(50).permutation(pages)[:n].tolist()
    d_ids = np.random.default_rng(51).permutation(pages)[:n].tolist()
    refused = []

    def send(tx):
        lib = _native.load()
        pool = ops.PagedPool(src)
        host = np.ascontiguousarray(s_ids, dtype=np.int32)
        rc = lib.pace_kv_channel_send(tx._require(), pool.table(), L, pages, host.ctypes.data, n, pool.page_bytes,
                                      None, 0, 1000, None, torch.cuda.current_stream(gpu).cuda_stream)
        refused.append((rc, lib.pace_kv_last_error()))
        tx.send(src, s_ids, b"m", timeout=30)               # uploaded by KVChannel

    def recv(rx):
        h = rx.recv_header(timeout=30)
        assert (h.meta, h.n_pages) == (b"m", n)
        rx.recv(dst, d_ids, timeout=30)
        torch.cuda.synchronize()

    run_pair(1 << 20, 4, send, recv, RINGS[ring])
    assert refused[0][0] == _native.PACE_KV_ERANGE and b"at most 512" in refused[0][1], refused
    bad = workloads.migration_mismatch(src, dst, torch.tensor(s_ids, device=gpu), torch.tensor(d_ids, device=gpu),
                                       before)
    assert bad is None, bad
