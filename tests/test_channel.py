"""The cross-process channel's protocol on host payloads (no GPU): messages in
order with their metadata, payloads larger than the ring streaming through
it, layer- and page-sized chunks, another process as the sender, deadlines,
closing, abandoned messages, draining, threads sharing an endpoint message by
message, a peer process that dies mid-message, and argument errors."""
import ctypes
import os
import subprocess
import sys
import threading
import time
from pathlib import Path

import numpy as np
import pytest
import torch

from paceserve_amd import _native
from paceserve_amd.kv_transfer.channel import KVChannel, KVref, MessageHeader

ROOT = Path(__file__).resolve().parent.parent
_count = [0]


def name():
    _count[0] += 1
    return f"pace_test_{os.getpid()}_{_count[0]}"


def status(excinfo):
    return excinfo.value.status


def payload(L, n, page_shape, seed, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn((L, n) + tuple(page_shape), generator=g).to(dtype)


def pair(slot_bytes=64 << 10, num_slots=4, threads=4):
    nm = name()
    rx = KVChannel.create(nm, slot_bytes, num_slots, threads)
    tx = KVChannel.open(nm, threads, timeout=5)
    return tx, rx


# (L, n, page_shape): page chunks (a layer is larger than a 64 KiB slot),
# layer chunks, a single page, more layers than one launch takes
SHAPES = [(3, 40, (2, 16, 1, 64)), (8, 5, (2, 4, 2, 16)), (1, 1, (2, 1, 1, 8)), (70, 3, (2, 2, 1, 8))]


def test_messages_arrive_in_order_with_their_metadata():
    tx, rx = pair()
    sent = [(payload(L, n, ps, i), f"msg {i}".encode()) for i, (L, n, ps) in enumerate(SHAPES)]
    ids = []

    def send():
        for p, m in sent:
            ids.append(tx.send_host(p, m, timeout=10))

    t = threading.Thread(target=send)
    t.start()
    got = []
    for p, m in sent:
        h = rx.recv_header(timeout=10)
        assert h.meta == m and (h.num_layers, h.n_pages) == tuple(p.shape[:2])
        assert h.page_bytes == p[0, 0].numel() * 2
        out = torch.empty_like(p)
        rx.recv_host(out, timeout=10)
        got.append((h.msg_id, out))
    t.join()
    assert [g[0] for g in got] == ids == sorted(ids)
    for (p, _), (_, out) in zip(sent, got):
        assert torch.equal(p.view(torch.int16), out.view(torch.int16))
    tx.close()
    rx.close()


def test_payload_larger_than_the_ring_streams_through_it():
    tx, rx = pair(slot_bytes=4096, num_slots=2)
    p = payload(4, 300, (2, 4, 1, 16), 7)          # 300 pages of 256 B per layer: 19 page chunks per layer
    assert p.numel() * 2 > 20 * rx.slot_bytes * rx.num_slots
    t = threading.Thread(target=lambda: tx.send_host(p, b"big", timeout=10))
    t.start()
    h = rx.recv_header(timeout=10)
    out = torch.empty_like(p)
    rx.recv_host(out, timeout=10)
    t.join()
    assert h.meta == b"big" and torch.equal(out.view(torch.int16), p.view(torch.int16))
    tx.close()
    rx.close()


SENDER = r"""
import sys, torch
sys.path.insert(0, {root!r})
from paceserve_amd.kv_transfer.channel import KVChannel
ch = KVChannel.open({name!r}, 4, timeout=30)
for i in range(5):
    g = torch.Generator().manual_seed(100 + i)
    p = torch.randint(0, 256, (6, 7 + i, 2, 4, 1, 16), generator=g, dtype=torch.uint8)
    ch.send_host(p, ("from child %d" % i).encode(), timeout=30)
ch.close()
"""


def test_another_process_sends():
    nm = name()
    rx = KVChannel.create(nm, 8192, 4, 4)
    child = subprocess.Popen([sys.executable, "-c", SENDER.format(root=str(ROOT), name=nm)])
    try:
        for i in range(5):
            h = rx.recv_header(timeout=60)
            assert h.meta == f"from child {i}".encode()
            out = torch.empty((6, 7 + i, 2, 4, 1, 16), dtype=torch.uint8)
            rx.recv_host(out, timeout=60)
            g = torch.Generator().manual_seed(100 + i)
            assert torch.equal(out, torch.randint(0, 256, out.shape, generator=g, dtype=torch.uint8))
        assert child.wait(timeout=60) == 0
    finally:
        if child.poll() is None:
            child.kill()
        rx.close()


def test_waits_end_at_their_deadline():
    tx, rx = pair()
    t0 = time.monotonic()
    with pytest.raises(_native.PaceKVError) as e:
        rx.recv_header(timeout=0.2)
    assert status(e) == _native.PACE_KV_ETIMEDOUT
    assert 0.15 < time.monotonic() - t0 < 5
    # a full ring: the sender's wait for a free slot ends too
    with pytest.raises(_native.PaceKVError) as e:
        tx.send_host(payload(4, 40, (2, 16, 1, 64), 1), timeout=0.2)
    assert status(e) == _native.PACE_KV_ETIMEDOUT
    tx.close()
    rx.close()


def test_closing_wakes_the_peer():
    tx, rx = pair()
    seen = []

    def wait():
        try:
            rx.recv_header(timeout=30)
        except _native.PaceKVError as exc:
            seen.append(exc.status)

    t = threading.Thread(target=wait)
    t.start()
    time.sleep(0.2)
    tx.close()
    t.join(timeout=10)
    assert seen == [_native.PACE_KV_ECLOSED]
    rx.close()


def test_abandoned_message_fails_the_receiver_and_the_channel_recovers():
    tx, rx = pair(slot_bytes=4096, num_slots=2)
    big = payload(2, 64, (2, 4, 1, 16), 3)         # 16 chunks through 2 slots
    h = None
    errs = []

    def send():
        try:
            tx.send_host(big, b"big", timeout=0.3)
        except _native.PaceKVError as exc:
            errs.append(exc.status)

    t = threading.Thread(target=send)
    t.start()
    h = rx.recv_header(timeout=10)
    assert h.meta == b"big"
    t.join(timeout=10)                               # the receiver took nothing: the sender gave up
    assert errs == [_native.PACE_KV_ETIMEDOUT]
    with pytest.raises(_native.PaceKVError) as e:
        rx.recv_host(torch.empty_like(big), timeout=5)
    assert status(e) == _native.PACE_KV_ESTATE and "abandoned" in str(e.value)
    # the chunks already in the ring are skipped; the next message arrives whole
    small = payload(1, 2, (2, 4, 1, 16), 4)
    t = threading.Thread(target=lambda: tx.send_host(small, b"next", timeout=10))
    t.start()
    h = rx.recv_header(timeout=10)
    out = torch.empty_like(small)
    rx.recv_host(out, timeout=10)
    t.join()
    assert h.meta == b"next" and torch.equal(out.view(torch.int16), small.view(torch.int16))
    tx.close()
    rx.close()


def test_message_context_reports_the_receive_error():
    # An abandoned message taken with message(): the caller sees the
    # receive's own error (the sender abandoned the message), not one from
    # the clean-up drain, and the endpoint then takes the next message.
    tx, rx = pair(slot_bytes=4096, num_slots=2)
    big = payload(2, 64, (2, 4, 1, 16), 3)         # 16 chunks through 2 slots
    errs = []

    def send():
        try:
            tx.send_host(big, b"big", timeout=0.3)
        except _native.PaceKVError as exc:
            errs.append(exc.status)

    t = threading.Thread(target=send)
    t.start()
    with pytest.raises(_native.PaceKVError) as e:
        with rx.message(timeout=10) as h:
            assert h.meta == b"big"
            t.join(timeout=10)                       # the sender gives up
            rx.recv_host(torch.empty_like(big), timeout=5)
    assert errs == [_native.PACE_KV_ETIMEDOUT]
    assert status(e) == _native.PACE_KV_ESTATE and "abandoned" in str(e.value)
    small = payload(1, 2, (2, 4, 1, 16), 4)
    t = threading.Thread(target=lambda: tx.send_host(small, b"next", timeout=10))
    t.start()
    with rx.message(timeout=10) as h:
        out = rx.recv_host(torch.empty_like(small), timeout=10)
    t.join()
    assert h.meta == b"next" and torch.equal(out.view(torch.int16), small.view(torch.int16))
    tx.close()
    rx.close()


def test_discarded_payload_leaves_the_next_message_intact():
    tx, rx = pair(slot_bytes=4096, num_slots=2)
    a, b = payload(3, 30, (2, 4, 1, 16), 5), payload(2, 3, (2, 4, 1, 16), 6)

    def send():
        tx.send_host(a, b"a", timeout=10)
        tx.send_host(b, b"b", timeout=10)

    t = threading.Thread(target=send)
    t.start()
    assert rx.recv_header(timeout=10).meta == b"a"
    rx.discard(timeout=10)
    assert rx.recv_header(timeout=10).meta == b"b"
    out = torch.empty_like(b)
    rx.recv_host(out, timeout=10)
    t.join()
    assert torch.equal(out.view(torch.int16), b.view(torch.int16))
    tx.close()
    rx.close()


def test_large_metadata_and_empty_payload():
    tx, rx = pair(slot_bytes=256 << 10)
    ref = KVref("seq-9", list(range(20000)), 1.5, 3.0, 4.0)
    meta = ref.meta()
    assert len(meta) > 64 << 10                      # more than recv_header's first buffer
    tx.send_host(torch.empty((0, 0, 2, 4, 1, 16), dtype=torch.float16), meta, timeout=5)
    h = rx.recv_header(timeout=5)
    assert h.payload_bytes == 0
    back = KVref.from_header(h)
    assert (back.seq_id, back.kv_indices, back.size, back.msg_id) == ("seq-9", ref.kv_indices, 1.5, h.msg_id)
    with pytest.raises(RuntimeError):
        rx.recv_host(torch.empty(1))               # nothing pending
    tx.close()
    rx.close()


def test_argument_errors():
    lib = _native.load()
    h = __import__("ctypes").c_void_p()
    for bad_name in (b"", b"a/b", b"x" * 300):
        assert lib.pace_kv_channel_create(bad_name, 4096, 2, 1, __import__("ctypes").byref(h)) == _native.PACE_KV_EINVAL
    nm = name()
    for slot, slots, thr in ((100, 2, 1), (4096, 1, 1), (4096, 3, 1), (4096, 48, 1), (4096, 128, 1), (4096, 2, 0)):
        with pytest.raises(_native.PaceKVError) as e:
            KVChannel.create(nm, slot, slots, thr)
        assert status(e) == _native.PACE_KV_EINVAL
    rx = KVChannel.create(nm, 4096, 2, 1)
    with pytest.raises(_native.PaceKVError) as e:
        KVChannel.create(nm, 4096, 2, 1)
    assert status(e) == _native.PACE_KV_ESTATE
    with pytest.raises(_native.PaceKVError) as e:
        KVChannel.open(name() + "_missing", 1, timeout=0)
    assert status(e) == _native.PACE_KV_ETIMEDOUT
    tx = KVChannel.open(nm, 1, timeout=5)
    with pytest.raises(_native.PaceKVError) as e:
        tx.send_host(payload(1, 1, (2, 4, 1, 16), 0), b"m" * 5000, timeout=1)   # metadata > slot
    assert status(e) == _native.PACE_KV_ERANGE
    with pytest.raises(_native.PaceKVError) as e:
        tx.send_host(payload(1, 1, (2, 64, 1, 64), 0), timeout=1)               # page > slot
    assert status(e) == _native.PACE_KV_ERANGE
    assert lib.pace_kv_channel_recv_host(rx._handle, None, 0, 0) == _native.PACE_KV_ESTATE   # no header
    tx.send_host(payload(2, 2, (2, 4, 1, 16), 0), timeout=1)
    rx.recv_header(timeout=1)
    assert lib.pace_kv_channel_recv_header(rx._handle, None, 0, None, None, None, None, None, 0) == \
        _native.PACE_KV_ESTATE                                                   # payload pending
    out = torch.empty((2, 3, 2, 4, 1, 16), dtype=torch.float16)
    assert lib.pace_kv_channel_recv_host(rx._handle, out.data_ptr(), out.numel() * 2, 0) == _native.PACE_KV_EINVAL
    rx.discard(timeout=1)
    tx.close()
    rx.close()
    assert not os.path.exists(f"/dev/shm/{nm}")                                  # the creator unlinked it


def test_unlink_clears_a_name_left_behind():
    nm = name()
    first = KVChannel.create(nm, 4096, 2, 1)
    with pytest.raises(_native.PaceKVError):
        KVChannel.create(nm, 4096, 2, 1)
    KVChannel.unlink(nm)                       # as after a creator that died
    second = KVChannel.create(nm, 4096, 2, 1)  # a fresh channel under the same name
    KVChannel.unlink(nm + "_never_created")    # not an error
    first.close()                              # the name is second's now: first leaves it
    assert os.path.exists(f"/dev/shm/{nm}")
    third = KVChannel.open(nm, 1, timeout=5)   # and it still opens second's ring
    assert third.slot_bytes == 4096
    third.close()
    second.close()
    assert not os.path.exists(f"/dev/shm/{nm}")


def test_record_counters_wrap_at_2_32():
    # The control block counts records in two 32-bit words (head at byte 64,
    # tail at byte 128, pinned by a static_assert in the library).  Starting
    # both just below 2^32, a stream of multi-chunk messages crosses the wrap
    # with every payload intact and in order.
    import mmap
    import struct

    tx, rx = pair(slot_bytes=4096, num_slots=4)
    start = (1 << 32) - 6
    with open(f"/dev/shm/{rx.name}", "r+b") as f:
        m = mmap.mmap(f.fileno(), 4096)
        struct.pack_into("<I", m, 64, start)
        struct.pack_into("<I", m, 128, start)
        sent = [payload(2, 20 + i, (2, 4, 1, 16), 70 + i) for i in range(6)]  # 4 page chunks each
        t = threading.Thread(target=lambda: [tx.send_host(p, b"w%d" % i, timeout=10) for i, p in enumerate(sent)])
        t.start()
        for i, p in enumerate(sent):
            h = rx.recv_header(timeout=10)
            assert h.meta == b"w%d" % i
            out = torch.empty_like(p)
            rx.recv_host(out, timeout=10)
            assert torch.equal(out.view(torch.int16), p.view(torch.int16)), f"message {i}"
        t.join()
        head, tail = struct.unpack_from("<I", m, 64)[0], struct.unpack_from("<I", m, 128)[0]
        m.close()
    assert head == tail and head < 64          # both counters wrapped past 2^32
    tx.close()
    rx.close()


def test_open_refuses_a_slot_count_that_is_not_a_power_of_two():
    # The opener checks the control block too: a ring whose num_slots (byte
    # 12) is not a power of two is refused as incompatible.
    import mmap
    import struct

    nm = name()
    rx = KVChannel.create(nm, 4096, 4, 1)
    with open(f"/dev/shm/{nm}", "r+b") as f:
        m = mmap.mmap(f.fileno(), 4096)
        assert struct.unpack_from("<I", m, 12)[0] == 4
        struct.pack_into("<I", m, 12, 3)
        m.close()
    with pytest.raises(_native.PaceKVError) as e:
        KVChannel.open(nm, 1, timeout=1)
    assert status(e) == _native.PACE_KV_ESTATE and "incompatible" in str(e.value)
    rx.close()


def test_threads_share_an_endpoint_message_by_message():
    # Four receiving threads take whole messages from one endpoint with
    # message(); every message arrives exactly once, whole.
    tx, rx = pair(slot_bytes=4096, num_slots=8)
    sent = {f"m{i}".encode(): payload(2, 3 + i, (2, 4, 1, 16), 50 + i) for i in range(12)}
    got, errors = {}, []

    def receive():
        try:
            while True:
                with rx.message(timeout=10) as h:
                    if h.meta == b"stop":
                        return
                    out = torch.empty((h.num_layers, h.n_pages, 2, 4, 1, 16), dtype=torch.float16)
                    rx.recv_host(out, timeout=10)
                    got[h.meta] = out
        except Exception as e:                         # reported below
            errors.append(repr(e))

    ts = [threading.Thread(target=receive) for _ in range(4)]
    for t in ts:
        t.start()
    for m, p in sent.items():
        tx.send_host(p, m, timeout=10)
    for _ in ts:
        tx.send_host(torch.empty((0, 0, 2, 4, 1, 16), dtype=torch.float16), b"stop", timeout=10)
    for t in ts:
        t.join(timeout=30)
    assert not errors, errors
    assert sorted(got) == sorted(sent)
    for m, p in sent.items():
        assert torch.equal(got[m].view(torch.int16), p.view(torch.int16)), m
    tx.close()
    rx.close()


def test_message_drains_a_payload_left_unreceived():
    tx, rx = pair(slot_bytes=4096, num_slots=2)
    a, b = payload(2, 20, (2, 4, 1, 16), 7), payload(1, 2, (2, 4, 1, 16), 8)

    def send():
        tx.send_host(a, b"a", timeout=10)
        tx.send_host(b, b"b", timeout=10)

    t = threading.Thread(target=send)
    t.start()
    with rx.message(timeout=10) as h:
        assert h.meta == b"a"                          # payload not taken: drained on exit
    with rx.message(timeout=10) as h:
        out = torch.empty_like(b)
        rx.recv_host(out, timeout=10)
    t.join()
    assert h.meta == b"b" and torch.equal(out.view(torch.int16), b.view(torch.int16))
    tx.close()
    rx.close()


def test_kvref_round_trips_the_kvobj_fields():
    r = KVref(17, [5, 3, 9], 2.25, 1.0, 2.0, 0)
    h = MessageHeader(42, r.meta(), 32, 3, 65536)
    b = KVref.from_header(h)
    assert (b.seq_id, b.kv_indices, b.size, b.left_prefill, b.kv_transfer_start, b.msg_id) == \
        (17, [5, 3, 9], 2.25, 1.0, 2.0, 42)


STALLED_SENDER = r"""
import sys, torch
sys.path.insert(0, {root!r})
from paceserve_amd.kv_transfer.channel import KVChannel
ch = KVChannel.open({name!r}, 1, timeout=30)
ch.send_host(torch.zeros((2, 64, 2, 4, 1, 16), dtype=torch.float16), b"big", timeout=120)
"""

STALLED_RECEIVER = r"""
import sys, time
sys.path.insert(0, {root!r})
from paceserve_amd.kv_transfer.channel import KVChannel
ch = KVChannel.open({name!r}, 1, timeout=30)
ch.recv_header(timeout=120)
print("got", flush=True)
time.sleep(120)
"""


def test_a_dead_sender_ends_the_receivers_wait():
    nm = name()
    rx = KVChannel.create(nm, 4096, 2, 1)
    child = subprocess.Popen([sys.executable, "-c", STALLED_SENDER.format(root=str(ROOT), name=nm)])
    try:
        h = rx.recv_header(timeout=60)
        assert h.meta == b"big"
        child.kill()                                  # a zombie until reaped: still counts as exited
        t0 = time.monotonic()
        with pytest.raises(_native.PaceKVError) as e:
            rx.recv_host(torch.empty((2, 64, 2, 4, 1, 16), dtype=torch.float16), timeout=60)
        assert status(e) == _native.PACE_KV_ECLOSED and "exited" in str(e.value)
        assert time.monotonic() - t0 < 5
    finally:
        child.kill()
        child.wait()
        rx.close()


def test_a_dead_receiver_ends_the_senders_wait():
    nm = name()
    tx = KVChannel.create(nm, 4096, 2, 1)
    child = subprocess.Popen([sys.executable, "-c", STALLED_RECEIVER.format(root=str(ROOT), name=nm)],
                             stdout=subprocess.PIPE, text=True)
    errs = []

    def send():
        try:
            tx.send_host(torch.zeros((2, 64, 2, 4, 1, 16), dtype=torch.float16), b"big", timeout=60)
        except _native.PaceKVError as exc:
            errs.append(exc)

    t = threading.Thread(target=send)
    try:
        t.start()
        assert child.stdout.readline().strip() == "got"
        t0 = time.monotonic()
        child.kill()
        t.join(timeout=30)
        assert len(errs) == 1 and errs[0].status == _native.PACE_KV_ECLOSED and "exited" in str(errs[0])
        assert time.monotonic() - t0 < 5
    finally:
        child.kill()
        child.wait()
        t.join(timeout=30)
        tx.close()


def test_device_ring_arguments_are_checked_before_any_device_call():
    """Bad device-ring sizes are refused before the shared object or any HIP
    call (this runs without a GPU)."""
    lib = _native.load()
    h = ctypes.c_void_p()
    nm = f"pace_dev_args_{os.getpid()}".encode()
    assert lib.pace_kv_channel_create_device(nm, 4096, 4, 1, 0, ctypes.byref(h)) == _native.PACE_KV_EINVAL
    assert lib.pace_kv_channel_create_device(nm, 4096, 4, 1, 1000, ctypes.byref(h)) == _native.PACE_KV_EINVAL
    assert lib.pace_kv_channel_create_device(nm, 4096, 4, 1, 512 << 20, ctypes.byref(h)) == _native.PACE_KV_ERANGE
    assert b"exceeds 1073741824 bytes" in lib.pace_kv_last_error()
    assert not os.path.exists(f"/dev/shm/{nm.decode()}")


def test_host_channel_reports_no_device_ring():
    ch = KVChannel.create(f"pace_nodev_{os.getpid()}", 4096, 2, 1)
    try:
        assert ch.device_ring() == (0, False)
    finally:
        ch.close()


def test_host_page_ids_become_int32_arrays_for_the_kernel_arguments():
    """Block tables of at most 512 ids in host memory reach the library as
    int32 numpy arrays (the kernels carry them in their arguments and skip
    out-of-pool ids, as they do device ids); repeated destination ids and
    values beyond int32 are refused before any device call."""
    from paceserve_amd.kv_transfer import channel as chan

    dev = torch.device("cpu")              # not touched on the host path
    ids = chan._ids([5, 3, -1, 2**31 - 1], dev)
    assert isinstance(ids, np.ndarray) and ids.dtype == np.int32 and ids.tolist() == [5, 3, -1, 2**31 - 1]
    assert chan._count(ids) == 4 and chan._ptr(ids) == ids.ctypes.data
    t = chan._ids(torch.tensor([7, 1, 4], dtype=torch.int64), dev)
    assert t.dtype == np.int32 and t.tolist() == [7, 1, 4]
    assert chan._ids(list(range(chan.HOST_IDS_MAX)), dev).size == chan.HOST_IDS_MAX
    with pytest.raises(ValueError, match="appears more than once"):
        chan._ids([3, 9, 3], dev, distinct=True)
    assert chan._ids([3, 9, 3], dev).tolist() == [3, 9, 3]      # source ids may repeat
    with pytest.raises(ValueError, match="int32"):
        chan._ids([2**31], dev)
    assert chan._count(chan._ids([], dev)) == 0
