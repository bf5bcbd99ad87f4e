"""Benchmark of the KV-cache migration hot path on one MI355X.

Default workload (N=1): llama3-70b-256req-bf16, the largest of the five
migration workloads and one that fits one GPU - 256 requests of U{64..2048}
tokens at the Llama-3-70B KV shape (80 layers, 8 KV heads, head_dim 128, page
16), bf16, 20480-page source and destination pools with the source pages dealt
to requests round-robin (heavily fragmented), moved in 8-layer chunks.  One
step = pack every request's pages from all layers into the contiguous transfer
buffer, then unpack the buffer into the destination pages (the reference's
get_kv_cache + insert_kv_cache, moved on-device).

value = 4 * payload / elapsed, in GB/s (1e9 B/s): pack reads and writes the
payload, unpack reads and writes it; elapsed is measured with HIP events on
the stream the kernels run on, over the K timed steps.  Inputs are resident in
HBM before timing starts.  After the timed steps every layer of both pools is
compared byte for byte with torch's own gather/scatter of the same pages
(`verified`).  Also reported: the roofline of the copy kernel (algorithmic
bytes per launch / mean launch time vs 8 TB/s), the other four workloads and
one GPU's share of the 70B workload at tensor parallelism 8 in the same
process (`configs`: GB/s, fraction of peak and the same exact check; the
pinned-host legs of the two that have one, `staging`, run first in the
process and again at its end, `staging_warm`), p50/p90 promote latency
of one 4096-token request (dst allocation + remap + block-table H2D + pack +
unpack, to completion; also timed from C) and the reference's CPU path (torch
index_select / index_copy_ on host tensors) timed on a bounded sample on this
host's cores.

Usage: python bench.py [--steps K] [--warmup W] [--workload NAME]
       [--no-cpu] [--no-promote] [--no-verify] [--no-configs] ...
(NAME: one of paceserve_amd.workloads.NAMES or SHARDS; see that module and
--help for the other legs' switches)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from array import array
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "KV pack+unpack GB/s (% of HBM peak); p50 promote latency, 4k-token request"
HBM_PEAK_GBS = 8000.0
# The path copies pages as raw bytes; dtype names the cache's element type.
DTYPE_NAMES = {"bfloat16": "bf16", "float16": "fp16", "float32": "fp32"}
INIT_NAMES = {"normal": "N(0,1)", "uniform4": "U[-4,4]"}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    from paceserve_amd import workloads

    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default=workloads.DEFAULT, choices=workloads.NAMES + workloads.SHARDS)
    ap.add_argument("--mode", default="buffer", choices=["buffer", "fused"],
                    help="buffer: pack + unpack (the metric); fused: pool-to-pool move")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-promote", action="store_true")
    ap.add_argument("--no-verify", dest="verify", action="store_false",
                    help="skip the exact check of both pools against torch's gather/scatter")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other workloads (timed, checked and, where they have one, staged after the "
                         "headline workload)")
    ap.add_argument("--cpu-layers", type=int, default=0, help="layers in the CPU sample (0 = auto)")
    ap.add_argument("--calibrate", action="store_true",
                    help="after timing, run torch's contiguous copy of 1 GiB three times (PMC scale reference)")
    ap.add_argument("--staging", action="store_true",
                    help="also time the pinned-host round trip (default for workloads 3 and 4)")
    ap.add_argument("--no-warm-staging", action="store_true",
                    help="skip the second run of the pinned-host legs at the end of the process")
    ap.add_argument("--no-staging", action="store_true",
                    help="skip the pinned-host round trip, also for workloads 3 and 4")
    ap.add_argument("--no-append", action="store_true",
                    help="skip timing the paged-append producer kernel")
    ap.add_argument("--no-channel", action="store_true",
                    help="skip timing the cross-process channel (4096-token request between two processes)")
    ap.add_argument("--no-c-caller", action="store_true",
                    help="skip timing the promote from C (tests/c_abi/pace_kv_promote_latency, a child process); "
                         "for runs under a tracer, whose trace should hold this process's launches only")
    ap.add_argument("--no-dropin", action="store_true",
                    help="skip timing KVhelper get_kv_cache + insert_kv_cache against the reference's torch "
                         "code for the same calls (4096-token request)")
    return ap.parse_args()


def device_setup(w, dev):
    import torch

    from paceserve_amd.core.block_manager import BlockAllocator
    from paceserve_amd.kv_transfer import migrate, ops

    src = w.src_pool(dev)
    dst = w.dst_pool(dev)
    alloc = BlockAllocator(w.shape.page_size, w.dst_pool_pages, w.dst_free)
    plan = migrate.plan_batch(w.src_tables, w.src_pool_pages, alloc)
    s_ids = torch.tensor(plan.src_ids, dtype=torch.int32, device=dev)
    d_ids = torch.tensor(plan.dst_ids, dtype=torch.int32, device=dev)
    return ops.PagedPool(src), ops.PagedPool(dst), plan, s_ids, d_ids


def run_device(args, w, dev, src, dst, plan, s_ids, d_ids):
    """Times K steps of pack + unpack (or fused move) with HIP events.

    Two passes of K steps each, on the stream the kernels run on:
      - the timed steps (`value` and `roofline`): one event before the first
        step and one after the last, nothing recorded between launches; the
        mean launch duration is that span over the launches it holds;
      - the launch-timing steps (pack / unpack split only): an event before
        every launch and one after the last, so each launch's duration is the
        time between its event and the next.  Each event recorded between two
        launches adds ~3 us on MI355X, which a 20 us launch cannot hide, so
        these events stay out of the timed steps.
    """
    import torch

    from paceserve_amd.kv_transfer import ops

    L = w.shape.num_layers
    n = plan.n_pages
    k = w.device_layers_per_chunk or L
    buf = torch.empty((min(k, L), n) + w.shape.page_shape, dtype=w.shape.dtype, device=dev)
    stream = torch.cuda.current_stream(dev)

    chunks = -(-L // k)
    launches = args.steps * chunks * (1 if args.mode == "fused" else 2)
    # Events are created (first record) before the launch-timing pass, so the
    # pass enqueues launches faster than the GPU runs them even for 20 us
    # launches; creating an event inside the loop would starve the GPU.
    pool = [torch.cuda.Event(enable_timing=True) for _ in range(launches + 1)]
    for e in pool:
        e.record(stream)
    torch.cuda.synchronize()
    pool.reverse()

    def mark(evs, kind, layers):
        if evs is not None:
            ev = pool.pop()
            ev.record(stream)
            evs.append((kind, layers, ev))

    def step(evs=None):
        for lb in range(0, L, k):
            le = min(L, lb + k)
            if args.mode == "fused":
                mark(evs, "move", le - lb)
                ops.move(src, s_ids, dst, d_ids, layer_begin=lb, layer_end=le)
            else:
                b = buf[: le - lb]
                mark(evs, "pack", le - lb)
                ops.pack(src, s_ids, b, layer_begin=lb, layer_end=le)
                mark(evs, "unpack", le - lb)
                ops.unpack(b, dst, d_ids, layer_begin=lb, layer_end=le)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"{w.name}: {n} pages x {L} layers, payload {w.payload_bytes / 2**30:.3f} GiB; warmup done")

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    elapsed_ms = start.elapsed_time(end)

    # Launch-timing pass.
    evs = []
    for _ in range(args.steps):
        step(evs)
    mark(evs, "end", 0)
    torch.cuda.synchronize()
    timed_ms = evs[0][2].elapsed_time(evs[-1][2])
    launch_ms = {"pack": [], "unpack": [], "move": []}
    launch_layers = {"pack": [], "unpack": [], "move": []}
    for (kind, layers, ev), (_, _, nxt) in zip(evs[:-1], evs[1:]):
        if kind in launch_ms:
            launch_ms[kind].append(ev.elapsed_time(nxt))
            launch_layers[kind].append(layers)

    traffic_factor = 2 if args.mode == "fused" else 4
    value = traffic_factor * w.payload_bytes * args.steps / (elapsed_ms / 1e3) / 1e9
    kinds = ["move"] if args.mode == "fused" else ["pack", "unpack"]
    durs = [d for kd in kinds for d in launch_ms[kd]]
    lays = [x for kd in kinds for x in launch_layers[kd]]
    # Algorithmic bytes per launch: read + write of its layers' pages.  The
    # mean launch duration is the timed region over the launches it holds:
    # launches follow each other on one stream with no gap, and no event
    # sits between them (the launch-timing pass's durations each carry one
    # event's overhead, so they only split the step into pack and unpack).
    bytes_per_launch = [2 * x * n * w.shape.page_bytes for x in lays]
    launches_per_step = len(durs) // args.steps
    mean_launch_ms = elapsed_ms / (args.steps * launches_per_step)
    achieved = (sum(bytes_per_launch) / len(bytes_per_launch)) / (mean_launch_ms / 1e3) / 1e9
    res = {
        "value": value,
        "elapsed_ms": elapsed_ms,
        "ms_per_step": wall * 1e3 / args.steps,
        "event_ms_per_step": elapsed_ms / args.steps,
        "pack_ms_mean": statistics.mean(launch_ms["pack"]) if launch_ms["pack"] else None,
        "unpack_ms_mean": statistics.mean(launch_ms["unpack"]) if launch_ms["unpack"] else None,
        "move_ms_mean": statistics.mean(launch_ms["move"]) if launch_ms["move"] else None,
        "launches_per_step": launches_per_step,
        "launch_timing_ms_per_step": timed_ms / args.steps,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": copy_kernel_names(args.mode, w.shape.page_bytes),
            "algorithmic_bytes_per_launch": int(statistics.mean(bytes_per_launch)),
            # page ids read per launch (one int32 per page; not in `achieved`)
            "block_table_bytes_per_launch": 4 * n,
            "mean_launch_us": round(mean_launch_ms * 1e3, 2),
            "launch_timing": "HIP events around the K timed steps on the launch stream, divided by "
                             "the launches they hold",
            "evented_launch_us": round(statistics.mean(durs) * 1e3, 2),
            "launches_per_step": launches_per_step,
        },
    }
    return res


def copy_kernel_names(mode: str, page_bytes: int) -> str:
    """The page_copy_kernel instances a step launches (template arguments
    GUARD = page not a multiple of 1 KiB rows, PACK = the pack's cacheable
    write-through stores rather than streaming ones, POW2 = a power-of-two
    number of rows per page)."""
    guard = "true" if page_bytes % 1024 else "false"
    rows = -(-page_bytes // 1024)
    pow2 = "true" if rows & (rows - 1) == 0 else "false"

    def k(pack: str) -> str:
        return f"page_copy_kernel<{guard}, {pack}, {pow2}>"

    if mode == "fused":
        return f"{k('false')} (move, streaming write-through stores)"
    return f"{k('true')} (pack, write-through stores) and {k('false')} (unpack, streaming write-through stores)"


def run_ceiling(w, dev, src, dst, n: int, reps: int = 10) -> dict:
    """The same kernel with identity page ids (pages 0..n-1 of each pool, so
    both sides are contiguous): the device's copy ceiling for this kernel and
    payload, measured beside the indexed run."""
    import torch

    from paceserve_amd.kv_transfer import ops

    L = w.shape.num_layers
    k = w.device_layers_per_chunk or L
    ids = torch.arange(n, dtype=torch.int32, device=dev)
    buf = torch.empty((min(k, L), n) + w.shape.page_shape, dtype=w.shape.dtype, device=dev)
    stream = torch.cuda.current_stream(dev)

    def step():
        for lb in range(0, L, k):
            le = min(L, lb + k)
            ops.pack(src, ids, buf[: le - lb], layer_begin=lb, layer_end=le)
            ops.unpack(buf[: le - lb], dst, ids, layer_begin=lb, layer_end=le)

    step()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        step()
    b.record(stream)
    torch.cuda.synchronize()
    gbs = 4 * w.payload_bytes * reps / (a.elapsed_time(b) / 1e3) / 1e9
    log(f"contiguous ceiling (identity ids): {gbs:.1f} GB/s")
    # The runtime's own device copy (torch copy_ -> hipMemcpyAsync, a blit
    # kernel) of one launch's payload, between 1 GiB (smaller copies repeated
    # on the same buffers stay in the 256 MB memory-side cache) and 4 GiB: an
    # outside reference for what a contiguous copy reaches on this device.
    nbytes = max(1 << 30, min(min(k, L) * n * w.shape.page_bytes, 4 << 30))
    del buf
    x = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    y = torch.empty_like(x)
    y.copy_(x)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(reps):
        y.copy_(x)
    b.record(stream)
    torch.cuda.synchronize()
    runtime = 2 * nbytes * reps / (a.elapsed_time(b) / 1e3) / 1e9
    log(f"runtime device copy of {nbytes} B: {runtime:.1f} GB/s")
    del x, y
    return {"identity_ids_gbs": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
            "runtime_copy_gbs": round(runtime, 1), "runtime_copy_bytes": nbytes,
            "runtime_copy": "torch copy_ of one contiguous buffer (hipMemcpyAsync device to device)"}


def run_torch_device(w, dev, src, dst, s_ids, d_ids, reps: int = 3) -> dict:
    """The reference's own indexing, run on the device, layer by layer:
    buf = src[l][ids] (KVhelper.get_kv_cache's gather,
    paceserve/kv_transfer/kv_utils.py:44-46, without its host copy) and
    dst[l][dst_ids] = buf (insert_kv_cache's index_put_, kv_utils.py:51-52,
    without its host copy).  It writes the same bytes as the HIP path, so
    the destination stays verified."""
    import torch

    L = w.shape.num_layers
    si, di = s_ids.long(), d_ids.long()
    stream = torch.cuda.current_stream(dev)

    def step():
        for l in range(L):
            buf = src.layers[l][si]
            dst.layers[l][di] = buf

    step()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        step()
    b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    gbs = 4 * w.payload_bytes / (ms / 1e3) / 1e9
    log(f"torch device indexing (per layer): {gbs:.1f} GB/s")
    return {"value": round(gbs, 1), "unit": "GB/s", "ms_per_step": round(ms, 4), "steps": reps,
            "launches_per_step": 2 * L,
            "what": "per layer: buf = src[l][ids]; dst[l][dst_ids] = buf (torch advanced indexing on the device)"}


def run_append(dev, steps: int = 50, warmup: int = 5) -> dict:
    """The producer kernel (append_paged_kv_cache, NHD layout) on one
    Llama-3-8B layer cache [2048 pages, 2, 16, 8, 128] bf16:
      prefill: 16 requests x 1024 new tokens (16384 K and V rows);
      decode:  256 requests x 1 new token, sequences of 1..64 tokens.
    Two forms: the reference's (positions precomputed by
    get_batch_indices_positions, then the append) and the fused one
    (append_paged_kv_cache_indptr: positions derived in the same launch, the
    whole per-layer step in one call).  Algorithmic bytes per launch: each
    appended K and V row (8 * 128 * 2 B) read once and written once.  Kernel
    time comes from replays of a HIP graph of launches; the eager time per
    Python call is reported beside it.  Every appended row is checked
    against torch's own indexing of the cache after the replays."""
    import torch

    from paceserve_amd.kv_transfer import append as ap

    P, H, D, pages = 16, 8, 128, 2048
    row = H * D * 2
    g = torch.Generator(device=dev).manual_seed(1200)
    cache = torch.randn((pages, 2, P, H, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    perm = torch.randperm(pages, generator=torch.Generator().manual_seed(1201)).to(torch.int32)
    stream = torch.cuda.current_stream(dev)
    out = {"cache": f"[{pages}, 2, {P}, {H}, {D}] bf16", "unit": "GB/s"}
    lens_rng = torch.Generator().manual_seed(1202)
    cases = {
        "prefill": ([1024] * 16, [1024] * 16),
        "decode": (torch.randint(1, 65, (256,), generator=lens_rng).tolist(), [1] * 256),
    }

    def timed(fn, reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps * 1e3

    def graph_us(fn):
        # The Python wrapper costs more host time per call than a decode
        # launch takes on the GPU, so the kernel is timed from a HIP graph of
        # `steps` launches, replayed; it allocates nothing and records no
        # memset, and every replay rewrites the same rows.
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            fn()
        stream.wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            for _ in range(steps):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        return timed(graph.replay, 5) / steps

    for name, (seq_lens, new) in cases.items():
        npages = [-(-n // P) for n in seq_lens]
        kv_indptr = torch.tensor([0] + list(torch.tensor(npages).cumsum(0).tolist()), dtype=torch.int32, device=dev)
        kv_indices = perm[: int(kv_indptr[-1])].to(dev)
        last = torch.tensor([n - (k - 1) * P for n, k in zip(seq_lens, npages)], dtype=torch.int32, device=dev)
        append_indptr = torch.tensor([0] + list(torch.tensor(new).cumsum(0).tolist()), dtype=torch.int32, device=dev)
        nnz = int(append_indptr[-1])
        key = torch.randn((nnz, H, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
        value = torch.randn((nnz, H, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
        sl = ap.get_seq_lens(kv_indptr, last, P)
        bi, pos = ap.get_batch_indices_positions(append_indptr, sl, nnz)

        def launch():
            ap.append_paged_kv_cache(key, value, bi, pos, cache, kv_indices, kv_indptr, last)

        def fused():
            ap.append_paged_kv_cache_indptr(key, value, append_indptr, cache, kv_indices, kv_indptr, last)

        b_l, p_l = bi.long(), pos.long()
        page_t = kv_indices.long()[kv_indptr.long()[b_l] + p_l // P]

        def landed():
            return torch.equal(cache[page_t, 0, p_l % P].view(torch.int16), key.view(torch.int16)) and \
                torch.equal(cache[page_t, 1, p_l % P].view(torch.int16), value.view(torch.int16))

        alg = 4 * nnz * row
        res = {"tokens": nnz, "requests": len(seq_lens), "algorithmic_bytes_per_launch": alg}
        for form, fn in (("", launch), ("fused_", fused)):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            eager_us = timed(fn, steps)
            cache.zero_()
            us = graph_us(fn)
            ok = landed()
            res[f"{form}us_per_launch"] = round(us, 2)
            res[f"{form}eager_us_per_call"] = round(eager_us, 2)
            res[f"{form}gbs"] = round(alg / (us * 1e-6) / 1e9, 1)
            res[f"{form}frac_of_hbm_peak"] = round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
            res[f"{form}verified"] = bool(ok)
            log(f"append {name} {form or 'two-call '}: {nnz} tokens, {us:.2f} us per launch, "
                f"{res[f'{form}gbs']} GB/s, eager {eager_us:.2f} us per call, verified {ok}")
        # the reference's whole per-layer step, eager: get_seq_lens (torch),
        # get_batch_indices_positions, append_paged_kv_cache
        def step():
            s_l = ap.get_seq_lens(kv_indptr, last, P)
            b_i, p_s = ap.get_batch_indices_positions(append_indptr, s_l, nnz)
            ap.append_paged_kv_cache(key, value, b_i, p_s, cache, kv_indices, kv_indptr, last)

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        res["three_call_step_eager_us"] = round(timed(step, steps), 2)
        res["verified"] = res["verified"] and res["fused_verified"]
        out[name] = res
    return out


class _DropinModel:
    """Duck-typed model/cache configs and model runner for KVhelper: it reads
    only these attributes (paceserve/kv_transfer/kv_utils.py:17-23)."""

    def __init__(self, shape, cache):
        self.shape, self.dtype, self.block_size = shape, shape.dtype, shape.page_size

        class _Wrapper:
            gpu_cache = cache

        self.attention_backend_wrapper = _Wrapper()

    def get_num_q_heads(self, pc):
        return 4 * self.shape.num_kv_heads

    def get_num_kv_heads(self, pc):
        return self.shape.num_kv_heads

    def get_head_size(self):
        return self.shape.head_dim

    def get_num_layers(self, pc):
        return self.shape.num_layers


def run_dropin(dev, steps: int = 10, warmup: int = 2) -> dict:
    """The drop-in KVhelper moving the 4096-token request from one cache to
    another through host memory (get_kv_cache, then insert_kv_cache), against
    the reference's code for the same two calls written with torch: a
    pageable torch.zeros host tensor filled layer by layer from
    gpu_cache[i][tensor(ids)] (paceserve/kv_transfer/kv_utils.py:44-46), then
    gpu_cache[i][tensor(ids)] = content[i].to(device) per layer (:51-52).
    Wall-clock per call pair, to completion; both must leave the same bytes.
    The same for the request's first 1 and 32 pages (16 and 512 tokens), where
    fixed costs per call weigh more (`small`)."""
    import torch

    from paceserve_amd import workloads
    from paceserve_amd.kv_transfer.kv_utils import KVhelper

    w = workloads.get(workloads.PROMOTE)
    L, n = w.shape.num_layers, w.n_pages
    src = w.src_pool(dev)
    dst = w.dst_pool(dev)
    ids = list(w.src_tables[0])
    dst_ids = list(range(w.dst_pool_pages - 1, w.dst_pool_pages - 1 - n, -1))   # a fresh LIFO pool's pages

    def helper(cache):
        import contextlib

        m = _DropinModel(w.shape, cache)
        with contextlib.redirect_stdout(sys.stderr):       # KVhelper announces itself, as the reference does
            h = KVhelper(0, m, m, None)
        h.add_model_runner(m)
        return h

    class _Seq:
        seq_id = "r"

    src_h, dst_h = helper(src), helper(dst)

    def measure(ids, dst_ids, out, what):
        n = len(ids)
        payload = L * n * w.shape.page_bytes

        class _Tables:
            def _get_block_table(self, seq):
                return ids

        def ours():
            content, _ = src_h.get_kv_cache(_Seq(), _Tables())
            if not dst_h.insert_kv_cache(content, dst_ids, dev):
                raise RuntimeError("insert_kv_cache failed")

        def reference():
            seq_cache = torch.zeros((L, n) + w.shape.page_shape, dtype=w.shape.dtype)
            for i in range(L):
                seq_cache[i] = src[i][torch.tensor(ids), :, :, :, :]
            for i in range(L):
                dst[i][torch.tensor(dst_ids), :, :, :, :] = seq_cache[i].to(dev)

        for name, fn in (("kvhelper", ours), ("reference_torch", reference)):
            ts = []
            for i in range(warmup + steps):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                fn()
                torch.cuda.synchronize()
                if i >= warmup:
                    ts.append(time.perf_counter() - t0)
            ms = statistics.median(ts) * 1e3
            out[f"{name}_ms"] = round(ms, 3)
            out[f"{name}_gbs_per_direction"] = round(payload / (ms / 1e3) / 1e9, 2)
            log(f"drop-in {what} {name}: {ms:.3f} ms per get + insert")
            if name == "kvhelper":
                after = [d[torch.tensor(dst_ids, device=dev)].view(torch.int16).clone() for d in dst]
                for d in dst:
                    d.zero_()
        ok = all(torch.equal(d[torch.tensor(dst_ids, device=dev)].view(torch.int16), a) for d, a in zip(dst, after))
        ok = ok and all(torch.equal(s[torch.tensor(ids, device=dev)].view(torch.int16), a) for s, a in zip(src, after))
        out["same_bytes"] = ok
        out["speedup"] = round(out["reference_torch_ms"] / out["kvhelper_ms"], 2)
        return out

    out = measure(ids, dst_ids, {"payload_bytes": w.payload_bytes, "workload": w.name, "runs": steps}, "4096 tok")
    out["small"] = {}
    for pages in (1, 32):
        key = f"{pages * w.shape.page_size}tok"
        out["small"][key] = measure(ids[:pages], dst_ids[:pages], {"payload_bytes": L * pages * w.shape.page_bytes}, key)
    return out


# The cross-process channel leg: ring slots and host copy threads per side.
# Measured on MI355X with 16 host cores for the 512 MiB request: 31-32 GB/s
# for 16-64 MiB slots and 4-12 threads per side alike (the two DMA passes and
# two host copies per byte saturate host memory), 24 GB/s with 8 MiB slots.
CHANNEL_SLOT_BYTES = 32 << 20
CHANNEL_SLOTS = 4
CHANNEL_THREADS = 4
# The same-GPU device ring: 4 slots of 256 MiB (one 1 GiB allocation shared
# between the two processes, the largest the library exports).  Measured on
# the 4096-token request, from the pages' header to the last unpack: 329 us
# with 256 MiB slots, 368 us with 128 MiB, 394 us with 8 x 64 MiB and 456 us
# with 8 x 32 MiB: every chunk adds a pack, an unpack and a hand-over.
CHANNEL_DEVICE_SLOT_BYTES = 256 << 20


def channel_sender(name: str) -> None:
    """The sending process of the channel leg: builds the 4096-token
    request's source pool (seeded, on the GPU) and sends the request once per
    line read from stdin, as a prefill instance answers each pull.  On the
    GPU of a channel's device ring the pages go through that ring."""
    import torch

    from paceserve_amd import _native, workloads
    from paceserve_amd.kv_transfer import ops
    from paceserve_amd.kv_transfer.channel import KVChannel

    _native.load()
    dev = torch.device("cuda", 0)
    w = workloads.get(workloads.PROMOTE)
    # the worker's cache as its KVhelper holds it (one pool, built once)
    src = ops.PagedPool(w.src_pool(dev))
    torch.cuda.synchronize()
    ids = list(w.src_tables[0])
    with KVChannel.open(name, CHANNEL_THREADS, timeout=120) as ch:
        print("ready", flush=True)
        for line in sys.stdin:
            ch.send(src, ids, line.strip().encode(), timeout=120)


def channel_leg(dev, w, dst, d_ids, device_slot_bytes: int, runs: int, warmup: int) -> dict:
    """Moves the request `warmup + runs` times from a sender process into
    `dst` through one channel (device_slot_bytes > 0: with a device ring);
    wall-clock from the ask (a line on the sender's stdin) to the last unpack."""
    import subprocess

    import torch

    from paceserve_amd.kv_transfer.channel import KVChannel

    n = w.n_pages
    name = f"pace_bench_{os.getpid()}_{device_slot_bytes}"
    ch = KVChannel.create(name, CHANNEL_SLOT_BYTES, CHANNEL_SLOTS, CHANNEL_THREADS,
                          device_slot_bytes=device_slot_bytes)
    child = subprocess.Popen([sys.executable, str(ROOT / "bench.py"), "--channel-sender", name],
                             stdin=subprocess.PIPE, stdout=subprocess.PIPE, text=True)
    try:
        if child.stdout.readline().strip() != "ready":
            raise RuntimeError("channel sender did not start")
        ts = []
        for r in range(warmup + runs):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            child.stdin.write(f"{r}\n")
            child.stdin.flush()
            h = ch.recv_header(timeout=120)
            if h.meta != str(r).encode() or h.n_pages != n:
                raise RuntimeError(f"channel: unexpected message {h}")
            ch.recv(dst, d_ids, timeout=120)
            torch.cuda.synchronize()
            if r >= warmup:
                ts.append(time.perf_counter() - t0)
        child.stdin.close()
        if child.wait(timeout=120) != 0:
            raise RuntimeError(f"channel sender exited with {child.returncode}")
    finally:
        if child.poll() is None:
            child.kill()
        ch.close()
    ts.sort()
    ms = statistics.median(ts) * 1e3
    return {"ms": round(ms, 3), "gbs": round(w.payload_bytes / (ms / 1e3) / 1e9, 2),
            "p90_ms": round(ts[int(0.9 * (len(ts) - 1))] * 1e3, 3), "runs": runs}


def run_channel(dev, runs: int = 10, warmup: int = 2, ref_runs: int = 3) -> dict:
    """The 4096-token request moved from another process's cache into this
    one's through the channel: this process asks (a line on the sender's
    stdin, as a decode instance pulls a sequence), receives the header and
    unpacks the pages; wall-clock from the ask to the last unpack.  Two
    channels: one with a same-GPU device ring (the pages never leave HBM) and
    one through the shared-memory ring only (what two processes on different
    GPUs, or a host payload, use).  Beside them, the reference's path for the
    same hop, run in this process on a copy of the source pool: get_kv_cache
    into a pageable tensor (paceserve/kv_transfer/kv_utils.py:44-46), a pickle
    round trip standing in for the object store (prefill_instance.py:96-107,
    decode_instance.py:165-171; Ray's RPCs and inter-process copies are left
    out, so this understates its cost), and insert_kv_cache (:51-52)."""
    import pickle

    import torch

    from paceserve_amd import workloads
    from paceserve_amd.kv_transfer import ops

    w = workloads.get(workloads.PROMOTE)
    L, n = w.shape.num_layers, w.n_pages
    ids = list(w.src_tables[0])
    dst_ids = list(range(w.dst_pool_pages - 1, w.dst_pool_pages - 1 - n, -1))
    src = w.src_pool(dev)
    si, di = torch.tensor(ids, device=dev), torch.tensor(dst_ids, device=dev)
    out = {"payload_bytes": w.payload_bytes, "workload": w.name, "runs": runs,
           "slot_bytes": CHANNEL_SLOT_BYTES, "slots": CHANNEL_SLOTS, "copy_threads_per_side": CHANNEL_THREADS,
           "device_slot_bytes": CHANNEL_DEVICE_SLOT_BYTES}
    for label, dsb in (("device_ring", CHANNEL_DEVICE_SLOT_BYTES), ("shm_ring", 0)):
        dst = ops.PagedPool(w.dst_pool(dev))
        d_ids = ops.device_ids(dst_ids, dev)
        leg = channel_leg(dev, w, dst, d_ids, dsb, runs, warmup)
        leg["same_bytes"] = all(torch.equal(d[di].view(torch.int16), s[si].view(torch.int16))
                                for d, s in zip(dst.layers, src))
        out[label] = leg
        log(f"channel {label}: {leg['ms']} ms per request across processes, {leg['gbs']} GB/s, "
            f"same bytes {leg['same_bytes']}")
        del dst
    # the headline figures: the same-GPU device ring
    out["channel_ms"] = out["device_ring"]["ms"]
    out["channel_gbs"] = out["device_ring"]["gbs"]
    out["same_bytes"] = out["device_ring"]["same_bytes"] and out["shm_ring"]["same_bytes"]
    dst = w.dst_pool(dev)
    rts = []
    for r in range(1 + ref_runs):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        seq_cache = torch.zeros((L, n) + w.shape.page_shape, dtype=w.shape.dtype)
        for i in range(L):
            seq_cache[i] = src[i][torch.tensor(ids), :, :, :, :]
        got = pickle.loads(pickle.dumps(seq_cache))
        for i in range(L):
            dst[i][torch.tensor(dst_ids), :, :, :, :] = got[i].to(dev)
        torch.cuda.synchronize()
        if r >= 1:
            rts.append(time.perf_counter() - t0)
    rms = statistics.median(rts) * 1e3
    out["reference_emulated_ms"] = round(rms, 2)
    out["reference_emulated_gbs"] = round(w.payload_bytes / (rms / 1e3) / 1e9, 2)
    out["reference_emulated"] = ("get_kv_cache (pageable, per layer) + pickle.dumps/loads + insert_kv_cache "
                                 "(per layer), one process; excludes Ray's RPCs and object-store copies")
    out["speedup_vs_reference_emulated"] = round(rms / out["channel_ms"], 2)
    log(f"channel reference path (emulated): {rms:.2f} ms")
    return out


def link_settle(dev, target_gbs: float = 45.0, max_wait_s: float = 30.0, streak: int = 3) -> dict:
    """Waits until `streak` consecutive 64 MiB pinned device-to-host copies,
    0.2 s apart, each run at target_gbs or more (other DMA work, such as the
    driver scrubbing device memory that an earlier process freed, shares the
    engines in bursts), for at most max_wait_s; returns what it saw."""
    import torch

    nbytes = 64 << 20
    a = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(3)
    h = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    t_start = time.perf_counter()
    rate, good = 0.0, 0
    while True:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        h.copy_(a, non_blocking=True)
        torch.cuda.synchronize()
        rate = nbytes / (time.perf_counter() - t0) / 1e9
        good = good + 1 if rate >= target_gbs else 0
        waited = time.perf_counter() - t_start
        if good >= streak or waited >= max_wait_s:
            break
        time.sleep(0.2)
    return {"d2h_gbs": round(rate, 1), "waited_s": round(waited, 2), "settled": good >= streak}


def staging_chunk_bytes(w) -> int:
    """Bytes of one layer chunk of a workload's pinned-host legs."""
    from paceserve_amd.kv_transfer import kv_utils

    layer_bytes = w.n_pages * w.shape.page_bytes
    k = w.layers_per_chunk or kv_utils.roundtrip_chunk_layers(w.shape.num_layers, layer_bytes)
    return k * layer_bytes


def run_staging(w, dev, src, dst, s_ids, d_ids, stager, reps: int = 3):
    """Pinned-host legs: pack_to_host, unpack_from_host and the overlapped
    round trip, in GB/s per direction against the PCIe Gen5 x16 peak, through
    `stager` (one for the whole process, as a serving worker keeps its own)."""
    import torch

    from paceserve_amd.kv_transfer import kv_utils, ops

    L, n, pb = w.shape.num_layers, s_ids.numel(), w.shape.page_bytes
    layer_bytes = n * pb
    k = w.layers_per_chunk or kv_utils.roundtrip_chunk_layers(L, layer_bytes)
    chunk = k * layer_bytes
    chunks = -(-L // k)
    if stager.slot_bytes < chunk:
        raise ValueError(f"stager slots of {stager.slot_bytes} B cannot hold {w.name}'s {chunk} B chunks")
    # host ring of up to 4 chunk regions (a full copy for short payloads)
    host_bytes = min(w.payload_bytes, 4 * chunk)
    host = torch.empty(host_bytes, dtype=torch.uint8, pin_memory=True)
    full = None
    if w.payload_bytes <= (8 << 30):
        full = torch.empty((L, n) + w.shape.page_shape, dtype=w.shape.dtype, pin_memory=True)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    out = {"layers_per_chunk": k, "chunks": chunks, "chunk_bytes": chunk, "host_ring_bytes": host_bytes,
           "pcie_peak_gbs_per_direction": 64.0}
    st = stager
    t_rt = timed(lambda: st.roundtrip(src, s_ids, dst, d_ids, host, k))
    out["roundtrip_ms"] = round(t_rt * 1e3, 3)
    out["roundtrip_gbs_per_direction"] = round(w.payload_bytes / t_rt / 1e9, 2)
    if full is not None:
        t_d2h = timed(lambda: st.pack_to_host(src, s_ids, full, k))
        t_h2d = timed(lambda: st.unpack_from_host(full, dst, d_ids, k))
        out["pack_to_host_gbs"] = round(w.payload_bytes / t_d2h / 1e9, 2)
        out["unpack_from_host_gbs"] = round(w.payload_bytes / t_h2d / 1e9, 2)
    torch.cuda.synchronize()
    log(f"staging: round trip {out['roundtrip_ms']} ms = {out['roundtrip_gbs_per_direction']} GB/s per direction")
    return out


def verify(w, src, dst, s_ids, d_ids, dev) -> bool:
    """Every layer of both pools, byte for byte: the destination equals its
    content before the migration (regenerated from its seed) with torch's
    index_copy_ of the index_select'ed source pages applied, and the source
    equals its content before (workloads.migration_mismatch)."""
    from paceserve_amd import workloads

    bad = workloads.migration_mismatch(src.layers, dst.layers, s_ids, d_ids, w.dst_before(dev), w.src_before(dev))
    if bad is not None:
        log(f"{w.name}: verification failed: {bad}")
    return bad is None


VERIFIED_WHAT = ("every layer of both pools compared byte for byte: destination = its seeded content before "
                 "with torch index_copy_(dst_ids, index_select(src, src_ids)) applied; source unchanged")


def config_steps(w, steps: int, seconds: float = 0.05) -> int:
    """Timed steps for a workload measured beside the headline: at least
    `steps`, and enough for about `seconds` of copying at 6.5 TB/s, so that the
    events around the timed region stay negligible on small payloads."""
    est = 4 * w.payload_bytes / 6.5e12
    return max(steps, min(2000, int(seconds / est) + 1))


CPU_CONFIG_SECONDS = 3.0
CPU_CONFIG_LAYERS = 4


def run_staging_leg(args, name: str, dev, stager) -> dict:
    """The pinned-host legs of a workload (run_staging) on its own pools,
    then the exact check of both pools (the round trip writes the same
    destination pages as the device path)."""
    from paceserve_amd import workloads

    w = workloads.get(name)
    log(f"staging {w.name}: {w.description}")
    src, dst, plan, s_ids, d_ids = device_setup(w, dev)
    st = run_staging(w, dev, src, dst, s_ids, d_ids, stager)
    st["workload"] = w.name
    if args.verify:
        st["verified"] = verify(w, src, dst, s_ids, d_ids, dev)
        log(f"staging {w.name}: verified {st['verified']}")
    return st


def run_config(args, name: str, dev, staging: dict = None) -> dict:
    """One of the other workloads, measured in the same process after the
    headline: K timed steps of pack + unpack (value and roofline as for the
    headline), the exact check of both pools, the identity-id copy ceiling
    (last: it writes pages no id names) and a short CPU sample.  `staging`:
    the workload's pinned-host legs, measured before the headline."""
    import argparse

    from paceserve_amd import workloads

    w = workloads.get(name)
    log(f"config {w.name}: {w.description}")
    src, dst, plan, s_ids, d_ids = device_setup(w, dev)
    sub = argparse.Namespace(**vars(args))
    sub.steps = config_steps(w, args.steps)
    sub.mode = "buffer"
    res = run_device(sub, w, dev, src, dst, plan, s_ids, d_ids)
    out = {"config": w.summary(), "value": round(res["value"], 1), "unit": "GB/s",
           "frac_of_hbm_peak": round(res["value"] / HBM_PEAK_GBS, 4), "steps": sub.steps, "warmup": args.warmup,
           "ms_per_step": round(res["event_ms_per_step"], 4), "pack_ms": res["pack_ms_mean"],
           "unpack_ms": res["unpack_ms_mean"], "roofline": res["roofline"]}
    tr = traffic_from_profiles(w.name)
    if tr is not None:
        out["roofline"]["traffic"] = tr["traffic_bytes_per_launch"]
        out["roofline"]["traffic_source"] = (f"profiles/page_copy_{w.name}_traffic.json "
                                             "(rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)")
    log(f"config {w.name}: {out['value']} GB/s ({out['frac_of_hbm_peak'] * 100:.1f}% of peak), K={sub.steps}")
    if args.verify:
        out["verified"] = verify(w, src, dst, s_ids, d_ids, dev)
        log(f"config {w.name}: verified {out['verified']}")
    if staging is not None:
        out["staging"] = staging
    out["copy_ceiling"] = run_ceiling(w, dev, src, dst, plan.n_pages)
    if not args.no_cpu:
        layers = min(CPU_CONFIG_LAYERS, cpu_sample_layers(w))
        out["cpu_baseline"] = run_cpu_baseline(w, layers, src, dst, plan, CPU_CONFIG_SECONDS)
        log(f"config {w.name}: CPU baseline {out['cpu_baseline']['value']} GB/s")
    return out


def run_promote(dev, steps=100, warmup=10, c_caller=True):
    """p50/p90 latency of promoting one 4096-token request."""
    import torch

    from paceserve_amd import workloads
    from paceserve_amd.core.block_manager import BlockAllocator, NativeBlockAllocator
    from paceserve_amd.kv_transfer import migrate

    w = workloads.get(workloads.PROMOTE)
    src = w.src_pool(dev)
    dst = w.dst_pool(dev)
    host = torch.empty(w.payload_bytes, dtype=torch.uint8, pin_memory=True)
    out = {}
    # The request's block table as a scheduler built on the native allocator
    # holds it: int32 ids and int64 offsets (CSR), no Python lists.
    csr_ids = array("i", w.src_tables[0])
    csr_indptr = array("q", (0, len(csr_ids)))
    # "buffer"/"fused": Python planner + ops; "*_native": one pace_kv_promote
    # call from KVMigrator.promote (list-of-lists block tables);
    # "buffer_native_csr": the same call from KVMigrator.promote_native (CSR)
    for mode in ("buffer", "fused", "pinned", "buffer_native", "fused_native", "buffer_native_csr"):
        native = "_native" in mode
        alloc = (NativeBlockAllocator if native else BlockAllocator)(w.shape.page_size, w.dst_pool_pages)
        mig = migrate.KVMigrator(src, dst, alloc)
        kind = mode.split("_")[0]
        lat = []
        n_iter = warmup + steps
        for i in range(n_iter):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            if mode == "buffer_native_csr":
                got = mig.promote_native(csr_ids, csr_indptr, mode=kind)
            else:
                got = mig.promote(w.src_tables, mode=kind, host_buf=host if kind == "pinned" else None)
            ev = torch.cuda.Event()
            ev.record()
            ev.synchronize()
            t1 = time.perf_counter()
            # return the pages (outside the timing)
            for t in (got.dst_tables if mode != "buffer_native_csr" else [got.tolist()]):
                alloc.free_many(reversed(t))
            if i >= warmup:
                lat.append((t1 - t0) * 1e6)
        lat.sort()
        out[mode] = {"p50_us": round(statistics.median(lat), 1),
                     "p90_us": round(lat[int(0.9 * (len(lat) - 1))], 1), "runs": len(lat)}
        log(f"promote 4096 tok {mode}: p50 {out[mode]['p50_us']} us")
    # swap of the same request into a pinned host page pool and back
    from paceserve_amd.kv_transfer import ops
    dpool = ops.PagedPool(src)
    hpool = ops.HostPagePool.like(dpool, len(w.src_tables[0]))
    hids = list(range(len(w.src_tables[0])))
    for name, fn in (("swap_out", lambda: ops.swap_out(dpool, w.src_tables[0], hpool, hids)),
                     ("swap_in", lambda: ops.swap_in(hpool, hids, ops.PagedPool(dst), w.src_tables[0]))):
        lat = []
        for i in range(warmup + steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            if i >= warmup:
                lat.append((time.perf_counter() - t0) * 1e6)
        lat.sort()
        out[name] = {"p50_us": round(statistics.median(lat), 1), "p90_us": round(lat[int(0.9 * (len(lat) - 1))], 1),
                     "gbs": round(w.payload_bytes / (statistics.median(lat) * 1e-6) / 1e9, 2), "runs": len(lat)}
        log(f"promote 4096 tok {name}: p50 {out[name]['p50_us']} us ({out[name]['gbs']} GB/s)")
    out["payload_bytes"] = w.payload_bytes
    out["c_caller"] = run_promote_c(w) if c_caller else None
    # the metric's promote latency: allocation + remap + id upload + pack +
    # unpack, through the single library call
    out["p50_us"] = out["buffer_native"]["p50_us"]
    out["p50_mode"] = ("buffer_native (KVMigrator.promote of list block tables -> pace_kv_promote: plan, ids, "
                       "pack, unpack)")
    return out


def run_promote_c(w):
    """The same promotion timed from C (tests/c_abi/pace_kv_promote_latency,
    built with the library): pace_kv_promote to the completion of an event
    after it, with no Python in the loop; buffer and fused modes, 100 runs
    after 10 warm-ups, and a check of the moved bytes.  None when the program
    is not built."""
    import subprocess

    from paceserve_amd.build import C_LATENCY_BIN

    if not C_LATENCY_BIN.exists():
        log(f"{C_LATENCY_BIN} is not built: no C-caller promote latency")
        return None
    sh = w.shape
    cmd = [str(C_LATENCY_BIN), str(sh.num_layers), str(w.src_pool_pages), str(len(w.src_tables[0])),
           str(sh.page_bytes), "100", "10"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        raise RuntimeError(f"{' '.join(cmd)} failed ({r.returncode}): {r.stdout} {r.stderr}")
    res = json.loads(r.stdout.strip().splitlines()[-1])
    log(f"promote 4096 tok from C: buffer p50 {res['buffer']['p50_us']} us, fused p50 {res['fused']['p50_us']} us, "
        f"verified {res['verified']}")
    return res


def cpu_sample_layers(w) -> int:
    """Layers in the CPU sample: up to 16, within 64 GiB and half of the host's
    free memory (two host pools plus the buffer per layer)."""
    try:
        import psutil
        free = psutil.virtual_memory().available
    except ImportError:
        free = 32 << 30
    per_layer = (w.src_pool_pages + w.dst_pool_pages + w.n_pages) * w.shape.page_bytes
    budget = min(64 << 30, int(0.5 * free))
    return max(1, min(w.shape.num_layers, budget // per_layer, 16))


def run_calibration(dev) -> None:
    """torch's contiguous device copy of 1 GiB, three times: the reference
    dispatch whose FETCH_SIZE / WRITE_SIZE counters scale ours to bytes."""
    import torch

    a = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(CALIBRATION_COPIES):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"calibration: {CALIBRATION_COPIES} x 1 GiB torch copy_ done")


CPU_SAMPLE_SECONDS = 10.0


def run_cpu_baseline(w, layers_sample: int, src_pool, dst_pool, plan, seconds: float = None):
    """The reference's CPU path on pageable host tensors: per layer,
    index_select into the buffer then index_copy_ into the destination.  The
    host pools are copies of the first layers of the device pools (same
    bytes, same block tables)."""
    import torch

    from oracle import kv_oracle as orc

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    L = layers_sample
    src = [t.cpu() for t in src_pool.layers[:L]]
    dst = [t.cpu() for t in dst_pool.layers[:L]]
    s_idx = torch.tensor(plan.src_ids, dtype=torch.long)
    d_idx = torch.tensor(plan.dst_ids, dtype=torch.long)
    buf = torch.empty((L, plan.n_pages) + w.shape.page_shape, dtype=w.shape.dtype)
    for _ in range(2):                                                # warm-up (first touch)
        orc.torch_cpu_pack_unpack(src, s_idx, dst, d_idx, buf)
    # Passes until `seconds` (CPU_SAMPLE_SECONDS) of work are timed (5 to 5000 passes).
    times = []
    end = time.perf_counter() + (CPU_SAMPLE_SECONDS if seconds is None else seconds)
    while len(times) < 5 or (len(times) < 5000 and time.perf_counter() < end):
        t0 = time.perf_counter()
        orc.torch_cpu_pack_unpack(src, s_idx, dst, d_idx, buf)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    payload = L * plan.n_pages * w.shape.page_bytes
    return {
        "value": round(4 * payload / t / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{L} of {w.shape.num_layers} layers, all {plan.n_pages} pages of {w.name} "
                  f"({payload / 2**30:.2f} GiB payload), full-size pools per layer; median of {len(times)} "
                  f"passes ({sum(times):.1f} s) after 2 warm-up passes; torch {torch.__version__} "
                  f"index_select/index_copy_ on host tensors",
        "seconds_per_pass": round(t, 4),
    }


PROFILES = ROOT / "profiles"


def _rows(csv_path: str) -> list:
    import csv

    with open(csv_path, newline="") as f:
        return list(csv.DictReader(f))


def _json(path: str) -> dict:
    with open(path) as f:
        return json.load(f)
KERNEL_TAG = "page_copy_kernel"


# Copies of 1 GiB that --calibrate runs last in a bench run.
CALIBRATION_COPIES = 3


def _per_dispatch(csv_path: str, counter: str):
    """Counter values per kernel name, in dispatch order."""
    by = {}
    rows = [r for r in _rows(csv_path) if r["Counter_Name"] == counter]
    for r in sorted(rows, key=lambda r: int(r["Dispatch_Id"])):
        by.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    return by


def summarize_pmc(fetch_csv: str, write_csv: str, workload: str) -> dict:
    """HBM bytes per copy-kernel launch from two rocprofv3 --pmc runs
    (FETCH_SIZE, WRITE_SIZE; KiB per dispatch), each scaled so that the 1 GiB
    device copy run by --calibrate (dispatched as __amd_rocclr_copyBuffer)
    reads 1 GiB fetched and 1 GiB written.  The calibration copies are the
    run's last CALIBRATION_COPIES large copy dispatches: earlier ones (the
    runtime copy beside the copy ceiling) have other sizes."""
    gib_kib = float(1 << 20)
    out = {"workload": workload, "kernel": KERNEL_TAG, "fetch_csv": fetch_csv, "write_csv": write_csv}
    for name, path, counter in (("fetch", fetch_csv, "FETCH_SIZE"), ("write", write_csv, "WRITE_SIZE")):
        by = _per_dispatch(path, counter)
        names = sorted({k.replace("void pace_kv::(anonymous namespace)::", "").split("(")[0]
                        for k in by if "page_copy_kernel" in k})
        if names:
            out["kernel"] = " and ".join(names)
        ours = [v for k, vals in by.items() if "page_copy_kernel" in k for v in vals]
        calib = [v for k, vals in by.items() if "copyBuffer" in k for v in vals if v > 0.25 * gib_kib]
        calib = calib[-CALIBRATION_COPIES:]
        if not ours or not calib:
            raise SystemExit(f"{path}: missing page_copy_kernel or calibration dispatches")
        factor = gib_kib / statistics.mean(calib)
        out[f"{name}_kib_per_dispatch_raw"] = statistics.mean(ours)
        out[f"{name}_calibration_kib_raw"] = statistics.mean(calib)
        out[f"{name}_scale"] = round(factor, 4)
        out[f"{name}_bytes_per_launch"] = int(statistics.mean(ours) * factor * 1024)
        out[f"{name}_dispatches"] = len(ours)
    out["traffic_bytes_per_launch"] = out["fetch_bytes_per_launch"] + out["write_bytes_per_launch"]
    return out


def requests_per_launch(rdreq_csv: str, wrreq_csv: str) -> dict:
    """HBM bytes per page-copy launch from request counts, with no scale
    factor: TCC read requests are 128 bytes unless counted as 32-byte ones
    (TCC_EA0_RDREQ_sum, TCC_EA0_RDREQ_32B_sum), write requests 64 bytes
    unless 32 (TCC_EA0_WRREQ_sum, TCC_EA0_WRREQ_64B_sum); TCC_BUBBLE_sum is
    reported beside them (0 here: the 128-byte reads it would count are the
    ones FETCH_SIZE weighs at 64 bytes)."""
    def mean(path, counter):
        vals = [v for k, vs in _per_dispatch(path, counter).items() if "page_copy_kernel" in k for v in vs]
        return statistics.mean(vals) if vals else 0.0

    rd, rd32, bubble = (mean(rdreq_csv, c) for c in ("TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_BUBBLE_sum"))
    wr, wr64 = mean(wrreq_csv, "TCC_EA0_WRREQ_sum"), mean(wrreq_csv, "TCC_EA0_WRREQ_64B_sum")
    read = (rd - rd32) * 128 + rd32 * 32
    write = wr64 * 64 + (wr - wr64) * 32
    return {"rdreq": rd, "rdreq_32b": rd32, "bubble": bubble, "wrreq": wr, "wrreq_64b": wr64,
            "read_bytes_per_launch": int(read), "write_bytes_per_launch": int(write),
            "bytes_per_launch": int(read + write), "rdreq_csv": rdreq_csv, "wrreq_csv": wrreq_csv}


def timed_dispatches(trace_csv: str, bench: dict):
    """The page-copy dispatches of the timed steps in a rocprofv3 kernel
    trace of one bench.py run.  The headline's launches are the page-copy
    dispatches whose grid covers its batch (64 threads per 1 KiB row of each
    of its pages; the staging legs that run earlier and the other workloads
    that run later have other batches); in dispatch order they are the W
    warm-up steps, then the K timed steps, then the launch-timing pass and
    the copy ceiling.  Returns (durations ns, span ns) of the timed ones."""
    cfg = bench["config"]
    page_bytes = cfg["payload_bytes"] // (cfg["layers"] * cfg["pages"])
    grid_x = -(-page_bytes // 1024) * cfg["pages"] * 64
    rows = [r for r in _rows(trace_csv) if "page_copy_kernel" in r["Kernel_Name"]
            and int(r.get("Grid_Size_X", grid_x)) == grid_x]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    per_step = bench["roofline"]["launches_per_step"]
    first = bench["warmup"] * per_step
    timed = rows[first:first + bench["steps"] * per_step]
    durs = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in timed]
    span = int(timed[-1]["End_Timestamp"]) - int(timed[0]["Start_Timestamp"])
    return durs, span


def summarize_stats(stats_csv: str, bench_json: str, command: str, trace_csv: str = "") -> str:
    """Markdown summary of a rocprofv3 --stats kernel table beside the bench
    line of the same run (mean launch time measured with HIP events); with
    the kernel trace, also the timed steps' own dispatches."""
    rows = _rows(stats_csv)
    bench = _json(bench_json)
    cfg, rf = bench["config"], bench["roofline"]
    out = [f"# page copy kernel on {cfg['workload']} - kernel trace statistics", "",
           f"Workload: {cfg['description']}; {cfg['pages']} pages x {cfg['layers']} layers, "
           f"payload {cfg['payload_bytes']} B.", "", "Command (repo root, one MI355X):", "", "```",
           "export TMPDIR=/tmp", command, "```", "",
           "| kernel | calls | average ns | min ns | max ns | std dev ns |", "|---|---|---|---|---|---|"]
    ours = [r for r in rows if "pace_kv::" in r["Name"]]
    others = sorted((r for r in rows if "pace_kv::" not in r["Name"]),
                    key=lambda r: -float(r["TotalDurationNs"]))
    for r in ours + others[:4]:
        name = r["Name"]
        if "pace_kv::" in name:
            short = name.split("(anonymous namespace)::", 1)[-1].split("(")[0]
        else:
            short = "torch normal_ (pool fill)" if "distribution" in name else name[:48]
        out.append(f"| {short} | {r['Calls']} | {float(r['AverageNs']):.0f} | {r['MinNs']} | {r['MaxNs']} | "
                   f"{float(r['StdDev']):.0f} |")
    if others[4:]:
        rest = others[4:]
        out.append(f"| {len(rest)} more kernels (torch: checks, baselines, set-up) | "
                   f"{sum(int(r['Calls']) for r in rest)} | | | | |")
    pc = [r for r in rows if "page_copy_kernel" in r["Name"]]
    if pc:
        calls = sum(int(r["Calls"]) for r in pc)
        avg_us = sum(float(r["AverageNs"]) * int(r["Calls"]) for r in pc) / calls / 1e3
        per_launch = rf["algorithmic_bytes_per_launch"]
        out += ["", f"bench.py in the same run (HIP events on the launch stream): mean launch "
                f"{rf['mean_launch_us']} us, achieved {rf['achieved']} GB/s ({rf['frac'] * 100:.1f}% of 8 TB/s); "
                f"headline value {bench['value']} GB/s.",
                f"rocprofv3 average over all {calls} page-copy launches of the run (every leg and workload it "
                f"ran, of every size) {avg_us:.2f} us; the headline's own launches are the line below."]
        if trace_csv:
            durs, span = timed_dispatches(trace_csv, bench)
            mean_us = statistics.mean(durs) / 1e3
            span_us = span / 1e3 / len(durs)
            out += [f"Timed steps only ({len(durs)} launches, from the kernel trace): mean kernel duration "
                    f"{mean_us:.2f} us ({per_launch / (mean_us * 1e-6) / 1e9:.0f} GB/s per launch); first start to "
                    f"last end {span_us:.2f} us per launch vs bench {rf['mean_launch_us']} us "
                    f"({(rf['mean_launch_us'] / span_us - 1) * 100:+.2f}%)."]
    return "\n".join(out) + "\n"


def summarize_promote(trace_csv: str, bench_json: str, command: str) -> str:
    """Markdown summary of the promote kernels in a rocprofv3 kernel trace of
    one bench.py run.  pace_kv_promote carries a 4096-token request's page ids
    in the kernel arguments, so its launches are the run's only
    page_copy_inline_kernel dispatches: a pack (source ids inline) and an
    unpack (destination ids inline) per buffer-mode promote, one move (both
    inline) per fused promote."""
    bench = _json(bench_json)
    pr = bench["promote_4k"]
    kinds = {"true, false>": "pack (source ids inline)", "false, true>": "unpack (destination ids inline)",
             "true, true>": "move (both inline)"}
    durs = {}
    for r in _rows(trace_csv):
        name = r["Kernel_Name"]
        if "page_copy_inline_kernel" not in name:
            continue
        tmpl = name.split("page_copy_inline_kernel<", 1)[1].split(">", 1)[0] + ">"
        kind = next((v for k, v in kinds.items() if tmpl.endswith(k)), tmpl)
        durs.setdefault(kind, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    payload = pr["payload_bytes"]
    out = ["# promote kernels on llama3-8b-4096tok-bf16 - kernel trace", "",
           "One 4096-token request (256 pages), Llama-3-8B KV, bf16, 2048-page pools; "
           f"payload {payload} B. `pace_kv_promote` plans, allocates and launches in one call.", "",
           "Command (repo root, one MI355X):", "", "```", "export TMPDIR=/tmp", command, "```", "",
           "| kernel | launches | mean us | p50 us | min us | max us | GB/s (2 x payload / p50) |",
           "|---|---|---|---|---|---|---|"]
    for kind in ("pack (source ids inline)", "unpack (destination ids inline)", "move (both inline)"):
        d = sorted(durs.get(kind, []))
        if not d:
            continue
        p50 = statistics.median(d)
        out.append(f"| {kind} | {len(d)} | {statistics.mean(d):.1f} | {p50:.1f} | {d[0]:.1f} | {d[-1]:.1f} | "
                   f"{2 * payload / (p50 * 1e-6) / 1e9:.0f} |")
    pk = statistics.median(durs.get("pack (source ids inline)", [0.0]))
    up = statistics.median(durs.get("unpack (destination ids inline)", [0.0]))
    mv = statistics.median(durs.get("move (both inline)", [0.0]))
    out += ["", f"bench.py in the same run: promote p50 {pr['buffer_native']['p50_us']} us (pack + unpack, "
            f"{pr['buffer_native']['runs']} runs), of which {pk + up:.1f} us are the two kernels "
            f"({4 * payload / ((pk + up) * 1e-6) / 1e9:.0f} GB/s of pack+unpack bytes); fused promote p50 "
            f"{pr['fused_native']['p50_us']} us, of which {mv:.1f} us is the move kernel. The rest is host "
            f"time (Python, planning, launch) and completion."]
    if pr.get("c_caller"):
        c = pr["c_caller"]
        out += ["", f"The same call from C (tests/c_abi/pace_kv_promote_latency, in the same run): buffer p50 "
                f"{c['buffer']['p50_us']} us, fused p50 {c['fused']['p50_us']} us."]
    return "\n".join(out) + "\n"


def summarize_copies(copy_csv: str, kernel_csv: str, bench_json: str, command: str) -> str:
    """Markdown summary of the pinned-host round trip from a rocprofv3
    --memory-copy-trace (DMA-engine copies) and --kernel-trace (the round
    trip's copy_to_host_kernel; hipMemcpyAsync device-to-host copies that the
    runtime ran as __amd_rocclr_copyBuffer blit kernels): per-direction busy
    time and how long both directions ran at once."""
    bench = _json(bench_json)
    st = bench.get("staging") or {}
    chunk = int(st.get("chunk_bytes", 0))
    spans = {"D2H": [], "H2D": []}
    for r in _rows(copy_csv):
        d = "D2H" if "DEVICE_TO_HOST" in r["Direction"] else ("H2D" if "HOST_TO_DEVICE" in r["Direction"] else None)
        if d:
            spans[d].append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), "DMA engine"))
    min_ns = 1_000_000   # blits shorter than 1 ms are not chunk copies
    for r in _rows(kernel_csv):
        s0, e0 = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        if "copyBuffer" in r["Kernel_Name"] and e0 - s0 > min_ns:
            spans["D2H"].append((s0, e0, "runtime blit kernel"))
        elif "copy_to_host_kernel" in r["Kernel_Name"]:
            spans["D2H"].append((s0, e0, "copy_to_host_kernel"))
    k = int(st.get("chunks", 0))
    # The last round trip: its k host-to-device copies are the run's last
    # ones; its device-to-host copies are the last k that end before them
    # (later blits, such as the device-to-device copies beside the copy
    # ceiling, are not chunk copies).
    h2d = sorted(spans["H2D"])[-k:]
    t_end = max(e for _, e, _ in h2d) if h2d else 0
    last = {"H2D": h2d, "D2H": sorted(x for x in spans["D2H"] if x[1] <= t_end)[-k:]}
    t0 = min(v[0][0] for v in last.values() if v)
    t1 = max(v[-1][1] for v in last.values() if v)

    def busy(v):
        return sum(e - s for s, e, _ in v)

    both = sum(max(0, min(e1, e2) - max(s1, s2)) for s1, e1, _ in last["D2H"] for s2, e2, _ in last["H2D"])
    out = ["# pinned-host round trip on " + bench["config"]["workload"] + " - memory copy trace", "",
           bench["config"]["description"] + ".", "", "Command (repo root, one MI355X):", "", "```",
           "export TMPDIR=/tmp", command, "```", "",
           f"Last round trip: {k} chunks of {chunk} B each way (layers_per_chunk={st.get('layers_per_chunk')}), "
           f"host ring {st.get('host_ring_bytes')} B.", "",
           "| direction | copies | executed as | busy ms | mean GB/s while busy |", "|---|---|---|---|---|"]
    for d in ("D2H", "H2D"):
        v = last[d]
        if v:
            kinds = ", ".join(f"{sum(1 for x in v if x[2] == kd)} {kd}" for kd in sorted({x[2] for x in v}))
            out.append(f"| {d} | {len(v)} | {kinds} | {busy(v) / 1e6:.2f} | "
                       f"{len(v) * chunk / (busy(v) * 1e-9) / 1e9:.1f} |")
    out += ["", f"Wall span of the last round trip: {(t1 - t0) / 1e6:.2f} ms; both directions busy at once for "
            f"{both / 1e6:.2f} ms ({both / max(1, t1 - t0) * 100:.0f}% of the span).",
            f"bench.py in the same run: round trip {st.get('roundtrip_ms')} ms = "
            f"{st.get('roundtrip_gbs_per_direction')} GB/s per direction (PCIe Gen5 x16 peak 64 GB/s per direction)."]
    return "\n".join(out) + "\n"


def summarize_kernel_pmc(kernel: str, command: str, csvs: list) -> str:
    """Markdown table of rocprofv3 --pmc counter values per dispatch for the
    kernels whose names contain `kernel` (alternatives separated by '|'),
    grouped by kernel and grid size (each counter's mean over the dispatches
    of a group), from one or more counter-collection CSVs (one pass each).
    `command` may hold several commands, one per line."""
    groups = {}
    wanted = kernel.split("|")
    for path in csvs:
        for r in _rows(path):
            name = r["Kernel_Name"]
            if not any(k in name for k in wanted):
                continue
            short = name.split("(anonymous namespace)::", 1)[-1].split("(")[0]
            if short.startswith("__amd_rocclr"):
                short = short.split("<")[0]
            key = (short, int(r.get("Grid_Size", 0) or 0))
            groups.setdefault(key, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    counters = sorted({c for g in groups.values() for c in g})
    out = [f"# rocprofv3 counters per dispatch: {kernel}", "", "Command (repo root, one MI355X; one pass per CSV):",
           "", "```", "export TMPDIR=/tmp", command, "```", "",
           "| kernel | grid size (threads) | dispatches | " + " | ".join(counters) + " |",
           "|---|---|---|" + "---|" * len(counters)]
    for (short, grid), vals in sorted(groups.items(), key=lambda kv: kv[0][1]):
        n = max(len(v) for v in vals.values())
        cells = [f"{statistics.mean(vals[c]):.4g}" if c in vals else "" for c in counters]
        out.append(f"| {short} | {grid} | {n} | " + " | ".join(cells) + " |")
    return "\n".join(out) + "\n"


def traffic_verdict(t: dict, alg: int) -> str:
    """What the measured traffic says against the algorithmic bytes: within
    0.1% of them, no re-reads and no partial-line writes; above that, the
    excess of each direction (half of `alg` is read, half written)."""
    if t["traffic_bytes_per_launch"] <= 1.001 * alg:
        return "no re-reads, no partial-line writes (within 0.1%)."
    rd = t["fetch_bytes_per_launch"] / (alg / 2) - 1
    wr = t["write_bytes_per_launch"] / (alg / 2) - 1
    return (f"{(t['traffic_bytes_per_launch'] / alg - 1) * 100:.2f}% above them; reads {rd * 100:+.2f}%, "
            f"writes {wr * 100:+.2f}% against the bytes read and written once.")


def pmc_markdown(traffic_json: str) -> str:
    """Markdown form of a --summarize-pmc result (the committed summary)."""
    t = _json(traffic_json)
    wl = t["workload"]
    from paceserve_amd import workloads

    w = workloads.get(wl)
    # one launch reads and writes its layer chunk's pages once
    chunk = min(w.device_layers_per_chunk or w.shape.num_layers, w.shape.num_layers)
    alg = 2 * chunk * w.n_pages * w.shape.page_bytes
    run = (f"python3 bench.py --workload {wl} --no-cpu --no-promote --no-staging --no-dropin --no-append --no-channel "
           "--no-configs --no-verify --steps 3 --warmup 1 --calibrate")
    # the counter runs wrote their CSVs (<dir>/f_counter_collection.csv and
    # <dir>/w_counter_collection.csv) where the summary read them
    fdir = os.path.dirname(t.get("fetch_csv", f"pmc_fetch_{wl}/f_counter_collection.csv"))
    wdir = os.path.dirname(t.get("write_csv", f"pmc_write_{wl}/w_counter_collection.csv"))
    rq = t.get("requests")
    extra = f" {rq['rdreq_csv']} {rq['wrreq_csv']}" if rq else ""
    cmds = [
        "export TMPDIR=/tmp",
        f"timeout -s KILL 240 rocprofv3 --pmc FETCH_SIZE --output-format csv -d {fdir} -o f -- {run}",
        f"timeout -s KILL 240 rocprofv3 --pmc WRITE_SIZE --output-format csv -d {wdir} -o w -- {run}",
        f"python3 bench.py --summarize-pmc {fdir}/f_counter_collection.csv "
        f"{wdir}/w_counter_collection.csv {wl}{extra} > profiles/page_copy_{wl}_traffic.json",
        f"python3 bench.py --pmc-markdown profiles/page_copy_{wl}_traffic.json > profiles/page_copy_{wl}_traffic.md",
    ]
    out = [f"# {t['kernel']} on {wl} - HBM traffic per launch (rocprofv3 PMC)", "",
           "Commands (repo root, one MI355X; one counter per pass):", "", "```", *cmds, "```", "",
           "`--calibrate` runs a device copy of 1 GiB three times in the same process (torch `copy_`, "
           "dispatched as `__amd_rocclr_copyBuffer`): the reference dispatch of known size.", "",
           f"| counter | page copy kernel, KiB per dispatch (raw, {t['fetch_dispatches']} dispatches) | "
           "1 GiB copy, KiB (raw) | scale to 1 GiB | bytes per launch |", "|---|---|---|---|---|",
           f"| FETCH_SIZE | {t['fetch_kib_per_dispatch_raw']:.1f} | {t['fetch_calibration_kib_raw']:.1f} | "
           f"{t['fetch_scale']} | {t['fetch_bytes_per_launch']} |",
           f"| WRITE_SIZE | {t['write_kib_per_dispatch_raw']:.1f} | {t['write_calibration_kib_raw']:.1f} | "
           f"{t['write_scale']} | {t['write_bytes_per_launch']} |", ""]
    if alg:
        out += [f"Algorithmic bytes per launch: {alg} ({chunk} layers x {w.n_pages} pages x {w.shape.page_bytes} B, "
                "read once and written once).",
                f"Measured HBM traffic per launch: {t['traffic_bytes_per_launch']} B = "
                f"{t['traffic_bytes_per_launch'] / alg:.5f} x algorithmic: {traffic_verdict(t, alg)}"]
    if rq:
        rdir = os.path.dirname(rq["rdreq_csv"])
        qdir = os.path.dirname(rq["wrreq_csv"])
        out += ["", "Cross-check from request counts, with no scale factor (two more passes of the same run, "
                "made before the summary above):", "",
                "```",
                f"timeout -s KILL 240 rocprofv3 --pmc TCC_EA0_RDREQ_sum TCC_EA0_RDREQ_32B_sum TCC_BUBBLE_sum "
                f"--output-format csv -d {rdir} -o r -- {run}",
                f"timeout -s KILL 240 rocprofv3 --pmc TCC_EA0_WRREQ_sum TCC_EA0_WRREQ_64B_sum "
                f"--output-format csv -d {qdir} -o q -- {run}",
                "```", "",
                f"- read requests per launch {rq['rdreq']:.0f} (32-byte: {rq['rdreq_32b']:.0f}; TCC_BUBBLE "
                f"{rq['bubble']:.0f}) x 128 B = {rq['read_bytes_per_launch']} B;",
                f"- write requests per launch {rq['wrreq']:.0f} (64-byte: {rq['wrreq_64b']:.0f}) x 64 B = "
                f"{rq['write_bytes_per_launch']} B;",
                f"- together {rq['bytes_per_launch']} B = {rq['bytes_per_launch'] / alg:.5f} x algorithmic. "
                "FETCH_SIZE weighs the 128-byte read requests at 64 bytes (TCC_BUBBLE, which it uses to "
                "count them, stays 0), hence the scale of 2 above."]
    out += ["(Counter collection serialises dispatches, so runs under --pmc report lower throughput; "
            "only the byte counts are used.)"]
    return "\n".join(out) + "\n"


def traffic_from_profiles(workload: str):
    path = PROFILES / f"page_copy_{workload}_traffic.json"
    if not path.exists():
        return None
    d = json.loads(path.read_text())
    return d if d.get("workload") == workload else None


def main():
    if len(sys.argv) > 2 and sys.argv[1] == "--channel-sender":
        # the sending process of the channel leg (started by run_channel)
        channel_sender(sys.argv[2])
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize-pmc":
        # python bench.py --summarize-pmc FETCH.csv WRITE.csv WORKLOAD [RDREQ.csv WRREQ.csv]
        d = summarize_pmc(sys.argv[2], sys.argv[3], sys.argv[4])
        if len(sys.argv) > 6:
            d["requests"] = requests_per_launch(sys.argv[5], sys.argv[6])
        print(json.dumps(d, indent=1))
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--pmc-markdown":
        # python bench.py --pmc-markdown profiles/page_copy_WORKLOAD_traffic.json
        print(pmc_markdown(sys.argv[2]), end="")
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize-stats":
        # python bench.py --summarize-stats KERNEL_STATS.csv BENCH_LINE.json "COMMAND" [KERNEL_TRACE.csv]
        print(summarize_stats(*sys.argv[2:6]), end="")
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize-promote":
        # python bench.py --summarize-promote KERNEL_TRACE.csv BENCH_LINE.json "COMMAND"
        print(summarize_promote(sys.argv[2], sys.argv[3], sys.argv[4]), end="")
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize-kernel-pmc":
        # python bench.py --summarize-kernel-pmc KERNEL_SUBSTRING "COMMAND" COUNTERS.csv [COUNTERS.csv ...]
        print(summarize_kernel_pmc(sys.argv[2], sys.argv[3], sys.argv[4:]), end="")
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--only-append":
        # python bench.py --only-append: the paged-append leg alone (for profiling)
        import torch

        from paceserve_amd import _native

        _native.load()
        print(json.dumps({"append": run_append(torch.device("cuda", 0))}), flush=True)
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize-copies":
        # python bench.py --summarize-copies MEMORY_COPY_TRACE.csv KERNEL_TRACE.csv BENCH_LINE.json "COMMAND"
        print(summarize_copies(sys.argv[2], sys.argv[3], sys.argv[4], sys.argv[5]), end="")
        return
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU: the KV migration path is measured on "
                          "one device's share; --gpus N>1 is not supported"}), flush=True)
        sys.exit(2)

    import torch

    from paceserve_amd import _native, workloads

    _native.load()
    dev = torch.device("cuda", 0)
    w = workloads.get(args.workload)
    # Host-link legs first, in a process that has run no other GPU work yet.
    # How the runtime carries a stream's copies (DMA engine or blit kernel)
    # depends on the process's earlier GPU work: after some sequences of graph
    # captures and small copies, the same pinned round trip ran at 26-28 GB/s
    # per direction instead of 45-48, with the device-to-host copies carried
    # by blit kernels.  Device legs are not affected.
    staging_names = []
    if not args.no_staging:
        if args.staging or w.staging in ("pinned", "both"):
            staging_names.append(w.name)
        if not args.no_configs:
            staging_names += [n for n in workloads.NAMES
                              if n != w.name and workloads.get(n).staging in ("pinned", "both")]
    promote = None
    early_staging = {}
    # One stager for every staging leg, created before them and kept to the
    # end of the process, as a serving worker creates its own once.  With a
    # stager per leg, each leg freed the previous one's device rings, and the
    # driver scrubs freed memory with the DMA engines the next leg's H2D
    # copies need (warm legs measured 46.2-48.3 GB/s per direction over three
    # runs, against 47.6-48.0 with the one stager).
    stager = None
    if staging_names:
        from paceserve_amd.kv_transfer import kv_utils, ops

        slot = max(staging_chunk_bytes(workloads.get(n)) for n in staging_names)
        stager = ops.Stager(-(-slot // 256) * 256, kv_utils.ROUNDTRIP_SLOTS, dev)
    if staging_names or not args.no_promote:
        settle = link_settle(dev)
        log(f"host link settled after {settle['waited_s']} s at {settle['d2h_gbs']} GB/s D2H")
        if not args.no_promote:
            promote = run_promote(dev, c_caller=not args.no_c_caller)
            promote["link_probe"] = settle
        for name in staging_names:
            early_staging[name] = run_staging_leg(args, name, dev, stager)
            early_staging[name]["link_probe"] = settle
    if early_staging:
        # The staging pools go back to the driver, which scrubs them with the
        # DMA engines and HBM bandwidth: the headline waits until a D2H probe
        # runs at the link's rate again.
        torch.cuda.empty_cache()
        after = link_settle(dev)
        log(f"after the staging legs: link settled after {after['waited_s']} s at {after['d2h_gbs']} GB/s D2H")
    log(f"workload {w.name}: {w.description}")
    src, dst, plan, s_ids, d_ids = device_setup(w, dev)
    res = run_device(args, w, dev, src, dst, plan, s_ids, d_ids)
    log(f"device: {res['value']:.1f} GB/s ({res['value'] / HBM_PEAK_GBS * 100:.1f}% of peak), "
        f"pack {res['pack_ms_mean']} ms, unpack {res['unpack_ms_mean']} ms")
    if args.verify:
        res["verified"] = verify(w, src, dst, s_ids, d_ids, dev)
        log(f"verified: {res['verified']}")
    torch_dev = run_torch_device(w, dev, src, dst, s_ids, d_ids)
    append = None if args.no_append else run_append(dev)
    cpu = None
    if not args.no_cpu:
        layers = args.cpu_layers or cpu_sample_layers(w)
        log(f"CPU baseline on {os.cpu_count()} cores, {layers} layers ...")
        cpu = run_cpu_baseline(w, layers, src, dst, plan)
        log(f"CPU baseline: {cpu['value']} GB/s")
    staging = early_staging.get(w.name)
    # The identity-id ceiling writes destination pages that no id names, so it
    # runs after every check of the pools; the calibration copies come last.
    ceiling = run_ceiling(w, dev, src, dst, plan.n_pages) if args.mode == "buffer" else None
    if args.calibrate:
        run_calibration(dev)
    dropin = None
    if not args.no_dropin:
        settle = link_settle(dev)
        dropin = run_dropin(dev)
        dropin["link_probe"] = settle
    # Memory freed from here on stays in torch's cache for the later legs and
    # workloads (no empty_cache), so the driver scrubs nothing while they run.
    del src, dst, s_ids, d_ids
    channel = None
    if not args.no_channel:
        settle = link_settle(dev)
        channel = run_channel(dev)
        channel["link_probe"] = settle
    configs = None
    if not args.no_configs:
        configs = {name: run_config(args, name, dev, early_staging.get(name))
                   for name in workloads.NAMES + workloads.SHARDS if name != w.name}
    if staging is None and early_staging:
        staging = next(iter(early_staging.values()))
    # The same pinned-host legs again at the end, in a process that has run
    # every other leg: a serving worker is never a fresh process.
    staging_warm = None
    if early_staging and not args.no_warm_staging:
        staging_warm = {}
        for name in early_staging:
            settle = link_settle(dev)
            staging_warm[name] = run_staging_leg(args, name, dev, stager)
            staging_warm[name]["link_probe"] = settle
    if stager is not None:
        stager.close()

    line = {
        "metric": METRIC,
        "value": round(res["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_NAMES.get(w.shape.dtype_name, w.shape.dtype_name),
        "data": f"synthetic (seeded {INIT_NAMES[w.init]} pages generated on the GPU)",
        "config": dict(w.summary(), mode=args.mode),
        "pct_hbm_peak": round(res["value"] / HBM_PEAK_GBS * 100, 2),
        "event_ms_per_step": round(res["event_ms_per_step"], 4),
        "launch_timing_ms_per_step": round(res["launch_timing_ms_per_step"], 4),
        "pack_ms": res["pack_ms_mean"],
        "unpack_ms": res["unpack_ms_mean"],
        "roofline": res["roofline"],
        "copy_ceiling": ceiling,
        "torch_device_baseline": torch_dev,
        "append": append,
        "promote_4k": promote,
        "staging": staging,
        "staging_warm": staging_warm,
        "dropin": dropin,
        "channel": channel,
        "cpu_baseline": cpu,
        "configs": configs,
    }
    tr = traffic_from_profiles(w.name) if args.mode == "buffer" else None
    if tr is not None:
        line["roofline"]["traffic"] = tr["traffic_bytes_per_launch"]
        line["roofline"]["traffic_source"] = f"profiles/page_copy_{w.name}_traffic.json (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)"
    if "verified" in res:
        line["verified"] = res["verified"]
    if "verified" in res:
        line["verified_what"] = VERIFIED_WHAT
    if configs:
        line["configs_summary"] = {name: {"value": c["value"], "frac": c["frac_of_hbm_peak"],
                                          "verified": c.get("verified")} for name, c in configs.items()}
    if early_staging:
        # round trip GB/s per direction, first in the process and again at its end
        line["staging_summary"] = {
            name: {"fresh_gbs_per_direction": st["roundtrip_gbs_per_direction"], "fresh_verified": st.get("verified"),
                   "warm_gbs_per_direction": (staging_warm or {}).get(name, {}).get("roundtrip_gbs_per_direction"),
                   "warm_verified": (staging_warm or {}).get(name, {}).get("verified")}
            for name, st in early_staging.items()}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
