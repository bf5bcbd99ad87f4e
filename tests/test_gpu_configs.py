"""The five reference-shaped workloads at full size on the GPU, and one GPU's
share of the 70B workload under tensor parallelism 8 (8 KiB pages).

For each: plan (LIFO destination allocation + remap), move the pages through
the HIP path, then check every layer of both pools exactly, as raw bytes
(workloads.migration_mismatch): the destination layer must equal its content
before the migration, regenerated from the pool's seed, with torch's own
index_copy_ of index_select'ed source pages applied, and the source layer its
content before.  A page written twice, swapped, missed, or written where no
id points fails.  Also:
  - the 512-token request against the CPU oracle;
  - the 8 x 4095-token and 32768-token requests through the pinned-host round
    trip, and the 16-request batch through the fused move, to the same check.
"""
import gc

import numpy as np
import pytest
import torch

from oracle import kv_oracle as orc
from paceserve_amd import workloads
from paceserve_amd.core.block_manager import BlockAllocator
from paceserve_amd.kv_transfer import migrate, ops

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _free_memory():
    yield
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()


def words(t):
    return t.view(torch.int16)


def setup(c, dev):
    w = workloads.get(c)
    free_gb = torch.cuda.mem_get_info(dev)[0] / 1e9
    need_gb = (w.src_pool_pages + w.dst_pool_pages) * w.shape.num_layers * w.shape.page_bytes / 1e9
    if need_gb > 0.9 * free_gb:
        pytest.skip(f"{w.name} needs {need_gb:.0f} GB of device memory, {free_gb:.0f} GB free")
    src = ops.PagedPool(w.src_pool(dev))
    dst = ops.PagedPool(w.dst_pool(dev))
    plan = migrate.plan_batch(w.src_tables, w.src_pool_pages, BlockAllocator(16, w.dst_pool_pages))
    s_ids = torch.tensor(plan.src_ids, dtype=torch.long, device=dev)
    d_ids = torch.tensor(plan.dst_ids, dtype=torch.long, device=dev)
    return w, src, dst, plan, s_ids, d_ids


def check_after(w, src, dst, s_ids, d_ids, label):
    dev = src.device
    bad = workloads.migration_mismatch(src.layers, dst.layers, s_ids, d_ids, w.dst_before(dev), w.src_before(dev))
    assert bad is None, f"{label}: {bad}"


def run_buffer(w, src, dst, plan, dev):
    mig = migrate.KVMigrator(src, dst, BlockAllocator(16, w.dst_pool_pages))
    s32 = torch.tensor(plan.src_ids, dtype=torch.int32, device=dev)
    d32 = torch.tensor(plan.dst_ids, dtype=torch.int32, device=dev)
    mig.move_pages(s32, d32, "buffer", w.device_layers_per_chunk)
    torch.cuda.synchronize()


@pytest.mark.parametrize("c", workloads.NAMES + workloads.SHARDS)
def test_workload_buffer_path(gpu, c):
    w, src, dst, plan, s_ids, d_ids = setup(c, gpu)
    print(f"{w.name}: {plan.n_pages} pages x {w.shape.num_layers} layers", flush=True)
    small = w.payload_bytes <= 64 << 20
    if small:       # CPU oracle on the full (small) workload
        np_src = [words(s).cpu().numpy() for s in src.layers]
        np_dst = [words(d).cpu().numpy() for d in dst.layers]
        want = orc.move(np_src, plan.src_ids, np_dst, plan.dst_ids)
    run_buffer(w, src, dst, plan, gpu)
    check_after(w, src, dst, s_ids, d_ids, w.name)
    if small:
        for l in range(w.shape.num_layers):
            np.testing.assert_array_equal(words(dst.layers[l]).cpu().numpy(), want[l])


@pytest.mark.parametrize("c", ["llama2-7b-8x4095tok-fp16", "llama3-8b-32768tok-bf16"])
def test_workload_pinned_roundtrip(gpu, c):
    w, src, dst, plan, s_ids, d_ids = setup(c, gpu)
    from paceserve_amd.kv_transfer import kv_utils
    n = plan.n_pages
    k = w.layers_per_chunk or kv_utils.roundtrip_chunk_layers(w.shape.num_layers, n * w.shape.page_bytes)
    chunk = k * n * w.shape.page_bytes
    host = torch.empty(min(w.payload_bytes, 3 * chunk), dtype=torch.uint8, pin_memory=True)
    with ops.Stager(chunk, 3, gpu) as st:
        st.roundtrip(src, plan.src_ids, dst, plan.dst_ids, host, k)
        torch.cuda.synchronize()
    check_after(w, src, dst, s_ids, d_ids, f"{w.name} pinned")


def test_workload_fused_move_matches(gpu):
    w, src, dst, plan, s_ids, d_ids = setup("llama3-8b-16req-bf16", gpu)
    ops.move(src, plan.src_ids, dst, plan.dst_ids)
    torch.cuda.synchronize()
    check_after(w, src, dst, s_ids, d_ids, f"{w.name} fused")


def test_promote_4k_all_modes(gpu):
    w = workloads.get(workloads.PROMOTE)
    src = ops.PagedPool(w.src_pool(gpu))
    s_ids = torch.tensor(w.src_tables[0], dtype=torch.long, device=gpu)
    for mode in ("buffer", "fused", "pinned"):
        dst = ops.PagedPool(w.dst_pool(gpu))
        alloc = BlockAllocator(16, w.dst_pool_pages)
        mig = migrate.KVMigrator(src, dst, alloc)
        plan = mig.promote(w.src_tables, mode=mode)
        torch.cuda.synchronize()
        assert plan.dst_tables == [list(range(2047, 2047 - 256, -1))]    # fresh LIFO pool
        d_ids = torch.tensor(plan.dst_tables[0], dtype=torch.long, device=gpu)
        check_after(w, src, dst, s_ids, d_ids, f"promote {mode}")
        del dst, mig
