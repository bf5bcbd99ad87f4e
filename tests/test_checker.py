"""The exact whole-layer migration check (workloads.migration_mismatch) on
small CPU pools: it accepts a correct migration and rejects planted mistakes,
including ones a sum of words cannot see (two pages swapped, two words of a
page swapped).  The GPU tests and bench.py check every full-size workload
with it."""
import pytest
import torch

from paceserve_amd import workloads


def small_workload(dtype=torch.bfloat16):
    shape = workloads.KVShape(num_layers=3, num_kv_heads=2, head_dim=8, page_size=4, dtype=dtype)
    # two requests over a 12-page source pool; destination pool of 10 pages
    return workloads.Workload("small", "checker test", shape, 12, 10, [9, 4], [[7, 2, 11], [5]], seed=77)


def migrate_cpu(w, src_ids, dst_ids):
    """The reference's gather then scatter with torch on CPU tensors."""
    src, dst = w.src_pool("cpu"), w.dst_pool("cpu")
    si, di = torch.tensor(src_ids), torch.tensor(dst_ids)
    for s, d in zip(src, dst):
        d.index_copy_(0, di, s.index_select(0, si))
    return src, dst, si, di


def mismatch(w, src, dst, si, di):
    return workloads.migration_mismatch(src, dst, si, di, w.dst_before("cpu"), w.src_before("cpu"))


SRC_IDS = [7, 2, 11, 5]
DST_IDS = [9, 8, 7, 6]          # a fresh LIFO pool's pages; page 5 is the untouched n+1 page


def test_pool_layers_regenerate_fill_pool():
    w = small_workload()
    for a, b in zip(w.dst_pool("cpu"), w.dst_before("cpu")):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    for a, b in zip(w.src_pool("cpu"), w.src_before("cpu")):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_correct_migration_passes(dtype):
    w = small_workload(dtype)
    assert mismatch(w, *migrate_cpu(w, SRC_IDS, DST_IDS)) is None


def plant(name, src, dst):
    l = 1
    if name == "untouched pages swapped":
        dst[l][[0, 1]] = dst[l][[1, 0]]
    elif name == "touched pages swapped":
        dst[l][[9, 8]] = dst[l][[8, 9]]
    elif name == "words of one page swapped":       # the page's sum is unchanged
        flat = dst[l][9].view(-1)
        flat[[0, 1]] = flat[[1, 0]].clone()
    elif name == "stray write to an untouched page":
        dst[l][3].view(-1)[5] += 1
    elif name == "n+1 page overwritten":
        dst[l][5] = src[l][5]
    elif name == "source page written":
        src[l][2].view(-1)[0] -= 1
    elif name == "one page missed":                 # page 7 of the last layer keeps its old bytes
        dst[2][7] = small_workload().dst_pool("cpu")[2][7]
    elif name == "last layer not written":
        dst[2].copy_(small_workload().dst_pool("cpu")[2])
    else:
        raise ValueError(name)


PLANTED = ["untouched pages swapped", "touched pages swapped", "words of one page swapped",
           "stray write to an untouched page", "n+1 page overwritten", "source page written", "one page missed",
           "last layer not written"]


@pytest.mark.parametrize("name", PLANTED)
def test_planted_mistake_fails(name):
    w = small_workload()
    src, dst, si, di = migrate_cpu(w, SRC_IDS, DST_IDS)
    # the pools must really differ from the correct result (a planted swap of
    # two identical pages would test nothing)
    ok_src, ok_dst, _, _ = migrate_cpu(w, SRC_IDS, DST_IDS)
    plant(name, src, dst)
    changed = any(not torch.equal(a.view(torch.int16), b.view(torch.int16))
                  for a, b in zip(src + dst, ok_src + ok_dst))
    assert changed, name
    msg = mismatch(w, src, dst, si, di)
    assert msg is not None, name
    assert msg.startswith("layer "), msg


def test_message_names_layer_and_pages():
    w = small_workload()
    src, dst, si, di = migrate_cpu(w, SRC_IDS, DST_IDS)
    dst[1][[0, 1]] = dst[1][[1, 0]]
    assert mismatch(w, src, dst, si, di) == "layer 1: destination pages [0, 1] differ"
    src, dst, si, di = migrate_cpu(w, SRC_IDS, DST_IDS)
    src[2][4].view(-1)[0] += 1
    assert mismatch(w, src, dst, si, di) == "layer 2: source pages [4] differ"
