"""KVhelper and the worker methods on the GPU: the reference's interface,
return values and error conventions over the HIP path, checked against the
oracle and torch's own indexing."""
import numpy as np
import pytest
import torch

from oracle import kv_oracle as orc
from paceserve_amd.core.kv_cache_obj import KVobj
from paceserve_amd.core.sequence import Sequence
from paceserve_amd.kv_transfer.kv_utils import KVhelper
from paceserve_amd.kv_transfer.worker import KVStatus, KVWorker, WorkerSequenceManager

pytestmark = pytest.mark.gpu

L, H, D, P, POOL = 4, 8, 128, 16, 64


class ModelConfig:
    def __init__(self, dtype):
        self.dtype = dtype

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


class _Wrapper:
    def __init__(self, cache):
        self.gpu_cache = cache


class _Runner:
    def __init__(self, cache):
        self.attention_backend_wrapper = _Wrapper(cache)


def make_helper(dev, dtype=torch.float16, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    cache = [torch.randn(POOL, 2, P, H, D, generator=g, device=dev, dtype=torch.float32).to(dtype)
             for _ in range(L)]
    h = KVhelper(0, ModelConfig(dtype), CacheConfig(), None)
    h.add_model_runner(_Runner(cache))
    return h, cache


def words(t):
    return t.view(torch.int16)


class _SeqManager:
    def __init__(self, table):
        self.table = table

    def _get_block_table(self, seq):
        if self.table is None:
            raise KeyError(seq.seq_id)
        return self.table


def test_get_kv_cache_matches_reference_gather(gpu):
    h, cache = make_helper(gpu)
    seq = Sequence.of_length("s", 100, P)
    table = [17, 3, 60, 8, 41, 22, 9]
    out, ids = h.get_kv_cache(seq, _SeqManager(table))
    assert ids == table
    assert out.device.type == "cpu" and out.shape == (L, 7, 2, P, H, D)
    for l in range(L):
        ref = cache[l][torch.tensor(table, device=gpu)].cpu()       # the reference's gather
        assert torch.equal(words(out[l]), words(ref))


def test_get_kv_cache_zero_fallback(gpu, capsys):
    h, _ = make_helper(gpu)
    seq = Sequence.of_length("s", 10, P)
    out, ids = h.get_kv_cache(seq, _SeqManager(None))
    assert ids == [0] and out.shape == (L, 1, 2, P, H, D) and not out.any()
    assert "was not allocated any memory" in capsys.readouterr().out
    out2, ids2 = h.get_kv_cache(seq, _SeqManager([]))
    assert ids2 == [0] and not out2.any()


def test_get_kv_cache_out_of_range_raises(gpu):
    h, _ = make_helper(gpu)
    with pytest.raises(IndexError):
        h.get_kv_cache(Sequence.of_length("s", 10, P), _SeqManager([POOL]))


def test_insert_kv_cache_matches_reference_scatter(gpu):
    h, cache = make_helper(gpu, torch.bfloat16, seed=1)
    content = torch.randn(L, 5, 2, P, H, D, dtype=torch.float32).to(torch.bfloat16)
    ids = [7, 63, 0, 12, 30]
    expect = [words(c).clone() for c in cache]
    for l in range(L):
        expect[l][torch.tensor(ids, device=gpu)] = words(content[l]).to(gpu)
    assert h.insert_kv_cache(content, ids, gpu) is True
    for l in range(L):
        assert torch.equal(words(cache[l]), expect[l])
    # pinned host content and device content take the same path results
    dev_content = content.to(gpu)
    h2, cache2 = make_helper(gpu, torch.bfloat16, seed=1)
    assert h2.insert_kv_cache(dev_content, ids, "cuda:0") is True
    for l in range(L):
        assert torch.equal(words(cache2[l]), expect[l])


def test_insert_kv_cache_negative_repeated_and_broadcast(gpu):
    h, cache = make_helper(gpu, seed=2)
    np_cache = [words(c).cpu().numpy() for c in cache]
    content = torch.randn(L, 3, 2, P, H, D).half()
    ids = [5, -1, 5]                               # -1 wraps; page 5 written twice
    assert h.insert_kv_cache(content, ids, gpu)
    want = orc.unpack(words(content).numpy(), np_cache, ids)
    for l in range(L):
        np.testing.assert_array_equal(words(cache[l]).cpu().numpy(), want[l])
    one = torch.randn(L, 1, 2, P, H, D).half()    # a single page broadcasts
    assert h.insert_kv_cache(one, [1, 2], gpu)
    for l in range(L):
        assert torch.equal(words(cache[l][1]).cpu(), words(one[l, 0]))
        assert torch.equal(words(cache[l][2]).cpu(), words(one[l, 0]))


@pytest.mark.parametrize("bad", ["empty", "dtype", "count", "range", "shape", "cpu"])
def test_insert_kv_cache_errors_return_false(gpu, capsys, bad):
    h, cache = make_helper(gpu, seed=3)
    before = [words(c).clone() for c in cache]
    content = torch.randn(L, 2, 2, P, H, D).half()
    ids, dev = [1, 2], gpu
    if bad == "empty":
        ids = []
    elif bad == "dtype":
        content = content.float()
    elif bad == "count":
        ids = [1, 2, 3]
    elif bad == "range":
        ids = [1, POOL]
    elif bad == "shape":
        content = torch.randn(L, 2, 2, P, H, D // 2).half()
    elif bad == "cpu":
        dev = "cpu"
    assert h.insert_kv_cache(content, ids, dev) is False
    assert "error during insert kv cache" in capsys.readouterr().out
    for l in range(L):
        assert torch.equal(words(cache[l]), before[l])


def test_reset_kv_cache(gpu):
    h, cache = make_helper(gpu)
    h.reset_kv_cache(10)
    new = h.model_runner.attention_backend_wrapper.gpu_cache
    assert all(t.shape == (10, 2, P, H, D) and not t.any() for t in new[:L])
    out, _ = h.get_kv_cache(Sequence.of_length("s", 20, P), _SeqManager([3, 4]))
    assert not out.any()


@pytest.mark.parametrize("tokens_src,tokens_dst", [(40, 40), (48, 49)])
def test_worker_migration_end_to_end(gpu, tokens_src, tokens_dst):
    """prefill-side get (frees source pages) -> KVobj -> decode-side insert with
    LIFO allocation and the n / n+1 remap; the extra page stays untouched."""
    src_h, src_cache = make_helper(gpu, seed=4)
    dst_h, dst_cache = make_helper(gpu, seed=5)
    src_sm = WorkerSequenceManager(P, POOL, free_list=np.random.default_rng(4).permutation(POOL).tolist())
    dst_sm = WorkerSequenceManager(P, POOL)
    src_w, dst_w = KVWorker(src_h, src_sm), KVWorker(dst_h, dst_sm)
    seq = Sequence.of_length("r", tokens_src, P)
    src_sm.add_seq(seq)
    src_sm.block_manager.allocate(seq)
    src_table = src_sm._get_block_table(seq)
    free_before = src_sm.block_manager.get_num_free_gpu_blocks()
    kv_cache, kv_indices, rank = src_w._get_kv_cache(seq)
    assert kv_indices == src_table and rank == 0
    assert src_sm.block_manager.get_num_free_gpu_blocks() == free_before + len(src_table)
    obj = KVobj(seq.seq_id, kv_cache, kv_indices)
    # the decode side's sequence holds the prompt and the first generated token(s)
    dst_seq = Sequence.of_length("r", tokens_src, P, tokens_dst - tokens_src)
    dst_before = [words(c).clone() for c in dst_cache]
    st = dst_w._insert_kv_cache(dst_seq, obj, gpu)
    assert isinstance(st, KVStatus) and st.status
    dst_table = dst_sm._get_block_table(dst_seq)
    n = len(src_table)
    assert dst_table[:n] == list(range(POOL - 1, POOL - 1 - n, -1))
    for l in range(L):
        assert torch.equal(words(dst_cache[l][torch.tensor(dst_table[:n], device=gpu)]),
                           words(src_cache[l][torch.tensor(src_table, device=gpu)]))
        untouched = sorted(set(range(POOL)) - set(dst_table[:n]))
        assert torch.equal(words(dst_cache[l][untouched]), dst_before[l][untouched])


def test_concurrent_inserts_and_gets_from_worker_threads(gpu):
    # The reference inserts from up to 8 threads of one worker at once
    # (decode_instance.py:50-51, Ray max_concurrency=8).  Requests of
    # different sizes make later calls grow the shared staging pipeline
    # while other threads wait for it.
    import threading

    h, cache = make_helper(gpu, torch.bfloat16, seed=7)
    src_h, src_cache = make_helper(gpu, torch.bfloat16, seed=8)
    perm = np.random.default_rng(9).permutation(POOL).tolist()
    sizes = [1, 3, 8, 2, 12, 5, 9, 4]                      # 44 pages, disjoint
    tables, pos = [], 0
    for k in sizes:
        tables.append(perm[pos:pos + k])
        pos += k
    contents = [torch.randn(L, k, 2, P, H, D).to(torch.bfloat16) for k in sizes]
    contents = [c.pin_memory() if i % 2 == 0 else c for i, c in enumerate(contents)]   # pinned and pageable
    got, errors = {}, []

    def insert(i):
        try:
            if not h.insert_kv_cache(contents[i], tables[i], gpu):
                errors.append((i, "insert returned False"))
            out, ids = src_h.get_kv_cache(Sequence.of_length(f"s{i}", 16 * sizes[i], P), _SeqManager(tables[i]))
            got[i] = out
        except Exception as e:                             # reported by the main thread
            errors.append((i, repr(e)))

    ts = [threading.Thread(target=insert, args=(i,)) for i in range(len(sizes))]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i, table in enumerate(tables):
        idx = torch.tensor(table, device=gpu)
        for l in range(L):
            assert torch.equal(words(cache[l][idx]).cpu(), words(contents[i][l])), f"insert {i} layer {l}"
            assert torch.equal(words(got[i][l]), words(src_cache[l][idx]).cpu()), f"get {i} layer {l}"
