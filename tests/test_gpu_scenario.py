"""The path's components together, as a serving loop uses them, on one GPU:
a low-priority (LP) and a high-priority (HP) instance's caches as two pools.

  1. LP prefill: a batch of prompts appended in one launch per layer
     (append_paged_kv_cache_indptr), pages from the LP allocator;
  2. LP decode steps (the two-call form: get_seq_lens,
     get_batch_indices_positions, append_paged_kv_cache), opening a page
     whenever a sequence's last page is full;
  3. promotion of some sequences to HP (KVMigrator.promote on the native
     allocator, rotating through the buffer, fused and pinned modes), with the
     n+1 destination page when the next token opens a page, then the LP
     pages freed (paceserve/worker/base_worker.py:236-281);
  4. HP decode steps on the promoted sequences, growing into the +1 page;
  5. preemption: two HP sequences swapped out to pinned host pages
     (SwapSpace) and their device pages freed, further decode steps that
     reuse those pages, then the two swapped back into new pages
     (paceserve/engine/decode_llm_engine.py:31-41,
     paceserve/disutil/decode_instance.py:176-192);
  6. more HP decode steps, the swapped-in sequences included.

A torch model keeps every sequence's K and V rows as they were appended.  At
the end every token of every live sequence, read back through its final
block table with torch indexing, must equal the model bit for bit, on every
layer, in whichever pool the sequence lives."""
import numpy as np
import pytest
import torch

from paceserve_amd.core.block_manager import NativeBlockAllocator
from paceserve_amd.kv_transfer import append as ap
from paceserve_amd.kv_transfer import migrate, ops
from paceserve_amd.kv_transfer.swap import SwapSpace

pytestmark = pytest.mark.gpu

L, P, H, D = 4, 16, 2, 64
POOL = 256
DT = torch.bfloat16


class Instance:
    """One instance's cache (L layer tensors), its allocator and the
    sequences it holds: seq_id -> block table, and the token count."""

    def __init__(self, dev, seed):
        g = torch.Generator(device=dev).manual_seed(seed)
        self.cache = [torch.randn((POOL, 2, P, H, D), generator=g, device=dev, dtype=torch.float32).to(DT)
                      for _ in range(L)]
        self.pool = ops.PagedPool(self.cache)
        self.alloc = NativeBlockAllocator(P, POOL)
        self.tables, self.lens = {}, {}

    def append(self, model, rows, seq_ids, new_tokens, fused):
        """Appends new_tokens[i] tokens to seq_ids[i] (pages grown first),
        rows: per layer (key, value) of [sum(new_tokens), H, D]."""
        dev = self.cache[0].device
        for s, k in zip(seq_ids, new_tokens):
            need = -(-(self.lens[s] + k) // P) - len(self.tables[s])
            if need > 0:
                self.tables[s] += self.alloc.allocate_many(need)
            self.lens[s] += k
        indices = [p for s in seq_ids for p in self.tables[s]]
        kv_indptr = torch.tensor(np.cumsum([0] + [len(self.tables[s]) for s in seq_ids]), dtype=torch.int32,
                                 device=dev)
        kv_indices = torch.tensor(indices, dtype=torch.int32, device=dev)
        last = torch.tensor([self.lens[s] - (len(self.tables[s]) - 1) * P for s in seq_ids], dtype=torch.int32,
                            device=dev)
        append_indptr = torch.tensor(np.cumsum([0] + list(new_tokens)), dtype=torch.int32, device=dev)
        nnz = int(sum(new_tokens))
        for l in range(L):
            key, value = rows[l]
            if fused:
                ap.append_paged_kv_cache_indptr(key, value, append_indptr, self.cache[l], kv_indices, kv_indptr,
                                                last)
            else:
                sl = ap.get_seq_lens(kv_indptr, last, P)
                bi, pos = ap.get_batch_indices_positions(append_indptr, sl, nnz)
                ap.append_paged_kv_cache(key, value, bi, pos, self.cache[l], kv_indices, kv_indptr, last)
        model.add(seq_ids, new_tokens, rows)

    def free(self, s):
        self.alloc.free_many(reversed(self.tables.pop(s)))
        del self.lens[s]

    def check(self, model):
        dev = self.cache[0].device
        for s, tab in self.tables.items():
            T = self.lens[s]
            assert len(tab) == -(-T // P), s
            idx = torch.tensor(tab, dtype=torch.long, device=dev)
            for l in range(L):
                pages = self.cache[l][idx]                          # [n, 2, P, H, D]
                for kv in (0, 1):
                    got = pages[:, kv].reshape(len(tab) * P, H, D)[:T]
                    want = model.rows[s][l][kv]
                    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), \
                        f"sequence {s} layer {l} {'KV'[kv]}"


class Model:
    """The K and V rows of every sequence, in append order (torch only)."""

    def __init__(self):
        self.rows = {}      # seq_id -> per layer [K rows, V rows]

    def add(self, seq_ids, new_tokens, rows):
        pos = 0
        for s, k in zip(seq_ids, new_tokens):
            per = self.rows.setdefault(s, [[None, None] for _ in range(L)])
            for l in range(L):
                for kv in (0, 1):
                    chunk = rows[l][kv][pos:pos + k]
                    per[l][kv] = chunk.clone() if per[l][kv] is None else torch.cat([per[l][kv], chunk])
            pos += k


def rand_rows(g, dev, nnz):
    return [(torch.randn((nnz, H, D), generator=g, device=dev, dtype=torch.float32).to(DT),
             torch.randn((nnz, H, D), generator=g, device=dev, dtype=torch.float32).to(DT)) for _ in range(L)]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_lp_hp_promotion_decode_and_preemption(gpu, seed):
    print(f"scenario seed {seed}", flush=True)
    rng = np.random.default_rng(seed)
    g = torch.Generator(device=gpu).manual_seed(100 + seed)
    model = Model()
    lp, hp = Instance(gpu, 10 + seed), Instance(gpu, 20 + seed)

    # 1. LP prefill of 12 prompts, one fused launch per layer
    seqs = [f"s{i}" for i in range(12)]
    prompts = [int(x) for x in rng.integers(1, 100, size=len(seqs))]
    # after the three LP decode steps, the first sequence of each promotion
    # batch ends on a page boundary (its destination gets the n+1 page), and
    # s1 one token short of one
    prompts[0], prompts[1], prompts[2], prompts[4] = 29, 44, 13, 61
    for s in seqs:
        lp.tables[s], lp.lens[s] = [], 0
    lp.append(model, rand_rows(g, gpu, sum(prompts)), seqs, prompts, fused=True)

    # 2. LP decode: one token per sequence per step
    for step in range(3):
        lp.append(model, rand_rows(g, gpu, len(seqs)), seqs, [1] * len(seqs), fused=False)

    # 3. promote six sequences to HP, two per mode
    promoted = seqs[:6]
    modes = ["buffer", "fused", "pinned"]
    mig = migrate.KVMigrator(lp.pool, hp.pool, hp.alloc)
    host = torch.empty(L * POOL * lp.pool.page_bytes, dtype=torch.uint8, pin_memory=True)
    for i in range(0, len(promoted), 2):
        batch = promoted[i:i + 2]
        tables = [lp.tables[s] for s in batch]
        # the n+1 page when the next token opens one (the reference's decode side)
        dst_pages = [len(t) + (lp.lens[s] % P == 0) for s, t in zip(batch, tables)]
        plan = mig.promote(tables, dst_pages=dst_pages, mode=modes[i // 2],
                           host_buf=host if modes[i // 2] == "pinned" else None)
        for s, t in zip(batch, plan.dst_tables):
            hp.tables[s], hp.lens[s] = list(t), lp.lens[s]
            lp.free(s)
    # a promoted table holds one page more than its tokens fill exactly when
    # they fill whole pages: the next append writes into it
    extra = {s: len(hp.tables[s]) - -(-hp.lens[s] // P) for s in promoted}
    assert extra == {s: int(hp.lens[s] % P == 0) for s in promoted}
    assert extra["s0"] == extra["s2"] == extra["s4"] == 1 and extra["s1"] == 0

    # 4. HP decode of the promoted sequences; LP keeps decoding the rest
    for step in range(20):
        hp.append(model, rand_rows(g, gpu, len(promoted)), promoted, [1] * len(promoted), fused=step % 2 == 0)
        rest = [s for s in seqs if s in lp.tables]
        if step % 5 == 0:
            lp.append(model, rand_rows(g, gpu, len(rest)), rest, [1] * len(rest), fused=True)

    # 5. preempt two HP sequences to host memory; their pages are reused
    space = SwapSpace(hp.pool, num_host_pages=64)
    victims = promoted[1:3]
    parked = {}
    for s in victims:
        space.swap_out(s, hp.tables[s])
        parked[s] = hp.lens[s]
        hp.free(s)
    running = [s for s in promoted if s not in victims]
    for step in range(10):
        hp.append(model, rand_rows(g, gpu, 3 * len(running)), running, [3] * len(running), fused=step % 2 == 1)
    for s in victims:
        n = -(-parked[s] // P)
        table = hp.alloc.allocate_many(n)
        space.swap_in(s, table)
        hp.tables[s], hp.lens[s] = table, parked[s]
    assert space.num_free_host_pages() == 64

    # 6. every HP sequence decodes on
    for step in range(5):
        hp.append(model, rand_rows(g, gpu, len(promoted)), promoted, [1] * len(promoted), fused=True)

    torch.cuda.synchronize()
    lp.check(model)
    hp.check(model)
    assert set(hp.tables) == set(promoted) and set(lp.tables) == set(seqs[6:])
