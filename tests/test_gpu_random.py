"""Seeded random batches through pack, unpack and move, checked bit-exactly
against torch's own device gather (index_select) and scatter (index_copy_):
layer counts on both sides of the 64-layer launch split, page shapes from
16 B to 256 KiB (whole and partial 1 KiB rows), four element types, pool
sizes from one page up, and batches from empty to the whole pool."""
import numpy as np
import pytest
import torch

from paceserve_amd.kv_transfer import ops

pytestmark = pytest.mark.gpu

WORD = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32,
        torch.uint8: torch.uint8}
POOL_BYTES_MAX = 48 << 20          # per pool, all layers


def words(t):
    return t.view(WORD[t.dtype])


def pool(L, pages, shape, dtype, gpu, g):
    if dtype == torch.uint8:
        return [torch.randint(0, 256, (pages,) + shape, generator=g, device=gpu, dtype=torch.uint8)
                for _ in range(L)]
    return [torch.randn((pages,) + shape, generator=g, device=gpu, dtype=torch.float32).to(dtype)
            for _ in range(L)]


@pytest.mark.parametrize("seed", range(4))
def test_random_batches_match_torch(gpu, seed):
    rng = np.random.default_rng(3000 + seed)
    g = torch.Generator(device=gpu).manual_seed(3000 + seed)
    for case in range(12):
        L = int(rng.choice([1, 2, 5, 32, 64, 65, 97]))
        shape = (2, int(rng.choice([1, 3, 16, 32])), int(rng.choice([1, 2, 8])), int(rng.choice([8, 24, 64, 128])))
        dtype = [torch.float16, torch.bfloat16, torch.float32, torch.uint8][int(rng.integers(0, 4))]
        page_bytes = int(np.prod(shape)) * torch.empty(0, dtype=dtype).element_size()
        pages = int(rng.integers(1, 300))
        pages = max(1, min(pages, POOL_BYTES_MAX // (L * page_bytes)))
        n = int(rng.integers(0, pages + 1))
        s_ids = torch.from_numpy(rng.permutation(pages)[:n].astype(np.int64)).to(gpu)
        d_ids = torch.from_numpy(rng.permutation(pages)[:n].astype(np.int64)).to(gpu)
        print(f"seed {seed} case {case}: L={L} shape={shape} {dtype} pages={pages} n={n} "
              f"page_bytes={page_bytes}", flush=True)
        src = pool(L, pages, shape, dtype, gpu, g)
        dst = pool(L, pages, shape, dtype, gpu, g)
        want_buf = torch.stack([words(s).index_select(0, s_ids) for s in src])
        want_dst = [words(d).clone().index_copy_(0, d_ids, want_buf[l]) for l, d in enumerate(dst)]

        buf = ops.pack(src, s_ids.to(torch.int32))
        unpacked = [d.clone() for d in dst]
        ops.unpack(buf, unpacked, d_ids.to(torch.int32))
        moved = [d.clone() for d in dst]
        ops.move(src, s_ids.to(torch.int32), moved, d_ids.to(torch.int32))
        torch.cuda.synchronize()
        assert torch.equal(words(buf), want_buf), f"case {case}: pack"
        for l in range(L):
            assert torch.equal(words(unpacked[l]), want_dst[l]), f"case {case}: unpack layer {l}"
            assert torch.equal(words(moved[l]), want_dst[l]), f"case {case}: move layer {l}"
