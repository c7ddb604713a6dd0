"""sf_kv_append: the paged in-place append reads back byte-equal to the
reference's torch.cat growth (DynamicCache.update), for sequential and
shuffled page orders and for appends that straddle page boundaries."""

import pytest
import torch

from specfold_amd.kv_cache import PagedKVCache

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("order", ["sequential", "shuffled"])
@pytest.mark.parametrize("page", [16, 32])
def test_append_equals_cat(order, page):
    L, Hkv, hd = 3, 4, 128
    gen = torch.Generator().manual_seed(page)
    cache = PagedKVCache(L, Hkv, hd, capacity=512, page_size=page, device="cuda",
                         page_order=order, seed=3)
    P0 = 37
    pre = [(torch.randn(1, Hkv, P0, hd, generator=gen).to(torch.bfloat16),
            torch.randn(1, Hkv, P0, hd, generator=gen).to(torch.bfloat16)) for _ in range(L)]
    cache.load_dense(pre)
    ref = [list(kv) for kv in pre]
    for step, n_tok in enumerate((32, 5, 32, 1)):
        kv_buf = torch.randn(n_tok + 3, 2 * Hkv * hd, generator=gen).to(torch.bfloat16)
        for li in range(L):
            cache.append_rows(li, kv_buf.cuda(), 2, n_tok)
            rows = kv_buf[2:2 + n_tok].view(n_tok, 2, Hkv, hd)
            ref[li][0] = torch.cat([ref[li][0], rows[:, 0].permute(1, 0, 2).unsqueeze(0)], dim=2)
            ref[li][1] = torch.cat([ref[li][1], rows[:, 1].permute(1, 0, 2).unsqueeze(0)], dim=2)
        cache.advance(n_tok)
        torch.cuda.synchronize()
        for li in range(L):
            k, v = cache[li]
            assert torch.equal(k.cpu().view(torch.int16), ref[li][0].view(torch.int16))
            assert torch.equal(v.cpu().view(torch.int16), ref[li][1].view(torch.int16))


def test_append_full_cache_raises():
    cache = PagedKVCache(1, 1, 128, capacity=32, page_size=16, device="cuda")
    kv = torch.zeros(40, 256, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        cache.append_rows(0, kv, 0, 33)
