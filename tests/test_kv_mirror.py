"""The engine's mirror of a reference-style cache (specfold_amd.kv_cache.ContiguousMirror),
on the CPU: it copies a transformers DynamicCache (or a list of per-layer (k, v)) into
fixed buffers with the length in device memory, copies again exactly when the cache's
length or a layer's storage changes (a torch.cat commit, a crop, another cache), and
hands the attention kernels a view of capacity-strided heads over the same keys."""

import torch

from specfold_amd.kv_cache import ContiguousMirror, cache_length, prefix_view


def _dyn(L, Hkv, P, hd, seed):
    from transformers.cache_utils import DynamicCache
    g = torch.Generator().manual_seed(seed)
    c = DynamicCache()
    for li in range(L):
        c.update(torch.randn(1, Hkv, P, hd, generator=g).to(torch.bfloat16),
                 torch.randn(1, Hkv, P, hd, generator=g).to(torch.bfloat16), li)
    return c, g


def _check_same(m, cache, L):
    P = cache_length(cache)
    assert m.length == P and int(m.length_dev.item()) == P
    for li in range(L):
        ref = prefix_view(cache, li)
        mv = m.view(li)
        assert mv.page_table is None and mv.capacity == m.capacity
        assert mv.head_stride == m.capacity * m.hd and mv.length_dev is m.length_dev
        assert torch.equal(mv.k[:, :P], ref.k) and torch.equal(mv.v[:, :P], ref.v)


def test_mirror_follows_commits_and_crops():
    L, Hkv, hd = 3, 2, 8
    cache, g = _dyn(L, Hkv, 20, hd, 1)
    m = ContiguousMirror(L, Hkv, hd, 64, device="cpu")
    assert m.sync(cache) is True
    _check_same(m, cache, L)
    assert m.sync(cache) is False            # unchanged: no copy
    # a block commit grows every layer by torch.cat (new storage, longer)
    for li in range(L):
        cache.update(torch.randn(1, Hkv, 8, hd, generator=g).to(torch.bfloat16),
                     torch.randn(1, Hkv, 8, hd, generator=g).to(torch.bfloat16), li)
    assert m.sync(cache) is True
    _check_same(m, cache, L)
    # crop back and commit other tokens to the same length: the storage moved
    cache.crop(20)
    for li in range(L):
        cache.update(torch.randn(1, Hkv, 8, hd, generator=g).to(torch.bfloat16),
                     torch.randn(1, Hkv, 8, hd, generator=g).to(torch.bfloat16), li)
    assert cache_length(cache) == 28
    assert m.sync(cache) is True
    _check_same(m, cache, L)
    # another sequence's cache (a list of per-layer tensors) at a shorter length
    other = [(torch.randn(1, Hkv, 5, hd).to(torch.bfloat16),
              torch.randn(1, Hkv, 5, hd).to(torch.bfloat16)) for _ in range(L)]
    assert m.sync(other) is True
    _check_same(m, other, L)
    m.invalidate()
    assert m.sync(other) is True


def test_mirror_rejects_a_longer_prefix():
    L, Hkv, hd = 2, 2, 8
    cache, _ = _dyn(L, Hkv, 40, hd, 2)
    m = ContiguousMirror(L, Hkv, hd, 32, device="cpu")
    try:
        m.sync(cache)
    except ValueError as e:
        assert "capacity" in str(e)
    else:
        raise AssertionError("a prefix longer than the capacity must be refused")


def test_mirror_resyncs_new_objects_on_reused_storage():
    """The drop-in path: the reference loop builds a fresh cache per generate
    call.  A new cache object (or new per-layer tensors in the same container)
    on the storage the old one used, at the same length, holds other contents:
    the mirror must copy again, though the length and every data pointer are
    unchanged (an id()-based key could also match, once CPython reuses the id)."""
    L, Hkv, hd, P = 2, 2, 8, 12
    g = torch.Generator().manual_seed(5)
    store = [(torch.randn(1, Hkv, P, hd, generator=g).to(torch.bfloat16),
              torch.randn(1, Hkv, P, hd, generator=g).to(torch.bfloat16)) for _ in range(L)]
    cache = [(k, v) for k, v in store]
    m = ContiguousMirror(L, Hkv, hd, 32, device="cpu")
    assert m.sync(cache) is True
    assert m.sync(cache) is False
    # the same list object (same id), new tensor objects over the same storage,
    # rewritten with other values
    for li in range(L):
        k, v = store[li]
        k2, v2 = k.view_as(k), v.view_as(v)
        k2.copy_(torch.randn(k.shape, generator=g))
        v2.copy_(torch.randn(v.shape, generator=g))
        cache[li] = (k2, v2)
    assert ContiguousMirror.signature(cache, L) == m._sig    # length and pointers unchanged
    assert m.sync(cache) is True
    _check_same(m, cache, L)
    # a DynamicCache dropped and a new one built on the same storage
    dyn, _ = _dyn(L, Hkv, P, hd, 6)
    assert m.sync(dyn) is True
    from transformers.cache_utils import DynamicCache
    layers = [(dyn.layers[li].keys, dyn.layers[li].values) for li in range(L)]
    del dyn
    dyn2 = DynamicCache()
    for li, (k, v) in enumerate(layers):
        k.mul_(-1)
        dyn2.update(k.view_as(k), v.view_as(v), li)
    assert m.sync(dyn2) is True
    _check_same(m, dyn2, L)
    assert m.sync(dyn2) is False
