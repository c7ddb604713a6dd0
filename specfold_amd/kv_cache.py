"""Paged prefix KV cache for the verify step.

Keeps the indexing contract the reference's verify step reads from its
``DynamicCache`` (specfold/generate/fastdllm_v2_folded.py:104, 122:
``get_seq_length()``, ``len(cache)``, ``cache[li] -> (k, v)`` as
``[1, Hkv, P, hd]``), but stores every layer's K and V in fixed pages of
``page_size`` tokens, ``[num_pages, Hkv, page_size, hd]`` bf16, addressed through
one page table shared by all layers.  Growth is an in-place append of the new
tokens (``sf_kv_append``) instead of the reference's ``torch.cat`` of the whole
cache (specfold/model_cache/nemotron_labs_diffusion/modeling_ministral.py:154-162).

``page_order="shuffled"`` stores logical page i in a seeded random physical
page, which must not change any result.
"""

from __future__ import annotations

import weakref
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch

from specfold_amd import _lib


@dataclass
class PrefixView:
    """What the attention kernel needs to address one layer's prefix."""
    k: Optional[torch.Tensor]
    v: Optional[torch.Tensor]
    page_table: Optional[torch.Tensor]
    length: int
    page_size: int
    page_stride: int
    head_stride: int
    capacity: int = 0                        # grid / workspace size when length_dev is used
    length_dev: Optional[torch.Tensor] = None  # device int32[1] copy of length


class PagedKVCache:
    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, capacity: int,
                 page_size: int = 16, device="cuda", dtype=torch.bfloat16,
                 page_order: str = "sequential", seed: int = 0):
        if page_order not in ("sequential", "shuffled"):
            raise ValueError(f"unknown page_order {page_order!r}")
        self.num_layers = num_layers
        self.Hkv = num_kv_heads
        self.hd = head_dim
        self.page_size = page_size
        self.num_pages = (capacity + page_size - 1) // page_size
        self.capacity = self.num_pages * page_size
        self.device = torch.device(device)
        shape = (num_layers, self.num_pages, num_kv_heads, page_size, head_dim)
        self.k_pages = torch.zeros(shape, dtype=dtype, device=self.device)
        self.v_pages = torch.zeros(shape, dtype=dtype, device=self.device)
        if page_order == "shuffled":
            g = torch.Generator().manual_seed(seed)
            perm = torch.randperm(self.num_pages, generator=g)
        else:
            perm = torch.arange(self.num_pages)
        self.page_table_cpu = perm.to(torch.int32)
        self.page_table = self.page_table_cpu.to(self.device)
        self.length = 0
        # device copy of the length, read by the attention kernel (graph-stable)
        self.length_dev = torch.zeros(1, dtype=torch.int32, device=self.device)

    # -- the reference cache contract ------------------------------------------------
    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.length

    def __len__(self) -> int:
        return self.num_layers

    def __getitem__(self, li: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """Logical-order copy of layer li as ([1, Hkv, P, hd], [1, Hkv, P, hd])."""
        return self.gather(li, self.k_pages), self.gather(li, self.v_pages)

    def gather(self, li: int, pages: torch.Tensor) -> torch.Tensor:
        P = self.length
        npg = (P + self.page_size - 1) // self.page_size
        idx = self.page_table[:npg].long()
        x = pages[li].index_select(0, idx)                      # [npg, Hkv, ps, hd]
        x = x.permute(1, 0, 2, 3).reshape(self.Hkv, npg * self.page_size, self.hd)
        return x[:, :P].unsqueeze(0).contiguous()

    # -- kernel views ------------------------------------------------------------------
    def view(self, li: int) -> PrefixView:
        ps, hd = self.page_size, self.hd
        return PrefixView(k=self.k_pages[li], v=self.v_pages[li], page_table=self.page_table,
                          length=self.length, page_size=ps, page_stride=self.Hkv * ps * hd,
                          head_stride=ps * hd, capacity=self.capacity,
                          length_dev=self.length_dev)

    def append_rows(self, li: int, kv_buf: torch.Tensor, row0: int, n_tok: int,
                    start_pos: Optional[int] = None) -> None:
        """Write n_tok kv_buf rows (k heads, then v heads) at start_pos.. of layer li."""
        pos = self.length if start_pos is None else start_pos
        if pos + n_tok > self.capacity:
            raise ValueError(f"KV cache full: {pos}+{n_tok} > capacity {self.capacity}")
        vw = self.view(li)
        _lib.kv_append(kv_buf, row0, n_tok, self.Hkv, self.hd, vw.k, vw.v, vw.page_table,
                       vw.page_size, vw.page_stride, vw.head_stride, pos)

    def advance(self, n_tok: int) -> None:
        if self.length + n_tok > self.capacity:
            raise ValueError("KV cache full")
        self.length += n_tok
        self.length_dev.fill_(self.length)

    def load_dense(self, kv: Sequence[Tuple[torch.Tensor, torch.Tensor]]) -> None:
        """Fill from per-layer ([1, Hkv, P, hd], [1, Hkv, P, hd]) tensors (any device)."""
        P = int(kv[0][0].shape[-2])
        if P > self.capacity:
            raise ValueError("prefix longer than capacity")
        ps = self.page_size
        npg = (P + ps - 1) // ps
        idx = self.page_table[:npg].long()
        for li, (k, v) in enumerate(kv):
            for src, dst in ((k, self.k_pages), (v, self.v_pages)):
                x = src[0].to(self.device, dst.dtype)                    # [Hkv, P, hd]
                pad = npg * ps - P
                if pad:
                    x = torch.cat([x, x.new_zeros(self.Hkv, pad, self.hd)], dim=1)
                x = x.reshape(self.Hkv, npg, ps, self.hd).permute(1, 0, 2, 3)
                dst[li].index_copy_(0, idx, x.contiguous())
        self.length = P
        self.length_dev.fill_(P)


class ContiguousMirror:
    """Engine-owned contiguous copy of a reference-style cache (the reference's
    ``DynamicCache``, which grows by ``torch.cat`` and so moves every layer's
    tensors at each commit: fastdllm_v2_folded.py:122 reads it per layer).

    K and V of every layer live in fixed buffers ``[L, Hkv, capacity, hd]`` with the
    length in device memory, so a verify step captured against the mirror stays
    valid while the reference cache grows: one capture per step shape instead of
    one per commit.  ``sync`` copies the whole prefix again unless the cache is the
    very object last synced, holding the very same per-layer tensor objects at the
    same length and storage: identity is kept by weak references (to the cache
    where it allows one, and to every layer's K and V tensor), never by ``id()``,
    which CPython hands to a new object once the old one is freed, just as the
    caching allocator hands its blocks to new tensors.  A cache rewritten in place
    at the same length and the same tensors is not detected (call ``invalidate``
    after such an update)."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, capacity: int,
                 device="cuda", dtype=torch.bfloat16):
        self.num_layers = num_layers
        self.Hkv = num_kv_heads
        self.hd = head_dim
        self.capacity = int(capacity)
        self.device = torch.device(device)
        shape = (num_layers, num_kv_heads, self.capacity, head_dim)
        self.k = torch.zeros(shape, dtype=dtype, device=self.device)
        self.v = torch.zeros(shape, dtype=dtype, device=self.device)
        self.length = 0
        self.length_dev = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._sig = None
        self._refs: tuple = ()

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.length

    def __len__(self) -> int:
        return self.num_layers

    def invalidate(self) -> None:
        self._sig = None
        self._refs = ()

    @staticmethod
    def signature(cache, num_layers: int) -> tuple:
        views = [prefix_view(cache, li) for li in range(num_layers)]
        return (cache_length(cache),
                tuple((0, 0) if pv is None else (pv.k.data_ptr(), pv.v.data_ptr())
                      for pv in views))

    @staticmethod
    def _identity(cache, num_layers: int) -> tuple:
        """The objects whose identity the mirror's contents stand for: the cache
        (when it can be weakly referenced; a list cannot) and each layer's K and V
        tensor objects as the cache holds them."""
        objs = [cache] if _weakrefable(cache) else [None]
        for li in range(num_layers):
            objs.extend(layer_kv(cache, li))
        return tuple(objs)

    def _same_objects(self, objs: tuple) -> bool:
        if len(objs) != len(self._refs):
            return False
        for o, r in zip(objs, self._refs):
            if (o is None) != (r is None) or (r is not None and r() is not o):
                return False
        return True

    def sync(self, cache) -> bool:
        """Make the mirror hold ``cache``'s prefix; returns True if it copied."""
        sig = self.signature(cache, self.num_layers)
        objs = self._identity(cache, self.num_layers)
        if sig == self._sig and self._same_objects(objs):
            return False
        P = sig[0]
        if P > self.capacity:
            raise ValueError(f"prefix of {P} keys exceeds the mirror's capacity {self.capacity}")
        for li in range(self.num_layers):
            pv = prefix_view(cache, li)
            if pv is None:
                continue
            self.k[li, :, :P].copy_(pv.k)
            self.v[li, :, :P].copy_(pv.v)
        self.length = P
        self.length_dev.fill_(P)
        self._sig = sig
        self._refs = tuple(None if o is None else weakref.ref(o) for o in objs)
        return True

    def view(self, li: int) -> PrefixView:
        return PrefixView(k=self.k[li], v=self.v[li], page_table=None, length=self.length,
                          page_size=max(self.capacity, 1), page_stride=0,
                          head_stride=self.capacity * self.hd, capacity=self.capacity,
                          length_dev=self.length_dev)


def contiguous_view(k: torch.Tensor, v: torch.Tensor) -> PrefixView:
    """Kernel view of a reference-style contiguous [1, Hkv, P, hd] layer cache."""
    if k.dim() != 4 or k.shape[0] != 1:
        raise ValueError("expected [1, Hkv, P, hd]")
    k0, v0 = k[0], v[0]
    if not (k0.is_contiguous() and v0.is_contiguous()):
        k0, v0 = k0.contiguous(), v0.contiguous()
    P, hd = k0.shape[1], k0.shape[2]
    return PrefixView(k=k0, v=v0, page_table=None, length=P, page_size=max(P, 1), page_stride=0,
                      head_stride=P * hd)


def cache_length(cache) -> int:
    """Prefix length of a PagedKVCache, a DynamicCache-like object or a list of (k, v)."""
    if cache is None:
        return 0
    if hasattr(cache, "get_seq_length"):
        return int(cache.get_seq_length())
    if len(cache) == 0 or cache[0][0] is None:
        return 0
    return int(cache[0][0].shape[-2])


def _weakrefable(obj) -> bool:
    try:
        weakref.ref(obj)
    except TypeError:
        return False
    return True


def layer_kv(cache, li: int) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
    """Layer li's (k, v) tensor objects as a reference-style cache holds them
    (a transformers DynamicCache, old or new API, or a list of per-layer pairs);
    (None, None) past its layers."""
    if len(cache) <= li:
        return None, None
    if hasattr(cache, "layers") and not hasattr(cache, "__getitem__"):
        return cache.layers[li].keys, cache.layers[li].values   # transformers>=5 DynamicCache
    return cache[li][0], cache[li][1]


def prefix_view(cache, li: int) -> Optional[PrefixView]:
    """Kernel view of layer li of either a PagedKVCache or a reference-style cache."""
    if cache is None:
        return None
    if isinstance(cache, (PagedKVCache, ContiguousMirror)):
        return cache.view(li)
    k, v = layer_kv(cache, li)
    if k is None or k.shape[-2] == 0:
        return None
    return contiguous_view(k, v)
