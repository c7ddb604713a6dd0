"""Folded multi-branch verify step on MI355X.

``FoldedVerifyEngine.forward`` runs SpecFold's verify step for B1 = 1 + B
branches of one N-token block over a prefix KV cache, all layers, and returns
the (unshifted) logits.  Per layer (reference: specfold/generate/
fastdllm_v2_folded.py:296-361 for the launch sequence, :117-220 for the math):

  sf_fold_gate       gate + compaction + src + input RMSNorm   (HIP)
  sf_qkv_rope        QKV MFMA GEMM + bias + RoPE + scatter     (HIP)
  sf_kv_append       optional in-place append (block commit)   (HIP)
  sf_attn_prefix_block  prefix + block attention with (m, Z)   (HIP)
  sf_chain_correct   folded rows' exact softmax update         (HIP)
  o_proj + residual, FFN on the compacted rows, hidden update  (torch/hipBLASLt)

Nothing here syncs with the host inside the layer loop: ``count`` stays on the
device and every kernel reads it.  The only host syncs are the parent map
(one D2H of the tokens, as the reference) and one read of the per-layer counts
after the last layer (fold statistics and bucket-overflow detection).
"""

from __future__ import annotations

import logging
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from specfold_amd import _lib
from specfold_amd.kv_cache import PagedKVCache, cache_length, prefix_view

logger = logging.getLogger(__name__)


def build_parent_map(batched_input: torch.Tensor) -> Tuple[List[Optional[int]], List[int]]:
    """Parent of every draft branch (reference: fastdllm_v2_folded.py:55-75).

    parent(i) = the lowest-indexed j != i whose differing-position set (vs. the
    main row) has one element fewer and is a subset of i's; main (0) if none.
    One D2H copy of the token block.
    """
    bi = batched_input.to("cpu", non_blocking=False)
    neq = bi != bi[0:1]
    counts_t = neq.sum(1)
    # extra[i, j] = diff(j) has a position that diff(i) lacks
    extra = (neq.unsqueeze(0) & ~neq.unsqueeze(1)).any(-1)
    counts = counts_t.tolist()
    extra_l = extra.tolist()
    B1 = bi.shape[0]
    parent: List[Optional[int]] = [None] * B1
    for i in range(1, B1):
        parent[i] = next((j for j in range(B1)
                          if j != i and counts[j] == counts[i] - 1 and not extra_l[i][j]), 0)
    return parent, counts


@dataclass
class StepStats:
    counts: List[int] = field(default_factory=list)   # recomputed rows per layer
    bucket: int = 0
    overflow: bool = False


class _Buffers:
    """Device buffers for one (B1, N, bucket, P-capacity) shape; reused across steps."""

    def __init__(self, eng: "FoldedVerifyEngine", B1: int, N: int, bucket: int, P: int):
        dev, bf = eng.device, torch.bfloat16
        BN = B1 * N
        D, H, Hkv, hd, L = eng.D, eng.H, eng.Hkv, eng.hd, eng.L
        i32 = dict(dtype=torch.int32, device=dev)
        self.key = (B1, N, bucket)
        self.P_cap = P
        self.rec = torch.zeros(BN, dtype=torch.int8, device=dev)
        self.f = torch.zeros(BN, **i32)
        self.src = torch.zeros(BN, **i32)
        self.rows = torch.zeros(bucket, **i32)
        self.count_slab = torch.zeros(L, **i32)
        self.seg = torch.zeros(BN, **i32)
        self.segcnt_slab = torch.zeros(L * B1, **i32)
        self.rstd = torch.zeros(BN, dtype=torch.float32, device=dev)
        self.xn = torch.zeros(BN, D, dtype=bf, device=dev)
        self.q_buf = torch.zeros(BN + 1, H * hd, dtype=bf, device=dev)
        self.kv_buf = torch.zeros(BN + 1, 2 * Hkv * hd, dtype=bf, device=dev)
        self.o32 = torch.zeros(BN, H * hd, dtype=torch.float32, device=dev)
        self.o_bf = torch.zeros(BN, H * hd, dtype=bf, device=dev)
        self.m_tab = torch.zeros(BN, H, dtype=torch.float32, device=dev)
        self.z_tab = torch.zeros(BN, H, dtype=torch.float32, device=dev)
        self.hp = torch.zeros(BN + 1, D, dtype=bf, device=dev)      # row BN stays zero (trash)
        self.ffn = torch.zeros(BN + 1, D, dtype=bf, device=dev)
        self.n_flat = torch.arange(N, device=dev, dtype=torch.int64).repeat(B1)
        nq = (H + 2 * Hkv) * hd
        self.ws_qkv = torch.empty(max(_lib.qkv_workspace_bytes(bucket, D, nq), 256),
                                  dtype=torch.uint8, device=dev)
        self.ws_attn = torch.empty(max(_lib.attn_workspace_bytes(bucket, H, P), 256),
                                   dtype=torch.uint8, device=dev)


class FoldedVerifyEngine:
    """Runs the folded verify step of a Qwen2-layout model through the HIP kernels."""

    def __init__(self, model, gate_mode: int = _lib.SF_GATE_MODEL_DTYPE,
                 rms_eps: Optional[float] = None, has_qkv_bias: Optional[bool] = None):
        _lib.load()  # fail loudly, before any work, if the HIP library is not built
        self.model = model
        base = model.model
        cfg = model.config
        self.cfg = cfg
        self.layers = base.layers
        self.L = len(self.layers)
        self.H = cfg.num_attention_heads
        self.Hkv = cfg.num_key_value_heads
        attn0 = self.layers[0].self_attn
        self.hd = attn0.head_dim
        self.scaling = float(attn0.scaling)
        self.D = base.embed_tokens.weight.shape[1]
        self.device = base.embed_tokens.weight.device
        if base.embed_tokens.weight.dtype != torch.bfloat16:
            raise TypeError("the HIP verify step runs bf16 models")
        if self.device.type != "cuda":
            raise ValueError("the HIP verify step needs the model on a GPU")
        self.eps = float(rms_eps if rms_eps is not None else
                         getattr(cfg, "rms_norm_eps", 1e-6))
        self.gate_mode = gate_mode
        self._packed: List[Tuple[torch.Tensor, Optional[torch.Tensor]]] = []
        for lyr in self.layers:
            a = lyr.self_attn
            w = torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight], 0).contiguous()
            use_bias = has_qkv_bias if has_qkv_bias is not None else a.q_proj.bias is not None
            b = (torch.cat([a.q_proj.bias, a.k_proj.bias, a.v_proj.bias], 0).contiguous()
                 if use_bias and a.q_proj.bias is not None else None)
            self._packed.append((w, b))
        self._bufs: Dict[Tuple[int, int, int], _Buffers] = {}

    # ------------------------------------------------------------------------
    def buffers(self, B1: int, N: int, bucket: int, P: int) -> _Buffers:
        key = (B1, N, bucket)
        buf = self._bufs.get(key)
        if buf is None or buf.P_cap < P:
            cap = max(P, 1024)
            if buf is not None:
                cap = max(cap, 2 * buf.P_cap)
            buf = _Buffers(self, B1, N, bucket, cap)
            self._bufs[key] = buf
        return buf

    def rope_tables(self, hidden: torch.Tensor, P: int, N: int):
        pos = torch.arange(P, P + N, device=self.device).unsqueeze(0)
        cos, sin = self.model.model.rotary_emb(hidden, pos)
        return cos[0].contiguous(), sin[0].contiguous()

    # ------------------------------------------------------------------------
    @torch.no_grad()
    def forward(self, batched_input: torch.Tensor, cache=None, delta: float = 0.1,
                bucket: Optional[int] = None, parent: Optional[List[Optional[int]]] = None,
                append: bool = False, compute_logits: bool = True,
                q_scale: Optional[torch.Tensor] = None,
                trace: Optional[list] = None,
                teacher: Optional[Dict[int, torch.Tensor]] = None,
                stats: Optional[StepStats] = None) -> Optional[torch.Tensor]:
        """Verify step -> logits [B1, N, V] (unshifted), or None if not compute_logits.

        batched_input  [B1, N] int64 on the model's device; row 0 = main branch.
        cache          PagedKVCache, a reference-style per-layer (k, v) cache, or None.
        append         also write the block's K/V into ``cache`` at its end and
                       advance it (block-commit forward; requires B1 == 1).
        trace          list to receive one dict of per-layer device tensors (clones).
        teacher        {layer: hidden [B1, N, D]} replacing that layer's input.
        """
        B1, N = batched_input.shape
        BN = B1 * N
        if bucket is None:
            bucket = BN
        bucket = max(1, min(int(bucket), BN))
        if append and (B1 != 1 or not isinstance(cache, PagedKVCache)):
            raise ValueError("append needs B1 == 1 and a PagedKVCache")
        if parent is None:
            parent = build_parent_map(batched_input)[0] if B1 > 1 else [None]
        par_host = [0] + [int(p) for p in parent[1:]]
        par = torch.tensor(par_host, dtype=torch.int32).to(self.device, non_blocking=True)

        P = cache_length(cache)
        buf = self.buffers(B1, N, bucket, P)
        base = self.model.model
        hidden = base.embed_tokens(batched_input).reshape(BN, self.D)
        cos, sin = self.rope_tables(hidden, P, N)
        H, Hkv, hd, D = self.H, self.Hkv, self.hd, self.D
        src_flat = None

        for li, lyr in enumerate(self.layers):
            if teacher is not None and li in teacher:
                hidden = teacher[li].reshape(BN, D).to(torch.bfloat16).contiguous()
            hidden = hidden.contiguous()
            count = buf.count_slab[li:li + 1]
            segcnt = buf.segcnt_slab[li * B1:(li + 1) * B1]
            _lib.fold_gate(hidden, par, lyr.input_layernorm.weight, B1, N, bucket, delta, self.eps,
                           self.gate_mode, buf.rec, buf.f, buf.src, buf.rows, count, buf.seg,
                           segcnt, buf.rstd, buf.xn)
            w_qkv, b_qkv = self._packed[li]
            _lib.qkv_rope(buf.xn, buf.rows, count, bucket, BN, w_qkv, b_qkv, cos, sin, q_scale,
                          N, D, H, Hkv, hd, buf.q_buf, buf.kv_buf, buf.ws_qkv)
            if append:
                cache.append_rows(li, buf.kv_buf, 0, N)
            pv = prefix_view(cache, li)
            Pl = pv.length if pv is not None else 0
            _lib.attn_prefix_block(
                buf.q_buf, buf.kv_buf, pv.k if pv else None, pv.v if pv else None,
                pv.page_table if pv else None, Pl, pv.page_size if pv else 1,
                pv.page_stride if pv else 0, pv.head_stride if pv else 0,
                buf.src, buf.rows, count, bucket, B1, N, H, Hkv, hd, self.scaling,
                buf.o32, buf.o_bf, buf.m_tab, buf.z_tab, buf.ws_attn)
            _lib.chain_correct(buf.q_buf, buf.kv_buf, buf.src, par, buf.rec, buf.seg, segcnt,
                               B1, N, H, Hkv, hd, self.scaling, buf.o32, buf.o_bf, buf.m_tab,
                               buf.z_tab)

            # o_proj + residual for every row (fastdllm_v2_folded.py:207-209)
            attn_out = torch.mm(buf.o_bf, lyr.self_attn.o_proj.weight.t())
            torch.add(hidden, attn_out, out=buf.hp[:BN])
            # FFN on the compacted rows; slots past count hold BN -> the zero row
            rows_l = buf.rows.long()
            z = lyr.post_attention_layernorm(buf.hp.index_select(0, rows_l))
            mlp = lyr.mlp
            act = F.silu(mlp.gate_proj(z)) * mlp.up_proj(z)
            buf.ffn.index_copy_(0, rows_l, mlp.down_proj(act))
            # folded rows reuse the FFN output of their nearest recomputing ancestor
            src_flat = buf.src.long() * N + buf.n_flat
            new_hidden = buf.hp[:BN] + buf.ffn.index_select(0, src_flat)
            if trace is not None:
                trace.append(dict(
                    h_in=hidden.clone(), rec=buf.rec.clone(), rows=buf.rows.clone(),
                    count=count.clone(), src=buf.src.clone(), f=buf.f.clone(),
                    seg=buf.seg.clone(), segcnt=segcnt.clone(), rstd=buf.rstd.clone(),
                    xn=buf.xn.clone(), q=buf.q_buf.clone(), kv=buf.kv_buf.clone(),
                    o32=buf.o32.clone(), o_bf=buf.o_bf.clone(), m=buf.m_tab.clone(),
                    z=buf.z_tab.clone(), hp=buf.hp[:BN].clone(), ffn=buf.ffn.clone(),
                    h_out=new_hidden.clone()))
            hidden = new_hidden

        if append:
            cache.advance(N)
        counts = buf.count_slab.tolist()       # the one post-loop host sync
        overflow = max(counts) > bucket
        if stats is not None:
            stats.counts, stats.bucket, stats.overflow = counts, bucket, overflow
        if overflow:
            if append:
                raise RuntimeError("bucket overflow during a block commit")
            logger.warning("SpecFold bucket overflow (%d > %d); recomputing with bucket=%d",
                           max(counts), bucket, BN)
            return self.forward(batched_input, cache, delta, bucket=BN, parent=parent,
                                compute_logits=compute_logits, q_scale=q_scale, trace=trace,
                                teacher=teacher, stats=stats)
        self.last_hidden = hidden
        self._last = dict(B1=B1, N=N, bucket=bucket, cache=cache, par=par, cos=cos, sin=sin,
                          q_scale=q_scale, hidden=hidden, delta=delta)
        if not compute_logits:
            return None
        final = base.norm(hidden.view(B1, N, D))
        return self.model.lm_head(final)

    # ------------------------------------------------------------------------
    def profile_launchers(self, li: int = -1):
        """No-argument callables that re-launch each HIP entry point of layer
        ``li`` on the buffers resident from the last forward (for timing).
        The gate runs on the last layer's output hidden states, so call it
        last: it rewrites rows/count/src for the other launchers."""
        st = self._last
        B1, N, bucket, cache = st["B1"], st["N"], st["bucket"], st["cache"]
        BN = B1 * N
        buf = self._bufs[(B1, N, bucket)]
        li = li % self.L
        lyr = self.layers[li]
        H, Hkv, hd, D = self.H, self.Hkv, self.hd, self.D
        count = buf.count_slab[li:li + 1]
        segcnt = buf.segcnt_slab[li * B1:(li + 1) * B1]
        pv = prefix_view(cache, li)
        w_qkv, b_qkv = self._packed[li]
        hidden = st["hidden"]

        def gate():
            _lib.fold_gate(hidden, st["par"], lyr.input_layernorm.weight, B1, N, bucket, st["delta"],
                           self.eps, self.gate_mode, buf.rec, buf.f, buf.src, buf.rows, count,
                           buf.seg, segcnt, buf.rstd, buf.xn)

        def qkv():
            _lib.qkv_rope(buf.xn, buf.rows, count, bucket, BN, w_qkv, b_qkv, st["cos"], st["sin"],
                          st["q_scale"], N, D, H, Hkv, hd, buf.q_buf, buf.kv_buf, buf.ws_qkv)

        def attn():
            _lib.attn_prefix_block(
                buf.q_buf, buf.kv_buf, pv.k if pv else None, pv.v if pv else None,
                pv.page_table if pv else None, pv.length if pv else 0,
                pv.page_size if pv else 1, pv.page_stride if pv else 0,
                pv.head_stride if pv else 0, buf.src, buf.rows, count, bucket, B1, N, H, Hkv, hd,
                self.scaling, buf.o32, buf.o_bf, buf.m_tab, buf.z_tab, buf.ws_attn)

        def chain():
            _lib.chain_correct(buf.q_buf, buf.kv_buf, buf.src, st["par"], buf.rec, buf.seg, segcnt,
                               B1, N, H, Hkv, hd, self.scaling, buf.o32, buf.o_bf, buf.m_tab,
                               buf.z_tab)

        out = dict(qkv=qkv, attn=attn, chain=chain, gate=gate)
        if isinstance(cache, PagedKVCache) and cache.length + N <= cache.capacity:
            def append():
                # writes past the logical end of the cache: never read, length unchanged
                cache.append_rows(li, buf.kv_buf, 0, N, start_pos=cache.length)
            out["append"] = append
        return out, dict(count=count, buf=buf, prefix=pv.length if pv else 0)
