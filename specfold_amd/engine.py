"""Folded multi-branch verify step on MI355X.

``FoldedVerifyEngine.forward`` runs SpecFold's verify step for B1 = 1 + B
branches of one N-token block over a prefix KV cache, all layers, and returns
the (unshifted) logits.  Per layer (reference: specfold/generate/
fastdllm_v2_folded.py:296-361 for the launch sequence, :117-220 for the math):

  sf_fold_gate(_residual)  the previous layer's residual update + gate +
                     compaction + src + input RMSNorm          (HIP)
  sf_qkv_rope        QKV MFMA GEMM + bias + RoPE + scatter     (HIP)
  sf_kv_append       optional in-place append (block commit)   (HIP)
  sf_attn_rows       attention of every row with (m, Z): recomputed rows over
                     [prefix ; own block], folded rows from their source row's
                     query over their own branch's keys (the chain correction's
                     result)                                   (HIP)
  sf_o_proj_post_norm  o_proj of every row (M = B1*N, all-rows MFMA GEMM), hp =
                     x + bf16(O Wo^T), post-attention RMSNorm of the
                     recomputed rows                           (HIP)
  sf_ffn_gate_up      gate/up GEMM + SiLU*mul on compacted rows  (HIP)
  sf_ffn_down_scatter down GEMM, scattered to the per-row FFN table (HIP)
and after the last layer the residual update + final RMSNorm (HIP) and the
head (HIP, sf_head_logits: one pass over the packed head weights for every row,
with Fast-dLLM's logit shift done by its stores when asked for).  sf_chain_correct
(the reference's incremental form of the folded rows' attention) stays in the C
ABI; the engine forms it with sf_attn_rows.

Nothing here syncs with the host: the branch parent map is computed from the
tokens on the device (sf_parent_map; the reference copies the tokens to the host
for it), ``count`` stays on the device and every kernel reads it, and the
per-layer counts are copied to the host only when read (fold statistics), or
once per step when a bucket below B1*N could overflow.
"""

from __future__ import annotations

import contextlib
import gc
import logging
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

from specfold_amd import _lib
from specfold_amd.kv_cache import ContiguousMirror, PagedKVCache, cache_length, prefix_view


@contextlib.contextmanager
def _capturing(graph: "torch.cuda.CUDAGraph"):
    """torch.cuda.graph(graph) with the garbage collector held off.

    A collection inside the capture may free an unreachable CUDAGraph (an engine
    dropped in a reference cycle still holds its graphs), and destroying a graph
    while a stream captures is refused by HIP and aborts the process.  The cycles
    are collected first, outside the capture."""
    gc.collect()
    was = gc.isenabled()
    gc.disable()
    try:
        with torch.cuda.graph(graph):
            yield
    finally:
        if was:
            gc.enable()


logger = logging.getLogger(__name__)


def _device_cache(cache) -> bool:
    """A cache whose buffers stay put and whose length lives in device memory."""
    return isinstance(cache, (PagedKVCache, ContiguousMirror))


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
    """Recomputed rows per layer of one verify step.  ``count_dev`` stays on the
    device; ``counts`` copies it to the host on first use."""
    count_dev: Optional[torch.Tensor] = None
    bucket: int = 0
    overflow: bool = False
    _counts: Optional[List[int]] = None

    @property
    def counts(self) -> List[int]:
        if self._counts is None:
            self._counts = [] if self.count_dev is None else self.count_dev.tolist()
        return self._counts


def decoder_parts(model):
    """(decoder stack, output head) of a causal-LM module tree: ``model.model`` /
    ``model.lm_head`` (Qwen2, Llama), or ``model.encoder`` / ``model.diffusion_head``
    (Nemotron-Labs-Diffusion, specfold/generate/nld_folded.py:105-108, 237)."""
    base = getattr(model, "model", None)
    if base is None or not hasattr(base, "layers"):
        base = model.encoder
    head = getattr(model, "lm_head", None)
    if head is None:
        head = model.diffusion_head
    return base, head


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
        self.par = torch.zeros(B1, **i32)          # branch parents (sf_parent_map)
        self.seg = torch.zeros(BN, **i32)
        self.slot = torch.zeros(BN, **i32)
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
        self.zn = torch.zeros(bucket, D, dtype=bf, device=dev)
        self.act = torch.zeros(bucket, eng.I, dtype=bf, device=dev)
        self.hid = torch.zeros(2, BN, D, dtype=bf, device=dev)       # layer outputs, ping-pong
        self.final = torch.zeros(BN, D, dtype=bf, device=dev)
        self.pos0 = torch.zeros(1, **i32)   # first block position (caches without length_dev)
        self.q_scale = torch.ones(N, dtype=torch.float32, device=dev)  # per-position q scale
        self.all_rows = torch.arange(BN, **i32)
        self.all_count = torch.full((1,), BN, **i32)
        nq = (H + 2 * Hkv) * hd
        # GEMM workspaces: fp32 partial slots of the stream-K split (gate/up and down
        # run one after the other on one stream and share theirs)
        self.ws_gemm = torch.empty(max(_lib.gemm_workspace_bytes(bucket, D, eng.I),
                                       _lib.gate_up_workspace_bytes(bucket, D, eng.I), 256),
                                   dtype=torch.uint8, device=dev)
        self.ws_qkv = torch.empty(max(_lib.qkv_workspace_bytes(bucket, D, nq), 256),
                                  dtype=torch.uint8, device=dev)
        self.ws_attn = torch.empty(max(_lib.attn_workspace_bytes(bucket, H, P), 256),
                                   dtype=torch.uint8, device=dev)
        # o_proj over every row: fp32 sums of its K ranges
        self.ws_oproj = torch.empty(max(_lib.o_proj_workspace_bytes(BN, D, H * hd), 256),
                                    dtype=torch.uint8, device=dev)


class _Batch:
    """Several sequences' branch trees stacked into one verify step: sequence s
    owns branches offsets[s] .. offsets[s] + sizes[s] - 1 (its main branch first)
    and its own prefix cache.  Static device tensors, so a captured step replays
    with new values: the per-branch first positions are re-read from the caches'
    device-side lengths inside the step (refresh_positions), the per-row q scales
    are copied into q_scale_rows before each run."""

    def __init__(self, eng: "FoldedVerifyEngine", sizes: List[int], caches: list, N: int,
                 q_scaled: bool):
        dev = eng.device
        self.sizes = list(sizes)
        self.offsets = [sum(self.sizes[:i]) for i in range(len(self.sizes))]
        self.caches = list(caches)
        B1 = sum(self.sizes)
        i32 = dict(dtype=torch.int32, device=dev)
        self.pos0_branch = torch.zeros(B1, **i32)
        self._zeros = torch.zeros(max(self.sizes), **i32)
        self.q_scale_rows = torch.ones(B1 * N, dtype=torch.float32, device=dev) \
            if q_scaled else None
        self.bounds = torch.tensor([o * N for o in self.offsets] + [B1 * N], **i32)
        self.idx = torch.arange(B1 * N, **i32)
        self.masked = torch.zeros(B1 * N, **i32)

    def set_q_scales(self, q_scales: Optional[list], N: int) -> None:
        if self.q_scale_rows is None:
            return
        for o, b, q in zip(self.offsets, self.sizes, q_scales):
            dst = self.q_scale_rows[o * N:(o + b) * N].view(b, N)
            if q is None:
                dst.fill_(1.0)
            else:
                dst.copy_(q.reshape(1, N).to(dtype=torch.float32).expand(b, N))

    def refresh_positions(self) -> None:
        """pos0_branch[b] = its sequence's prefix length, read on the device."""
        torch.cat([c.length_dev.expand(b) if c is not None else self._zeros[:b]
                   for c, b in zip(self.caches, self.sizes)], out=self.pos0_branch)

    def split_rows(self, rows: torch.Tensor, count: torch.Tensor, bucket: int, N: int):
        """Per-sequence runs of the ascending compacted rows: (rows_s [S, bucket],
        count_s [S]) on the device, without a host sync (a binary search of the
        sequences' first rows; no reduction kernel)."""
        idx = self.idx[:bucket]
        masked = self.masked[:bucket]
        # rows past the count -> B1*N, so the first `count` rows stay a sorted prefix
        torch.where(idx < count, rows[:bucket], self.bounds[-1], out=masked)
        below = torch.searchsorted(masked, self.bounds, out_int32=True)
        gather = (below[:-1].unsqueeze(1) + idx.unsqueeze(0)).clamp_(max=bucket - 1)
        rows_s = rows[gather.long()].contiguous()
        return rows_s, (below[1:] - below[:-1]).contiguous()


class FoldedVerifyEngine:
    """Runs the folded verify step of a Qwen2-layout model through the HIP kernels."""

    def __init__(self, model, gate_mode: int = _lib.SF_GATE_MODEL_DTYPE,
                 rms_eps: Optional[float] = None, has_qkv_bias: Optional[bool] = None):
        _lib.load()  # fail loudly, before any work, if the HIP library is not built
        model.requires_grad_(False)
        self.model = model
        base, head = decoder_parts(model)
        self.base, self.head = base, head
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
        self.I = self.layers[0].mlp.gate_proj.weight.shape[0]
        self.V = head.weight.shape[0]
        self.device = base.embed_tokens.weight.device
        if base.embed_tokens.weight.dtype != torch.bfloat16:
            raise TypeError("the HIP verify step runs bf16 models")
        self._check_device(self.device)
        self.eps = float(rms_eps if rms_eps is not None else
                         getattr(cfg, "rms_norm_eps", 1e-6))
        self.gate_mode = gate_mode
        # the gate's compaction runs in the QKV GEMM's prologue (one launch fewer per
        # layer); False: the gate's own compaction kernel, then sf_qkv_rope
        self.gated_qkv = True
        # Weights of the HIP GEMMs, packed once into the fragment-major layout the
        # weight-streaming kernels read (the reference packs W_qkv / W_gu once too,
        # fastdllm_v2_folded.py:77-87).  The module tree keeps its own tensors.
        self._packed: List[Tuple[torch.Tensor, Optional[torch.Tensor]]] = []
        self._packed_mlp: List[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = []
        self._packed_o: List[torch.Tensor] = []
        for lyr in self.layers:
            a = lyr.self_attn
            w = torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight], 0).contiguous()
            use_bias = has_qkv_bias if has_qkv_bias is not None else a.q_proj.bias is not None
            b = (torch.cat([a.q_proj.bias, a.k_proj.bias, a.v_proj.bias], 0).contiguous()
                 if use_bias and a.q_proj.bias is not None else None)
            self._packed.append((_lib.pack_weight(w), b))
            del w
            m = lyr.mlp
            self._packed_mlp.append((_lib.pack_weight(m.gate_proj.weight.contiguous()),
                                     _lib.pack_weight(m.up_proj.weight.contiguous()),
                                     _lib.pack_weight(m.down_proj.weight.contiguous())))
            self._packed_o.append(_lib.pack_weight(a.o_proj.weight.contiguous()))
        # the head, packed once; zero rows pad it to whole 128-column tiles of the
        # head kernel (their logit columns are never returned)
        self.V_pad = -(-self.V // 128) * 128
        w = head.weight.contiguous()
        if self.V_pad != self.V:
            w = torch.cat([w, w.new_zeros(self.V_pad - self.V, self.D)])
        self._packed_head = _lib.pack_weight(w)
        del w
        self.head_kernel = "hip"
        self._bufs: Dict[Tuple[int, int, int], _Buffers] = {}
        # HIP graphs of the layer loop, keyed by shape / prefix / delta / cache
        # (one per branch count the decode loop visits, B1 = 1..8, per sequence's
        # cache: several sequences decoded in turn each keep their own set)
        self.use_graphs = True
        self.max_graphs = 48
        self._graphs: Dict[tuple, tuple] = {}
        self._rope: Optional[Tuple[torch.Tensor, torch.Tensor]] = None
        self._mirror: Optional[ContiguousMirror] = None   # reference-style caches

    def lm_head(self, x: torch.Tensor, out: Optional[torch.Tensor] = None,
                shift_n: int = 0, rows: Optional[Tuple[int, int, int]] = None) -> torch.Tensor:
        """logits [M, V] = x . Wlm^T for every row of x [M, D] (sf_head_logits on the
        packed head weights; ``out``: an [M, V_pad] bf16 buffer, else a fresh one).
        shift_n = N: x holds blocks of N rows and the result is Fast-dLLM's shifted
        logits (row (b, n) takes row (b, n - 1)'s logits, row (b, 0) its own;
        fastdllm_v2_generation.py:121-126), written so by the head's stores.  A view of
        V columns (rows of V_pad elements, contiguous when V % 128 == 0).
        ``rows`` = (N, lo, n): only positions [lo, lo + n) of every N-row block are
        computed (the rest of ``out`` is not written): the rows a decode step reads."""
        M = x.shape[0]
        if out is None:
            out = torch.empty(M, self.V_pad, dtype=torch.bfloat16, device=self.device)
        if rows is None:
            _lib.head_logits(x, M, self._packed_head, self.D, self.V_pad, out, shift_n=shift_n)
        else:
            blk, lo, n = rows
            _lib.head_logits_rows(x, M, self._packed_head, self.D, self.V_pad, out, blk,
                                  shift_n > 0, lo, n)
        return out[:, :self.V]

    @staticmethod
    def _check_device(device: torch.device) -> None:
        """The kernels run on the GPU only; there is no CPU path."""
        if device.type != "cuda":
            raise ValueError("the HIP verify step needs the model on a GPU")

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

    def rope_tables(self, rows_needed: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """cos/sin [T, hd] over absolute positions 0..T-1 from the model's own
        rotary embedding (each entry is elementwise in its position, so a row of
        the full table equals the table of the block alone).  The kernels index it
        with the device-side prefix length.  Growing it moves the tables, so the
        captured graphs that point at them are dropped."""
        if self._rope is None or self._rope[0].shape[0] < rows_needed:
            T = max(int(rows_needed), int(getattr(self.cfg, "max_position_embeddings", 0) or 0),
                    4096)
            base = self.base
            pos = torch.arange(T, device=self.device).unsqueeze(0)
            cos, sin = base.rotary_emb(base.embed_tokens.weight, pos)
            self._rope = (cos[0].contiguous(), sin[0].contiguous())
            self._graphs.clear()
        return self._rope

    # ------------------------------------------------------------------------
    @torch.no_grad()
    def forward(self, batched_input: torch.Tensor, cache=None, delta: float = 0.1,
                bucket: Optional[int] = None, append: bool = False, compute_logits: bool = True,
                q_scale: Optional[torch.Tensor] = None,
                trace: Optional[list] = None,
                teacher: Optional[Dict[int, torch.Tensor]] = None,
                stats: Optional[StepStats] = None,
                causal: bool = False, shift: bool = False,
                head_rows: Optional[Tuple[int, int]] = None) -> Optional[torch.Tensor]:
        """Verify step -> logits [B1, N, V] (unshifted, or with ``shift`` Fast-dLLM's
        shifted logits, fastdllm_v2_generation.py:121-126, from the head's stores), or
        None if not compute_logits.  ``head_rows`` = (lo, n): only positions
        [lo, lo + n) of every branch get logits (the rest of the returned tensor is
        not written): the rows a decode step reads, so the head computes a fraction
        of its rows.

        batched_input  [B1, N] int64 on the model's device; row 0 = main branch.
        cache          PagedKVCache, a reference-style per-layer (k, v) cache, or None.
        append         also write the block's K/V into ``cache`` at its end and
                       advance it (block-commit forward; requires B1 == 1).
        q_scale        optional [N] fp32: roped q of block position n is multiplied by
                       bf16(q_scale[n]) (the llama-4 attention scale of NLD models).
        causal         block position n attends to block positions <= n only (an AR
                       forward: NLD's prefill / block commit); every row recomputed.
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
        batched_input = batched_input.to(self.device).contiguous()
        P = cache_length(cache)
        if cache is not None and not _device_cache(cache):
            # a reference-style cache is read through the engine's mirror: fixed
            # buffers and a device length, so the captured step outlives its commits
            cache = self._mirror_of(cache, P) if P > 0 else None
        P_alloc = cache.capacity if _device_cache(cache) else P
        buf = self.buffers(B1, N, bucket, P_alloc)
        if causal and self.gate_mode != _lib.SF_GATE_ALL:
            raise ValueError("a causal forward recomputes every row (gate mode SF_GATE_ALL)")
        self.rope_tables(P + N)
        if not _device_cache(cache):
            buf.pos0.fill_(P)
        qs = None
        if q_scale is not None:
            buf.q_scale.copy_(q_scale.reshape(-1).to(device=self.device, dtype=torch.float32))
            qs = buf.q_scale
        graphable = self.use_graphs and trace is None and teacher is None and not append
        if graphable:
            hidden = self._replay(buf, batched_input, cache, P, delta, bucket,
                                  qs is not None, causal)
        else:
            hidden = self._run_layers(buf, batched_input, cache, delta, bucket,
                                      append=append, q_scale=qs, trace=trace,
                                      teacher=teacher, causal=causal)

        if append:
            cache.advance(N)
        overflow = False
        if bucket < BN:
            # a bucket below B1*N can overflow: one host sync to check
            overflow = int(buf.count_slab.max()) > bucket
        if stats is not None:
            stats.count_dev, stats.bucket, stats.overflow = buf.count_slab.clone(), bucket, overflow
            stats._counts = None
        if overflow:
            if append:
                raise RuntimeError("bucket overflow during a block commit")
            logger.warning("SpecFold bucket overflow (> %d); recomputing with bucket=%d",
                           bucket, BN)
            return self.forward(batched_input, cache, delta, bucket=BN,
                                compute_logits=compute_logits, q_scale=q_scale, trace=trace,
                                teacher=teacher, stats=stats, causal=causal, shift=shift,
                                head_rows=head_rows)
        self.last_hidden = hidden
        self._last = dict(B1=B1, N=N, bucket=bucket, cache=cache, par=buf.par, q_scale=qs,
                          hidden=hidden, delta=delta, shift=shift)
        if not compute_logits:
            return None
        rows = None if head_rows is None else (N, int(head_rows[0]), int(head_rows[1]))
        return self.lm_head(buf.final, shift_n=N if shift else 0, rows=rows).view(B1, N, self.V)

    @torch.no_grad()
    def forward_batched(self, blocks: List[torch.Tensor], caches: list, delta: float = 0.1,
                        bucket: Optional[int] = None,
                        q_scales: Optional[List[Optional[torch.Tensor]]] = None,
                        stats: Optional[StepStats] = None, compute_logits: bool = True,
                        pad_to: Optional[int] = None,
                        trace: Optional[list] = None,
                        shift: bool = False) -> Optional[List[torch.Tensor]]:
        """One verify step over several independent sequences -> per-sequence logits
        [B1_s, N, V] (unshifted).

        blocks[s]  [B1_s, N] int64, sequence s's branches (row 0 = its main branch);
        caches[s]  its PagedKVCache (or None: no prefix); q_scales[s] optional [N].
        pad_to     pad every sequence to this many branches with copies of its main
                   branch, so the step's shape, and its captured HIP graph, depend
                   on the number of sequences only.  A copy is no branch's parent
                   and leaves every other row's result unchanged; it gates as
                   folded (no GEMM rows, no attention) wherever delta > 0.  At
                   delta = 0 a copy's folded-row attention output, which may
                   round one bf16 step away from its main branch's, can make it
                   recompute at later layers: extra rows, same results.
        The sequences' branches are stacked into one step of sum(B1_s) branches:
        the gate, compaction and GEMMs run once over all of them
        (the main branch of every sequence is a root: SF_GATE_ROOTS_BY_PARENT), the
        QKV epilogue ropes each branch at its sequence's positions, and attention
        runs per sequence over its own prefix.  Each sequence's result is that of
        ``forward`` on it alone.  No counterpart in the reference, whose verify step
        takes one sequence.  ``stats`` counts every recomputed row, padded ones
        included.  ``trace``: as in ``forward``, one dict per layer of the stacked
        step's buffers (runs eagerly).  ``shift``: Fast-dLLM's shifted logits, as in
        ``forward``."""
        if not blocks or len(blocks) != len(caches):
            raise ValueError("forward_batched needs one cache (or None) per token block")
        if q_scales is not None and len(q_scales) != len(blocks):
            raise ValueError("forward_batched needs one q scale (or None) per token block")
        N = blocks[0].shape[-1]
        for b in blocks:
            if b.dim() != 2 or b.shape[1] != N:
                raise ValueError("every token block must be [B1_s, N] with the same N")
        for c in caches:
            if c is not None and not isinstance(c, PagedKVCache):
                raise TypeError("forward_batched takes PagedKVCache prefixes (or None)")
        real = [int(b.shape[0]) for b in blocks]
        orig_blocks = blocks
        if pad_to is not None:
            if max(real) > pad_to:
                raise ValueError(f"a sequence has {max(real)} branches > pad_to={pad_to}")
            blocks = [b if b.shape[0] == pad_to else
                      torch.cat([b, b[0:1].expand(pad_to - b.shape[0], N)])
                      for b in (x.to(self.device) for x in blocks)]
        sizes = [int(b.shape[0]) for b in blocks]
        B1 = sum(sizes)
        BN = B1 * N
        if B1 > 64 or BN > 1024:
            raise ValueError(f"a batched step holds at most 64 branches and 1024 rows: "
                             f"{len(sizes)} sequences of {sizes} branches x {N} = {BN} rows")
        tokens = torch.cat([b.to(self.device) for b in blocks]).contiguous()
        bucket = BN if bucket is None else max(1, min(int(bucket), BN))
        P_alloc = max([c.capacity for c in caches if c is not None], default=0)
        buf = self.buffers(B1, N, bucket, P_alloc)
        self.rope_tables(max(cache_length(c) for c in caches) + N)
        q_scaled = q_scales is not None and any(q is not None for q in q_scales)
        if self.use_graphs and trace is None:
            hidden = self._replay_batched(buf, tokens, sizes, caches, N, delta, bucket,
                                          q_scales if q_scaled else None)
        else:
            batch = _Batch(self, sizes, caches, N, q_scaled)
            batch.set_q_scales(q_scales, N)
            hidden = self._run_layers(buf, tokens, None, delta, bucket, batch=batch,
                                      trace=trace)
        overflow = bucket < BN and int(buf.count_slab.max()) > bucket
        if stats is not None:
            stats.count_dev, stats.bucket, stats.overflow = buf.count_slab.clone(), bucket, overflow
            stats._counts = None
        if overflow:
            logger.warning("SpecFold bucket overflow (> %d); recomputing with bucket=%d",
                           bucket, BN)
            if trace is not None:
                trace.clear()
            return self.forward_batched(orig_blocks, caches, delta, bucket=BN, q_scales=q_scales,
                                        stats=stats, compute_logits=compute_logits,
                                        pad_to=pad_to, trace=trace, shift=shift)
        self.last_hidden = hidden
        if not compute_logits:
            return None
        logits = self.lm_head(buf.final, shift_n=N if shift else 0).view(B1, N, self.V)
        return [x[:r] for x, r in zip(logits.split(sizes, 0), real)]

    def _replay_batched(self, buf: _Buffers, tokens: torch.Tensor, sizes: List[int],
                        caches: list, N: int, delta: float, bucket: int,
                        q_scales: Optional[list]):
        """forward_batched's layers through a captured HIP graph, one per (branch
        counts, caches, delta, bucket): the tokens and q scales go through static
        buffers, the prefix lengths are read on the device inside the graph."""
        key = ("batched", buf.key, id(buf), tuple(sizes),
               tuple(self._cache_key(c) for c in caches), float(delta), bucket,
               self.gate_mode, q_scales is not None)
        entry = self._graphs.get(key)
        if entry is None:
            batch = _Batch(self, sizes, caches, N, q_scales is not None)
            batch.set_q_scales(q_scales, N)
            static_tok = tokens.clone()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):      # warm-up launch outside the capture
                self._run_layers(buf, static_tok, None, delta, bucket, batch=batch)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with _capturing(graph):
                out = self._run_layers(buf, static_tok, None, delta, bucket, batch=batch)
            entry = (graph, static_tok, out, batch)
            while len(self._graphs) >= self.max_graphs:
                self._graphs.pop(next(iter(self._graphs)))
            self._graphs[key] = entry
        graph, static_tok, out, batch = entry
        static_tok.copy_(tokens)
        batch.set_q_scales(q_scales, N)
        graph.replay()
        return out

    # ------------------------------------------------------------------------
    def _run_layers(self, buf: _Buffers, tokens: torch.Tensor, cache,
                    delta: float, bucket: int, append: bool = False,
                    q_scale: Optional[torch.Tensor] = None, trace: Optional[list] = None,
                    teacher: Optional[Dict[int, torch.Tensor]] = None,
                    causal: bool = False, batch: Optional["_Batch"] = None) -> torch.Tensor:
        """Embedding and every layer: device launches only (no host sync), so the
        sequence can be captured in a HIP graph.  RoPE rows and a paged cache's
        length come from the cache's device-side length (buf.pos0 for other
        caches), so a captured sequence stays valid as the cache grows.  Returns
        the last hidden state.  ``batch``: the branch trees of several sequences
        stacked in ``tokens`` (forward_batched)."""
        B1, N = tokens.shape
        BN = B1 * N
        H, Hkv, hd, D = self.H, self.Hkv, self.hd, self.D
        base = self.base
        par = buf.par
        gate_mode = self.gate_mode
        if self.gated_qkv:
            # the compaction runs in the QKV GEMM's prologue (sf_qkv_rope_gated)
            gate_mode |= _lib.SF_GATE_DEFER_COMPACT
        if batch is None:
            _lib.parent_map(tokens, par)          # on the device: no host round trip
        else:
            for o, b in zip(batch.offsets, batch.sizes):
                _lib.parent_map(tokens[o:o + b], par[o:o + b])
                if o:
                    par[o:o + b] += o
            gate_mode |= _lib.SF_GATE_ROOTS_BY_PARENT
            batch.refresh_positions()
        hidden = base.embed_tokens(tokens).reshape(BN, D)
        cos, sin = self._rope
        pos0 = cache.length_dev if _device_cache(cache) else buf.pos0
        for li, lyr in enumerate(self.layers):
            count = buf.count_slab[li:li + 1]
            segcnt = buf.segcnt_slab[li * B1:(li + 1) * B1]
            ln_w = lyr.input_layernorm.weight
            if teacher is not None and li in teacher:
                hidden = teacher[li].reshape(BN, D).to(torch.bfloat16).contiguous()
            if li == 0 or (teacher is not None and li in teacher):
                hidden = hidden.contiguous()
                _lib.fold_gate(hidden, par, ln_w, B1, N, bucket, delta, self.eps, gate_mode,
                               buf.rec, buf.f, buf.src, buf.rows, count, buf.seg, segcnt,
                               buf.rstd, buf.xn, slot=buf.slot)
            else:
                # the previous layer's folded residual update (fastdllm_v2_folded.py:218)
                # fused into this layer's gate: x = bf16(hp + ffn[src*N + n])
                hidden = buf.hid[li % 2]
                _lib.fold_gate_residual(buf.hp, buf.ffn, buf.src, par, ln_w, B1, N, D, bucket,
                                        delta, self.eps, gate_mode, hidden, buf.rec, buf.f,
                                        buf.src, buf.rows, count, buf.seg, segcnt, buf.slot,
                                        buf.rstd, buf.xn)
            w_qkv, b_qkv = self._packed[li]
            if self.gated_qkv:
                # compaction (rows, count, src, seg, slot) + QKV + bias + RoPE
                _lib.qkv_rope_gated(
                    buf.xn, buf.rec, par, B1, N, bucket, buf.f, buf.src, buf.rows, count, buf.seg,
                    segcnt, buf.slot, w_qkv, b_qkv, cos, sin,
                    q_scale if batch is None else batch.q_scale_rows, D, H, Hkv, hd, buf.q_buf,
                    buf.kv_buf, buf.ws_qkv, pos0=pos0 if batch is None else None,
                    pos0_branch=None if batch is None else batch.pos0_branch)
            elif batch is None:
                _lib.qkv_rope(buf.xn, buf.rows, count, bucket, BN, w_qkv, b_qkv, cos, sin,
                              q_scale, N, D, H, Hkv, hd, buf.q_buf, buf.kv_buf, buf.ws_qkv,
                              pos0=pos0)
            else:
                _lib.qkv_rope_branches(buf.xn, buf.rows, count, bucket, BN, w_qkv, b_qkv, cos,
                                       sin, batch.q_scale_rows, N, D, H, Hkv, hd, buf.q_buf,
                                       buf.kv_buf, buf.ws_qkv, batch.pos0_branch)
            if append:
                cache.append_rows(li, buf.kv_buf, 0, N)
            # attention of every row (fastdllm_v2_folded.py:164-204): the recomputed
            # rows over [prefix ; own block], the folded rows from their source row's
            # query over their own branch's keys (what the chain correction computes)
            if batch is None:
                self._attention(buf, cache, li, count, bucket, B1, N, causal=causal,
                                side=trace is not None)
            else:
                # each sequence's rows over its own prefix: the compacted rows are
                # ascending, so sequence s owns a contiguous run of them
                rows_s, count_s = batch.split_rows(buf.rows, count, bucket, N)
                for si, c in enumerate(batch.caches):
                    self._attention(buf, c, li, count_s[si:si + 1], bucket, B1, N,
                                    rows=rows_s[si], side=trace is not None,
                                    branches=(batch.offsets[si], batch.sizes[si]))

            # o_proj for every row (fastdllm_v2_folded.py:207-209) in one pass over Wo,
            # the residual hp = bf16(x + bf16(O Wo^T)) (two roundings as in the
            # reference) and the post-attention RMSNorm of the recomputed rows (:211-212)
            _lib.o_proj_post_norm(buf.o_bf, hidden, self._packed_o[li], BN, self.H * self.hd, D,
                                  buf.slot, lyr.post_attention_layernorm.weight, self.eps,
                                  buf.hp, buf.zn, buf.ws_oproj)
            # FFN on the compacted rows (:211-217)
            wg, wu, wd = self._packed_mlp[li]
            _lib.ffn_gate_up(buf.zn, count, bucket, wg, wu, D, self.I, buf.act, buf.ws_gemm)
            _lib.ffn_down_scatter(buf.act, count, bucket, buf.rows, wd, self.I, D, buf.ffn,
                                  buf.ws_gemm)
            if trace is not None:
                # folded rows reuse the FFN output of their nearest recomputing ancestor
                # (:218); the fused kernels form this inside the next gate, so the trace
                # computes it separately
                h_out = torch.empty(BN, D, dtype=torch.bfloat16, device=self.device)
                _lib.residual_gather_add(buf.hp, buf.ffn, buf.src, B1, N, D, h_out)
                trace.append(dict(
                    h_in=hidden.clone(), rec=buf.rec.clone(), rows=buf.rows.clone(),
                    count=count.clone(), src=buf.src.clone(), f=buf.f.clone(),
                    seg=buf.seg.clone(), segcnt=segcnt.clone(), rstd=buf.rstd.clone(),
                    xn=buf.xn.clone(), q=buf.q_buf.clone(), kv=buf.kv_buf.clone(),
                    o32=buf.o32.clone(), o_bf=buf.o_bf.clone(), m=buf.m_tab.clone(),
                    z=buf.z_tab.clone(), hp=buf.hp[:BN].clone(), ffn=buf.ffn.clone(),
                    h_out=h_out))
        # the last layer's residual update and the final norm (:218, :222)
        last = buf.hid[self.L % 2]
        _lib.residual_rmsnorm(buf.hp, buf.ffn, buf.src, base.norm.weight, B1, N, D, self.eps,
                              last, buf.final)
        return last

    def _attention(self, buf: _Buffers, cache, li: int, count, bucket: int, B1: int, N: int,
                   causal: bool = False, rows: Optional[torch.Tensor] = None,
                   branches: Optional[Tuple[int, int]] = None, side: bool = False):
        """Every row of the branches (first, count) (default: all): sf_attn_rows; a
        causal forward (every row recomputed) takes sf_attn_prefix_block.  side: also
        write the fp32 output and the softmax state (m, Z) (a traced step); o_proj
        reads only the bf16 output."""
        o32, m_tab, z_tab = (buf.o32, buf.m_tab, buf.z_tab) if side else (None, None, None)
        pv = prefix_view(cache, li)
        if pv is None:
            P_arg, plen = 0, None
        elif pv.length_dev is not None:
            P_arg, plen = pv.capacity, pv.length_dev
        else:
            P_arg, plen = pv.length, None
        view = (pv.k if pv else None, pv.v if pv else None, pv.page_table if pv else None, P_arg,
                pv.page_size if pv else 1, pv.page_stride if pv else 0,
                pv.head_stride if pv else 0)
        rows = buf.rows if rows is None else rows
        if causal:
            _lib.attn_prefix_block(buf.q_buf, buf.kv_buf, *view, buf.src, rows, count, bucket, B1,
                                   N, self.H, self.Hkv, self.hd, self.scaling, o32, buf.o_bf,
                                   m_tab, z_tab, buf.ws_attn, prefix_len=plen,
                                   block_causal=True)
        else:
            b0, nb = branches if branches is not None else (0, B1)
            _lib.attn_rows(buf.q_buf, buf.kv_buf, *view, buf.src, rows, count, bucket, B1, N,
                           b0, nb, self.H, self.Hkv, self.hd, self.scaling, o32, buf.o_bf,
                           m_tab, z_tab, buf.ws_attn, prefix_len=plen)

    @staticmethod
    def _cache_key(cache):
        """A paged cache's or the mirror's identity for a captured graph (its
        buffers' addresses)."""
        if cache is None:
            return None
        if isinstance(cache, ContiguousMirror):
            return (id(cache), cache.k.data_ptr(), cache.v.data_ptr(),
                    cache.length_dev.data_ptr(), cache.capacity)
        return (id(cache), cache.k_pages.data_ptr(), cache.v_pages.data_ptr(),
                cache.page_table.data_ptr(), cache.length_dev.data_ptr(), cache.capacity)

    def invalidate_prefix(self) -> None:
        """Make the next step re-read a reference-style cache in full (after the
        caller rewrote it in place at the same length and tensors, which the
        engine's mirror cannot see)."""
        if self._mirror is not None:
            self._mirror.invalidate()

    def _mirror_of(self, cache, P: int) -> ContiguousMirror:
        """The engine's mirror of a reference-style cache, synced to it.  Capacity:
        the next power of two above the prefix (at least 1024 keys); outgrowing it
        allocates a larger mirror and drops the graphs captured against the old."""
        m = self._mirror
        if m is None or m.capacity < P:
            cap = max(1024, 1 << max(0, int(P) - 1).bit_length())
            self._graphs.clear()
            self._mirror = m = ContiguousMirror(self.L, self.Hkv, self.hd, cap,
                                                device=self.device)
        m.sync(cache)
        return m

    def _graph_key(self, buf: _Buffers, cache, P: int, delta: float, bucket: int,
                   q_scaled: bool = False, causal: bool = False):
        if _device_cache(cache):
            # the prefix length is read on the device: one graph for every length
            P = -1
            ck = self._cache_key(cache)
        elif cache is None:
            ck = None
        else:
            ck = tuple((prefix_view(cache, li).k.data_ptr(), prefix_view(cache, li).v.data_ptr())
                       if prefix_view(cache, li) is not None else (0, 0)
                       for li in range(self.L))
        return (buf.key, id(buf), P, float(delta), bucket, self.gate_mode, ck, q_scaled, causal)

    def _replay(self, buf: _Buffers, tokens: torch.Tensor, cache, P: int,
                delta: float, bucket: int, q_scaled: bool = False, causal: bool = False):
        """Run the layers through a captured HIP graph (captured on first use for
        this shape / prefix length / cache); inputs go through static buffers
        (the tokens, and buf.q_scale when q_scaled; the parent map is computed
        from the tokens inside the graph)."""
        key = self._graph_key(buf, cache, P, delta, bucket, q_scaled, causal)
        qs = buf.q_scale if q_scaled else None
        entry = self._graphs.get(key)
        if entry is None:
            static_tok = tokens.clone()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):      # warm-up launch outside the capture
                self._run_layers(buf, static_tok, cache, delta, bucket, q_scale=qs,
                                 causal=causal)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with _capturing(graph):
                out = self._run_layers(buf, static_tok, cache, delta, bucket, q_scale=qs,
                                       causal=causal)
            entry = (graph, static_tok, out)
            while len(self._graphs) >= self.max_graphs:
                self._graphs.pop(next(iter(self._graphs)))
            self._graphs[key] = entry
        graph, static_tok, out = entry
        static_tok.copy_(tokens)
        graph.replay()
        return out

    # ------------------------------------------------------------------------
    def profile_launchers(self, li: int = -1, shared: Optional[dict] = None):
        """No-argument callables that re-launch each HIP entry point of layer
        ``li`` (its weights, its slice of the cache) on the buffers resident from
        the last forward (for timing).  The gate runs on the last layer's output
        hidden states, so call it last: it rewrites rows/count/src for the other
        launchers.  ``shared`` (a dict) lets the launchers of several layers
        share their scratch outputs."""
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

        shared = {} if shared is None else shared
        if "scratch" not in shared:
            shared["scratch"] = torch.empty_like(buf.hid[0])
            shared["normed"] = torch.empty_like(buf.hid[0])
            shared["logits"] = torch.empty(BN, self.V_pad, dtype=torch.bfloat16,
                                           device=self.device)
        scratch, normed, logits = shared["scratch"], shared["normed"], shared["logits"]

        gate_mode = self.gate_mode | (_lib.SF_GATE_DEFER_COMPACT if self.gated_qkv else 0)

        def gate():
            # the fused gate of a layer after the first (residual update + gate; the
            # compaction too unless the QKV launcher runs it)
            _lib.fold_gate_residual(buf.hp, buf.ffn, buf.src, st["par"], lyr.input_layernorm.weight,
                                    B1, N, D, bucket, st["delta"], self.eps, gate_mode,
                                    scratch, buf.rec, buf.f, buf.src, buf.rows, count, buf.seg,
                                    segcnt, buf.slot, buf.rstd, buf.xn)

        cos, sin = self._rope
        pos0 = cache.length_dev if _device_cache(cache) else buf.pos0

        def qkv():
            if self.gated_qkv:
                _lib.qkv_rope_gated(buf.xn, buf.rec, st["par"], B1, N, bucket, buf.f, buf.src,
                                    buf.rows, count, buf.seg, segcnt, buf.slot, w_qkv, b_qkv,
                                    cos, sin, st["q_scale"], D, H, Hkv, hd, buf.q_buf,
                                    buf.kv_buf, buf.ws_qkv, pos0=pos0)
            else:
                _lib.qkv_rope(buf.xn, buf.rows, count, bucket, BN, w_qkv, b_qkv, cos, sin,
                              st["q_scale"], N, D, H, Hkv, hd, buf.q_buf, buf.kv_buf, buf.ws_qkv,
                              pos0=pos0)

        def attn():
            self._attention(buf, cache, li, count, bucket, B1, N)

        wo = self._packed_o[li]

        def o_proj():
            # o_proj + residual + post-attention norm (one entry point)
            _lib.o_proj_post_norm(buf.o_bf, hidden, wo, BN, H * hd, D, buf.slot,
                                  lyr.post_attention_layernorm.weight, self.eps, buf.hp, buf.zn,
                                  buf.ws_oproj)

        wg, wu, wd = self._packed_mlp[li]

        def gate_up():
            _lib.ffn_gate_up(buf.zn, count, bucket, wg, wu, D, self.I, buf.act, buf.ws_gemm)

        def down():
            _lib.ffn_down_scatter(buf.act, count, bucket, buf.rows, wd, self.I, D, buf.ffn,
                                  buf.ws_gemm)

        def final_norm():
            _lib.residual_rmsnorm(buf.hp, buf.ffn, buf.src, self.base.norm.weight, B1, N, D,
                                  self.eps, scratch, normed)

        def lm_head():
            self.lm_head(buf.final, out=logits, shift_n=N if st.get("shift") else 0)

        out = dict(qkv=qkv, attn=attn, o_proj=o_proj, gate_up=gate_up, down=down,
                   final_norm=final_norm, lm_head=lm_head, gate=gate)
        if isinstance(cache, PagedKVCache) and cache.length + N <= cache.capacity:
            def append():
                # writes past the logical end of the cache: never read, length unchanged
                cache.append_rows(li, buf.kv_buf, 0, N, start_pos=cache.length)
            out["append"] = append
        return out, dict(count=count, buf=buf, prefix=pv.length if pv else 0)
