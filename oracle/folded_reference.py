"""ORACLE (test infrastructure): CPU restatement of the reference folded verify step.

Restates ``SpecFoldFastDLLMV2Generation._batched_block_forward``
(chungen04/specfold specfold/generate/fastdllm_v2_folded.py:89-223) with the same
per-op dtypes, so that on CPU it reproduces the reference's bf16 rounding
trajectory.  Every numbered step below cites the reference line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this.

The NLD variant (specfold/generate/nld_folded.py:89-237) is the same step with
the decoder at ``model.encoder`` and the head at ``model.diffusion_head``, no QKV
bias, the config's RMSNorm eps, no logit shift, and the llama-4 q scale after
RoPE (``q_scale``; nld_folded.py:37-53, 173-174).

The model argument is any module tree with the Qwen2 layout the reference reads:
``model.model.{embed_tokens, rotary_emb, layers[i], norm}``, ``model.lm_head``,
``model.config`` and per layer ``input_layernorm``,
``self_attn.{q,k,v,o}_proj`` (+ ``head_dim``, ``scaling``, ``layer_idx``),
``post_attention_layernorm`` and ``mlp.{gate,up,down}_proj``.
``past_key_values`` is a sequence of per-layer ``(k, v)`` tensors
``[1, Hkv, P, hd]`` (or anything with that indexing contract), or None.

How each function is pinned (all CPU tests):
  folded_verify_step / folded_layer / shift_logits / rope_tables — bit-exact
      against golden vectors written by the reference class itself
      (tests/golden, tests/test_oracle_golden.py);
  dense_layer — transformers' Qwen2DecoderLayer; with causal=True and q_scale,
      transformers' Ministral3ForCausalLM over [prefix; block] (test_oracle_pins.py,
      test_oracle_nld.py);
  folded == dense with every row recomputed (both families);
  chain-corrected (m, Z, O) — exact_branch_attention, fp64 brute force;
  parent_map / topo_order — exhaustive small families + hypothesis;
  llama4_q_scale — its closed form at the window boundaries.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F


# ---------------------------------------------------------------------------
# small primitives
# ---------------------------------------------------------------------------

def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """Qwen2/Llama rotate_half: (x1, x2) -> (-x2, x1) over the last dim.
    Follows fastdllm_v2_folded.py:22-25."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def expand_kv_heads(t: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[b, Hkv, s, d] -> [b, Hkv*n_rep, s, d], each kv head repeated n_rep times
    consecutively (GQA).  Follows fastdllm_v2_folded.py:29-34."""
    if n_rep == 1:
        return t
    b, hkv, s, d = t.shape
    return t[:, :, None].expand(b, hkv, n_rep, s, d).reshape(b, hkv * n_rep, s, d)


def parent_map(batched_input: torch.Tensor) -> Tuple[List[Optional[int]], List[int]]:
    """Parent of each draft branch.  Follows fastdllm_v2_folded.py:55-75.

    diff(i) = positions where branch i differs from branch 0 (main).
    parent(i) = the lowest-indexed j != i with |diff(j)| == |diff(i)| - 1 and
    diff(j) a subset of diff(i); 0 (main) when no such j exists.  Branch 0 has
    parent None.  Returns (parent, counts) with counts[i] = |diff(i)|.
    """
    bi = batched_input.detach().cpu()
    diff = (bi != bi[0:1]).tolist()
    b1 = len(diff)
    counts = [sum(1 for v in row if v) for row in diff]
    parent: List[Optional[int]] = [None] * b1
    for i in range(1, b1):
        chosen = 0
        for j in range(b1):
            if j == i or counts[j] != counts[i] - 1:
                continue
            if all((not dj) or di for dj, di in zip(diff[j], diff[i])):
                chosen = j
                break
        parent[i] = chosen
    return parent, counts


def topo_order(counts: Sequence[int]) -> List[int]:
    """Branches by ascending diff count, ties by index (stable sort): every
    parent precedes its children.  Follows fastdllm_v2_folded.py:108."""
    return sorted(range(len(counts)), key=lambda i: counts[i])


# ---------------------------------------------------------------------------
# trace containers
# ---------------------------------------------------------------------------

@dataclass
class LayerTrace:
    """Per-layer intermediates of one verify step (all on CPU)."""
    h_in: torch.Tensor = None      # [B1, N, D]    model dtype
    rec: torch.Tensor = None       # [B1, N]       bool (row 0 all True)
    q: torch.Tensor = None         # [B1, H, N, hd] model dtype (roped)
    k: torch.Tensor = None         # [B1, Hkv, N, hd]
    v: torch.Tensor = None         # [B1, Hkv, N, hd]
    m: torch.Tensor = None         # [B1, H, N]    fp32
    Z: torch.Tensor = None         # [B1, H, N]    fp32
    O: torch.Tensor = None         # [B1, H, N, hd] fp32
    hp: torch.Tensor = None        # [B1, N, D]    residual after attention
    ffn: torch.Tensor = None       # [B1, N, D]    per-row FFN output table
    h_out: torch.Tensor = None     # [B1, N, D]


@dataclass
class StepTrace:
    parent: List[Optional[int]] = None
    counts: List[int] = None
    layers: List[LayerTrace] = field(default_factory=list)
    final_hidden: torch.Tensor = None   # [B1, N, D] after the last layer (pre-norm)
    logits: torch.Tensor = None         # [B1, N, V] shifted (or not, per shift flag)


@dataclass
class FoldCounters:
    """fold_ratio bookkeeping.  Follows fastdllm_v2_folded.py:49-53, 142-143."""
    draft_positions: int = 0
    draft_recomputed: int = 0

    @property
    def fold_ratio(self) -> float:
        if not self.draft_positions:
            return float("nan")
        return 1.0 - self.draft_recomputed / self.draft_positions


# ---------------------------------------------------------------------------
# one layer
# ---------------------------------------------------------------------------

def delta_gate(x: torch.Tensor, x_par: torch.Tensor, delta: float) -> torch.Tensor:
    """Recompute mask [N] of a draft branch: relative L2 residual against its
    parent's hidden states, both norms taken in the model dtype.  Follows
    fastdllm_v2_folded.py:136-141 (``(x - xp).norm(-1) > delta * xp.norm(-1)``).
    ``x``, ``x_par``: [1, N, D]."""
    resid_norm = (x[0] - x_par[0]).norm(dim=-1)
    par_norm = x_par[0].norm(dim=-1)
    return resid_norm > delta * par_norm


def gate_margin(x: torch.Tensor, x_par: torch.Tensor, delta: float) -> torch.Tensor:
    """fp64 distance of each position from the gate's threshold,
    ||x - x_par|| / ||x_par|| - delta (diagnostic for a mask disagreement)."""
    xd, pd = x[0].double(), x_par[0].double()
    return (xd - pd).norm(dim=-1) / pd.norm(dim=-1).clamp_min(1e-300) - delta


def folded_layer(
    lyr,
    h: List[torch.Tensor],
    parent: List[Optional[int]],
    order: List[int],
    prefix_kv: Optional[Tuple[torch.Tensor, torch.Tensor]],
    cos_n: torch.Tensor,
    sin_n: torch.Tensor,
    delta: float,
    n_heads: int,
    n_kv_heads: int,
    counters: Optional[FoldCounters] = None,
    trace: Optional[LayerTrace] = None,
    q_scale: Optional[torch.Tensor] = None,
    qkv_rows=None,
) -> List[torch.Tensor]:
    """One decoder layer of the folded verify step for all B1 branches.

    Follows fastdllm_v2_folded.py:117-220 (and nld_folded.py:132-232, which adds
    ``q_scale``).  ``h`` is a list of B1 tensors [1, N, D]; returns the list of
    next-layer hidden states.

    ``qkv_rows`` (stage forcing, for tests): a callable (branch i, recomputed
    positions rsel) -> (q [H, n, hd], k [Hkv, n, hd], v [Hkv, n, hd]) that
    replaces the roped (and scaled) projections of those rows, so that the
    attention and the chain correction below run on given q/k/v.
    """
    attn = lyr.self_attn
    hd = attn.head_dim
    scaling = attn.scaling
    H, Hkv = n_heads, n_kv_heads
    G = H // Hkv
    B1 = len(h)
    N = h[0].shape[1]
    D = h[0].shape[2]
    dev = h[0].device
    x_dtype = h[0].dtype

    # :122-126 prefix K/V with kv heads repeated to all q heads
    if prefix_kv is not None and prefix_kv[0] is not None:
        pk, pv = prefix_kv
        pre_k = expand_kv_heads(pk, G)[0]      # [H, P, hd]
        pre_v = expand_kv_heads(pv, G)[0]
    else:
        pre_k = pre_v = None

    # per-branch tables, filled in topological order (:128-131)
    q_tab: List[Optional[torch.Tensor]] = [None] * B1
    k_tab: List[Optional[torch.Tensor]] = [None] * B1
    v_tab: List[Optional[torch.Tensor]] = [None] * B1
    m_tab: List[Optional[torch.Tensor]] = [None] * B1
    z_tab: List[Optional[torch.Tensor]] = [None] * B1
    o_tab: List[Optional[torch.Tensor]] = [None] * B1
    f_tab: List[Optional[torch.Tensor]] = [None] * B1
    hp_out: List[Optional[torch.Tensor]] = [None] * B1
    h_next: List[Optional[torch.Tensor]] = [None] * B1
    rec_mask = torch.zeros(B1, N, dtype=torch.bool)

    for i in order:
        x = h[i]
        p = parent[i]

        # (1) delta gate :136-144 — relative L2 residual against the parent,
        # norms taken in the model dtype.
        if p is None:
            rsel = torch.arange(N, device=dev)
        else:
            rsel = delta_gate(x, h[p], delta).nonzero(as_tuple=True)[0]
            if counters is not None:
                counters.draft_positions += N
                counters.draft_recomputed += int(rsel.numel())
        n_rec = int(rsel.numel())
        rec_mask[i, rsel.cpu()] = True

        # (2) Q/K/V tables: inherit the parent's, overwrite recomputed rows :147-162
        if p is None:
            qt = x.new_zeros(H, N, hd)
            kt = x.new_zeros(Hkv, N, hd)
            vt = x.new_zeros(Hkv, N, hd)
        else:
            qt = q_tab[p].clone()
            kt = k_tab[p].clone()
            vt = v_tab[p].clone()
        k_prev = v_prev = None
        if n_rec:
            normed = lyr.input_layernorm(x)[0, rsel]
            qn = attn.q_proj(normed).view(n_rec, H, hd).transpose(0, 1)
            kn = attn.k_proj(normed).view(n_rec, Hkv, hd).transpose(0, 1)
            vn = attn.v_proj(normed).view(n_rec, Hkv, hd).transpose(0, 1)
            c = cos_n[rsel].unsqueeze(0)
            s = sin_n[rsel].unsqueeze(0)
            qn = qn * c + rotate_half(qn) * s
            kn = kn * c + rotate_half(kn) * s
            if q_scale is not None:                               # nld_folded.py:173-174
                qn = qn * q_scale.to(qn.device)[rsel].view(1, n_rec, 1).to(qn.dtype)
            if qkv_rows is not None:
                qn, kn, vn = (t.to(device=dev, dtype=x_dtype) for t in qkv_rows(i, rsel))
            if p is not None:
                k_prev = kt[:, rsel].clone()
                v_prev = vt[:, rsel].clone()
            qt[:, rsel] = qn
            kt[:, rsel] = kn
            vt[:, rsel] = vn
        q_tab[i], k_tab[i], v_tab[i] = qt, kt, vt

        # keys/values seen by this branch: [prefix ; branch table] (:164-167)
        k_all_h = expand_kv_heads(kt.unsqueeze(0), G)[0] if Hkv != H else kt
        v_all_h = expand_kv_heads(vt.unsqueeze(0), G)[0] if Hkv != H else vt
        keys = torch.cat([pre_k, k_all_h], dim=1) if pre_k is not None else k_all_h
        vals = torch.cat([pre_v, v_all_h], dim=1) if pre_v is not None else v_all_h

        # (3) softmax state tables, inherited from the parent (:169-173)
        mt = torch.full((H, N), float("-inf"), dtype=torch.float32, device=dev)
        zt = torch.zeros(H, N, dtype=torch.float32, device=dev)
        ot = torch.zeros(H, N, hd, dtype=torch.float32, device=dev)
        if p is not None:
            mt.copy_(m_tab[p])
            zt.copy_(z_tab[p])
            ot.copy_(o_tab[p])

        # recomputed rows: exact fp32 attention keeping (m, Z, O) (:175-181)
        if n_rec:
            sc = torch.einsum("hrd,hkd->hrk", qt[:, rsel].float(), keys.float()) * scaling
            row_max = sc.max(dim=-1).values
            ex = torch.exp(sc - row_max.unsqueeze(-1))
            den = ex.sum(-1)
            out = torch.einsum("hrk,hkd->hrd", ex, vals.float()) / den.unsqueeze(-1)
            mt[:, rsel] = row_max
            zt[:, rsel] = den
            ot[:, rsel] = out

        # (4) folded rows: one-hop correction from the parent's state for the
        # keys this branch changed (:183-204)
        if p is not None and n_rec:
            keep = torch.ones(N, dtype=torch.bool, device=dev)
            keep[rsel] = False
            lsel = keep.nonzero(as_tuple=True)[0]
            if lsel.numel():
                qf = qt[:, lsel].float()
                k_old = expand_kv_heads(k_prev.unsqueeze(0), G)[0] if Hkv != H else k_prev
                v_old = expand_kv_heads(v_prev.unsqueeze(0), G)[0] if Hkv != H else v_prev
                k_new = k_all_h[:, rsel]
                v_new = v_all_h[:, rsel]
                s_old = torch.einsum("hld,hed->hle", qf, k_old.float()) * scaling
                s_new = torch.einsum("hld,hed->hle", qf, k_new.float()) * scaling
                m_par = m_tab[p][:, lsel]
                m_cur = torch.maximum(m_par, s_new.max(-1).values)
                rescale = torch.exp(m_par - m_cur)
                a_old = torch.exp(s_old - m_cur.unsqueeze(-1))
                a_new = torch.exp(s_new - m_cur.unsqueeze(-1))
                z_scaled = z_tab[p][:, lsel] * rescale
                num = o_tab[p][:, lsel] * z_scaled.unsqueeze(-1)
                num = num - torch.einsum("hle,hed->hld", a_old, v_old.float()) \
                    + torch.einsum("hle,hed->hld", a_new, v_new.float())
                z_cur = z_scaled - a_old.sum(-1) + a_new.sum(-1)
                mt[:, lsel] = m_cur
                zt[:, lsel] = z_cur
                ot[:, lsel] = num / z_cur.unsqueeze(-1)
        m_tab[i], z_tab[i], o_tab[i] = mt, zt, ot

        # (5) o_proj + residual for every row, in the model dtype (:207-209)
        o_rows = ot.permute(1, 0, 2).reshape(N, H * hd).to(x_dtype)
        hpi = x + (o_rows @ attn.o_proj.weight.t()).unsqueeze(0)
        hp_out[i] = hpi

        # (6) FFN on recomputed rows; folded rows reuse the parent's output (:211-218)
        ft = f_tab[p].clone() if p is not None else x.new_zeros(1, N, D)
        if n_rec:
            mlp = lyr.mlp
            z = lyr.post_attention_layernorm(hpi[0, rsel])
            ft[0, rsel] = mlp.down_proj(F.silu(mlp.gate_proj(z)) * mlp.up_proj(z))
        f_tab[i] = ft
        h_next[i] = hpi + ft

    if trace is not None:
        trace.h_in = torch.cat(h, 0).detach().cpu()
        trace.rec = rec_mask
        trace.q = torch.stack(q_tab).cpu()
        trace.k = torch.stack(k_tab).cpu()
        trace.v = torch.stack(v_tab).cpu()
        trace.m = torch.stack(m_tab).cpu()
        trace.Z = torch.stack(z_tab).cpu()
        trace.O = torch.stack(o_tab).cpu()
        trace.hp = torch.cat(hp_out, 0).cpu()
        trace.ffn = torch.cat(f_tab, 0).cpu()
        trace.h_out = torch.cat(h_next, 0).cpu()
    return h_next


# ---------------------------------------------------------------------------
# the whole step
# ---------------------------------------------------------------------------

def rope_tables(model, hidden: torch.Tensor, P: int, N: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [N, hd] for block positions P..P+N-1, via the model's rotary
    module in the model dtype.  Follows fastdllm_v2_folded.py:112-114."""
    pos = torch.arange(P, P + N, device=hidden.device).unsqueeze(0)
    cos, sin = decoder_parts(model)[0].rotary_emb(hidden, pos)
    return cos[0], sin[0]


def shift_logits(logits: torch.Tensor) -> torch.Tensor:
    """Position i takes the logits of position i-1 (position 0 keeps its own).
    Follows fastdllm_v2_generation.py:121-126."""
    return torch.cat([logits[:, :1], logits[:, :-1]], dim=1)


def decoder_parts(model):
    """(decoder, head): ``model.model`` / ``model.lm_head`` (fastdllm_v2_folded.py:
    105-108, 222) or ``model.encoder`` / ``model.diffusion_head`` (nld_folded.py:
    105-108, 237)."""
    base = getattr(model, "model", None)
    if base is None or not hasattr(base, "layers"):
        base = model.encoder
    head = getattr(model, "lm_head", None)
    if head is None:
        head = model.diffusion_head
    return base, head


def llama4_q_scale(cfg, P: int, N: int) -> Optional[torch.Tensor]:
    """Per-position llama-4 attention scale for block positions [P, P+N), fp32,
    or None when it is identically 1.  Follows nld_folded.py:37-53 (the scale of
    modeling_ministral.py:104-106: 1 + beta * log(1 + floor(pos / omax)))."""
    rp = getattr(cfg, "rope_parameters", None) or {}
    beta = rp.get("llama_4_scaling_beta")
    omax = rp.get("original_max_position_embeddings")
    if beta is None or omax is None:
        return None
    pos = torch.arange(P, P + N, dtype=torch.float32)
    scale = 1.0 + beta * torch.log(1.0 + torch.floor(pos / omax))
    if bool((scale == 1.0).all()):
        return None
    return scale


def prefix_length(past_key_values) -> int:
    if past_key_values is None:
        return 0
    if hasattr(past_key_values, "get_seq_length"):
        return int(past_key_values.get_seq_length())
    return int(past_key_values[0][0].shape[-2]) if len(past_key_values) else 0


@torch.no_grad()
def folded_verify_step(
    model,
    batched_input: torch.Tensor,
    past_key_values=None,
    delta: float = 0.1,
    counters: Optional[FoldCounters] = None,
    trace: Optional[StepTrace] = None,
    shift: bool = True,
    teacher_hidden: Optional[Dict[int, torch.Tensor]] = None,
    q_scale: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Folded verify step for B1 >= 2 branches -> logits [B1, N, V].

    Follows fastdllm_v2_folded.py:89-223 (the B1 >= 2 branch; B1 == 1 goes to
    the dense model forward in the reference, :91-95, restated by
    ``dense_verify_step``).  ``teacher_hidden[li]`` (optional) replaces layer
    li's input hidden states, for stage-by-stage comparison.
    """
    base, head = decoder_parts(model)
    cfg = model.config
    B1, N = batched_input.shape
    H = cfg.num_attention_heads
    Hkv = cfg.num_key_value_heads
    P = prefix_length(past_key_values)

    parent, counts = parent_map(batched_input)
    order = topo_order(counts)
    if trace is not None:
        trace.parent, trace.counts = parent, counts

    hidden = base.embed_tokens(batched_input)                      # :110
    cos_n, sin_n = rope_tables(model, hidden, P, N)                # :112-114
    h = [hidden[i:i + 1] for i in range(B1)]                       # :115

    for li, lyr in enumerate(base.layers):                         # :117
        if teacher_hidden is not None and li in teacher_hidden:
            th = teacher_hidden[li].to(hidden.dtype)
            h = [th[i:i + 1] for i in range(B1)]
        kv = None
        if past_key_values is not None and len(past_key_values) > li:
            kv = past_key_values[li]
        lt = LayerTrace() if trace is not None else None
        h = folded_layer(lyr, h, parent, order, kv, cos_n, sin_n, float(delta),
                         H, Hkv, counters=counters, trace=lt, q_scale=q_scale)
        if trace is not None:
            trace.layers.append(lt)

    final_h = torch.cat(h, dim=0)
    logits = head(base.norm(final_h))                              # :222-223
    if shift:
        logits = shift_logits(logits)
    if trace is not None:
        trace.final_hidden = final_h.cpu()
        trace.logits = logits.cpu()
    return logits


# ---------------------------------------------------------------------------
# dense baseline (the B1 == 1 / gate-off path)
# ---------------------------------------------------------------------------

def dense_layer(lyr, x: torch.Tensor, prefix_kv, cos_n, sin_n, n_heads: int, n_kv_heads: int,
                return_kv: bool = False, q_scale: Optional[torch.Tensor] = None,
                causal: bool = False):
    """Plain (unfolded) decoder layer for a [B, N, D] block that attends to the
    whole prefix and bidirectionally within the block, attention in fp32.

    This is what every folded row reduces to when the gate recomputes it, and
    it is the block-diffusion forward the reference's dense seam runs
    (fastdllm_v2_generation.py:151-186) for a block with a prefix cache.
    ``causal``: block position n sees block positions <= n only (the causal AR
    forward NLD commits blocks with, nld_generation.py:300-310).
    """
    attn = lyr.self_attn
    hd, scaling = attn.head_dim, attn.scaling
    H, Hkv = n_heads, n_kv_heads
    G = H // Hkv
    B, N, D = x.shape
    normed = lyr.input_layernorm(x)
    q = attn.q_proj(normed).view(B, N, H, hd).transpose(1, 2)
    k = attn.k_proj(normed).view(B, N, Hkv, hd).transpose(1, 2)
    v = attn.v_proj(normed).view(B, N, Hkv, hd).transpose(1, 2)
    c, s = cos_n[None, None], sin_n[None, None]
    q = q * c + rotate_half(q) * s
    k = k * c + rotate_half(k) * s
    if q_scale is not None:
        q = q * q_scale.to(q.device).view(1, 1, N, 1).to(q.dtype)
    kk, vv = expand_kv_heads(k, G), expand_kv_heads(v, G)
    if prefix_kv is not None and prefix_kv[0] is not None:
        pk, pv = prefix_kv
        kk = torch.cat([expand_kv_heads(pk, G).expand(B, -1, -1, -1), kk], dim=2)
        vv = torch.cat([expand_kv_heads(pv, G).expand(B, -1, -1, -1), vv], dim=2)
    sc = torch.einsum("bhnd,bhkd->bhnk", q.float(), kk.float()) * scaling
    if causal:
        P = kk.shape[2] - N
        blk = torch.ones(N, N, dtype=torch.bool, device=sc.device).triu(1)
        sc[..., P:] = sc[..., P:].masked_fill(blk, float("-inf"))
    w = torch.softmax(sc, dim=-1)
    o = torch.einsum("bhnk,bhkd->bhnd", w, vv.float())
    o = o.transpose(1, 2).reshape(B, N, H * hd).to(x.dtype)
    hp = x + o @ attn.o_proj.weight.t()
    mlp = lyr.mlp
    z = lyr.post_attention_layernorm(hp)
    out = hp + mlp.down_proj(F.silu(mlp.gate_proj(z)) * mlp.up_proj(z))
    if return_kv:
        return out, (k, v)
    return out


@torch.no_grad()
def dense_verify_step(model, batched_input: torch.Tensor, past_key_values=None, shift: bool = True,
                      return_new_kv: bool = False, q_scale: Optional[torch.Tensor] = None,
                      causal: bool = False):
    """Dense block forward of every branch (no folding) -> logits [B1, N, V].

    With ``return_new_kv`` also returns the per-layer (k, v) [B1, Hkv, N, hd]
    of the block, i.e. what a block-commit forward appends to the cache
    (fastdllm_v2_generation.py:557-575)."""
    base, head = decoder_parts(model)
    cfg = model.config
    B1, N = batched_input.shape
    P = prefix_length(past_key_values)
    x = base.embed_tokens(batched_input)
    cos_n, sin_n = rope_tables(model, x, P, N)
    new_kv = []
    for li, lyr in enumerate(base.layers):
        kv = past_key_values[li] if past_key_values is not None and len(past_key_values) > li else None
        x, kvb = dense_layer(lyr, x, kv, cos_n, sin_n, cfg.num_attention_heads,
                             cfg.num_key_value_heads, return_kv=True, q_scale=q_scale,
                             causal=causal)
        new_kv.append(kvb)
    logits = head(base.norm(x))
    if shift:
        logits = shift_logits(logits)
    if return_new_kv:
        return logits, new_kv
    return logits


# ---------------------------------------------------------------------------
# exact references used to pin the restatement
# ---------------------------------------------------------------------------

def exact_branch_attention(q: torch.Tensor, keys: torch.Tensor, vals: torch.Tensor, scaling: float):
    """fp64 softmax attention with its (m, Z) state.

    q [H, L, hd], keys/vals [H, K, hd] -> (m [H, L], Z [H, L], O [H, L, hd]) with
    m = max_k s, Z = sum_k exp(s - m), O = sum_k exp(s - m) v / Z."""
    s = torch.einsum("hld,hkd->hlk", q.double(), keys.double()) * scaling
    m = s.max(-1).values
    e = torch.exp(s - m.unsqueeze(-1))
    z = e.sum(-1)
    o = torch.einsum("hlk,hkd->hld", e, vals.double()) / z.unsqueeze(-1)
    return m, z, o
