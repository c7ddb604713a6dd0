"""The attention kernels alone (prefix pass + block/merge) against an fp32 torch
reference, at prefix lengths where the prefix pass splits the keys into ranges
of several chunks (long contexts) as well as one chunk per work item.

Each recomputed row r = b*N + n attends to [prefix keys ; block keys j of
branch src[b*N + j]] (fastdllm_v2_folded.py:164-181), optionally causally within
the block.  Tolerances: O within 2e-3 of max|O| (fp32 accumulation, P split
into bf16 hi + lo), m and Z within 2e-3 relative.
"""

import pytest
import torch

from specfold_amd import _lib
from specfold_amd.kv_cache import PagedKVCache
from tests.helpers import err_stats

pytestmark = pytest.mark.gpu

HD = 128


def reference(q_buf, kv_buf, pk, pv, src, rows, B1, N, H, Hkv, scaling, causal):
    """fp32 softmax attention of every listed row -> (O [R, H, hd], m [R, H], Z [R, H])."""
    G = H // Hkv
    kv = kv_buf[:B1 * N].float().view(B1 * N, 2, Hkv, HD)
    out_o, out_m, out_z = [], [], []
    for r in rows.tolist():
        b, n = divmod(r, N)
        q = q_buf[r].float().view(H, HD)
        brow = src[b * N:(b + 1) * N].long() * N + torch.arange(N, device=q.device)
        bk = kv[brow, 0].permute(1, 0, 2)                        # [Hkv, N, hd]
        bv = kv[brow, 1].permute(1, 0, 2)
        keys = torch.cat([pk.float(), bk], dim=1) if pk is not None else bk
        vals = torch.cat([pv.float(), bv], dim=1) if pv is not None else bv
        keys = keys.repeat_interleave(G, dim=0)                 # [H, P+N, hd]
        vals = vals.repeat_interleave(G, dim=0)
        s = torch.einsum("hd,hkd->hk", q, keys) * scaling
        if causal:
            P = s.shape[1] - N
            s[:, P + n + 1:] = float("-inf")
        m = s.max(dim=1).values
        e = torch.exp(s - m[:, None])
        z = e.sum(dim=1)
        out_o.append(torch.einsum("hk,hkd->hd", e, vals) / z[:, None])
        out_m.append(m)
        out_z.append(z)
    return torch.stack(out_o), torch.stack(out_m), torch.stack(out_z)


def run_case(P, B1, N, H, Hkv, count, seed, causal=False, P_cap=None, page_size=16,
             key_ramp=None):
    torch.manual_seed(seed)
    dev = "cuda"
    BN = B1 * N
    bucket = BN
    q_buf = torch.randn(BN + 1, H * HD, device=dev).to(torch.bfloat16)
    kv_buf = torch.randn(BN + 1, 2 * Hkv * HD, device=dev).to(torch.bfloat16)
    # each branch inherits block positions from itself or an earlier branch
    src = torch.stack([torch.randint(0, b + 1, (N,)) for b in range(B1)]).flatten()
    src = src.to(torch.int32).to(dev)
    rows = torch.sort(torch.randperm(BN)[:count]).values.to(torch.int32)
    rows_pad = torch.full((bucket,), BN, dtype=torch.int32)
    rows_pad[:count] = rows
    rows_pad = rows_pad.to(dev)
    cnt = torch.tensor([count], dtype=torch.int32, device=dev)
    pk = pv = None
    cache = None
    if P > 0:
        cap = P_cap or P
        cache = PagedKVCache(1, Hkv, HD, cap, page_size=page_size, device=dev,
                             page_order="shuffled", seed=seed)
        pk = torch.randn(1, Hkv, P, HD, device=dev)
        if key_ramp is not None:
            # key magnitudes growing along the prefix: the scores' maximum keeps rising
            pk = pk * torch.linspace(key_ramp[0], key_ramp[1], P, device=dev)[None, None, :, None]
        pk = pk.to(torch.bfloat16)
        pv = torch.randn(1, Hkv, P, HD, device=dev).to(torch.bfloat16)
        cache.load_dense([(pk, pv)])
    o32 = torch.zeros(BN, H * HD, device=dev)
    o_bf = torch.zeros(BN, H * HD, device=dev, dtype=torch.bfloat16)
    m_tab = torch.zeros(BN, H, device=dev)
    z_tab = torch.zeros(BN, H, device=dev)
    scaling = HD ** -0.5
    def call(o32, o_bf, m_tab, z_tab):
        if cache is not None:
            vw = cache.view(0)
            ws = torch.zeros(_lib.attn_workspace_bytes(bucket, H, vw.capacity),
                             dtype=torch.uint8, device=dev)
            _lib.attn_prefix_block(q_buf, kv_buf, vw.k, vw.v, vw.page_table, vw.capacity,
                                   vw.page_size, vw.page_stride, vw.head_stride, src, rows_pad,
                                   cnt, bucket, B1, N, H, Hkv, HD, scaling, o32, o_bf, m_tab,
                                   z_tab, ws, prefix_len=vw.length_dev, block_causal=causal)
        else:
            ws = torch.zeros(256, dtype=torch.uint8, device=dev)
            _lib.attn_prefix_block(q_buf, kv_buf, None, None, None, 0, 1, 0, 0, src, rows_pad,
                                   cnt, bucket, B1, N, H, Hkv, HD, scaling, o32, o_bf, m_tab,
                                   z_tab, ws, block_causal=causal)

    call(o32, o_bf, m_tab, z_tab)
    # without the side outputs (fp32 O, m, Z: what the verify step skips) the bf16
    # output is the same
    o_bf2 = torch.zeros_like(o_bf)
    call(None, o_bf2, None, None)
    torch.cuda.synchronize()
    r = rows.long().to(dev)
    assert torch.equal(o_bf2[r], o_bf[r])
    ro, rm, rz = reference(q_buf, kv_buf, pk[0] if pk is not None else None,
                           pv[0] if pv is not None else None, src, rows.to(dev), B1, N, H, Hkv,
                           scaling, causal)
    got_o = o32[r].view(-1, H, HD)
    st = err_stats(got_o.cpu(), ro.cpu())
    print(f"P={P} H={H}/{Hkv} R={count}: O {st}")
    assert st["max_abs"] <= 2e-3 * st["ref_absmax"]
    assert torch.allclose(m_tab[r], rm, rtol=2e-3, atol=2e-3)
    assert torch.allclose(z_tab[r], rz, rtol=2e-3, atol=1e-3)
    # bf16 output is the rounded fp32 output
    assert torch.equal(o_bf[r], o32[r].to(torch.bfloat16))


# (P, B1, N, H, Hkv, count): the prefix pass takes chunks of 64 keys, query tiles of
# 128 (n_qt = ceil(count*G/128)) and cpi = max(ceil(nch*n_qt*Hkv/256), ceil(nch/64))
# chunks per work item, nch = ceil(P/64)
CASES = [
    (16384, 8, 32, 40, 8, 39),      # 16 chunks per item, 16 ranges
    (16389, 8, 32, 40, 8, 39),      # 17 per item; ragged last chunk (5 keys) in a 2-chunk range
    (32768, 8, 32, 8, 8, 256),      # 32 per item, G = 1, every row
    (3000, 8, 32, 28, 4, 100),      # 5 per item, 6 query tiles
    (700, 2, 32, 16, 2, 5),         # one chunk per item, short prefix, few rows
    (20, 2, 32, 16, 2, 7),          # one 20-key chunk: the second key half of every wave empty
]


@pytest.mark.parametrize("P,B1,N,H,Hkv,count", CASES)
def test_attention_matches_fp32(P, B1, N, H, Hkv, count):
    run_case(P, B1, N, H, Hkv, count, seed=P % 97)


def test_attention_device_length_below_capacity():
    """Grid and workspace sized for 20000 keys, 9000 present (read on the device)."""
    run_case(9000, 8, 32, 40, 8, 60, seed=3, P_cap=20000)


def test_attention_causal_block_long_prefix():
    run_case(12000, 1, 32, 32, 8, 32, seed=5, causal=True)


def test_attention_no_prefix():
    run_case(0, 4, 32, 28, 4, 50, seed=6)


@pytest.mark.parametrize("P,B1,N,H,Hkv,count,ramp", [
    (16384, 8, 32, 40, 8, 39, (0.1, 8.0)),   # rising: the maximum passes the softmax
    (3000, 8, 32, 28, 4, 100, (0.1, 8.0)),   # reference many times inside a range
    (16384, 8, 32, 40, 8, 39, (8.0, 0.1)),   # falling: set by the first chunks
])
def test_attention_rising_and_falling_scores(P, B1, N, H, Hkv, count, ramp):
    """Scores whose maximum grows by several powers of two from chunk to chunk (the
    prefix pass moves its softmax reference up each time the maximum passes it by
    2^8, rescaling the accumulated terms) or shrinks along the prefix (one
    reference for the whole range)."""
    run_case(P, B1, N, H, Hkv, count, seed=11, key_ramp=ramp)
