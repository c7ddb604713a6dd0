"""The weight-streaming GEMM entry points against PyTorch references of the same
ops computed in fp64 on the CPU and rounded at the reference's bf16 rounding
points.  Tolerance: at most 0.5% of outputs may differ, each by at most one bf16
ulp (2^-7 relative) of the stated scale — the fp32 accumulation lands on the
other side of a rounding tie now and then (torch's own fp32 GEMM does too).

Weights go through sf_pack_weight (checked bit-exact against the layout's
definition); workspaces are reused across calls."""

import pytest
import torch
import torch.nn.functional as F

from specfold_amd import _lib

pytestmark = pytest.mark.gpu


def close_bf16(a, b, frac=5e-3, scale=None, atol=None):
    """scale: magnitude the rounding error is relative to (defaults to |b|; for a
    residual sum x + y it is |x + y| + |y|: one ulp of y, which survives
    cancellation, plus the re-rounding of the sum).  atol: absolute slack for
    fp32 accumulation under cancellation (see acc_bound)."""
    a = a.float().cpu()
    b = b.float().cpu()
    d = (a - b).abs()
    sc = b.abs() if scale is None else scale.float().cpu().abs()
    tol = 2 ** -7 * sc + 1e-6
    if atol is not None:
        tol = tol + atol.float().cpu()
    bad = d > tol
    diff = (d > 0).float().mean().item()
    assert int(bad.sum()) == 0, f"{int(bad.sum())} elements beyond 2 ulps, max {d.max().item()}"
    assert diff <= frac, f"{diff:.4f} of elements differ"


def mm64(a, w):
    """a @ w^T in fp64 on the CPU, rounded to bf16 (a bf16 GEMM output)."""
    return (a.double().cpu() @ w.double().cpu().t()).to(torch.bfloat16)


def acc_bound(a, w):
    """Statistical bound of fp32 accumulation error of a K-term dot product:
    2 * sqrt(K) * 2^-24 * sum_k |a_k w_k|.  Matters only where the terms cancel
    (an exact result far below sum |a_k w_k|)."""
    K = a.shape[-1]
    return 2 * K ** 0.5 * 2 ** -24 * (a.double().abs().cpu() @ w.double().abs().cpu().t())


def rnd(*shape, std=1.0, gen=None):
    return (std * torch.randn(*shape, generator=gen)).to(torch.bfloat16).cuda()


def packed(w):
    return _lib.pack_weight(w)


def zeros_ws(nbytes):
    return torch.zeros(nbytes, dtype=torch.uint8, device="cuda")


@pytest.mark.parametrize("N,K", [(16, 128), (48, 256), (4608, 3584)])
def test_pack_weight_layout(N, K):
    """word (t, c, l) = W[16t + l%16][32c + 8(l/16) .. +8], compared bit for bit
    with the layout written out by index arithmetic on the CPU."""
    g = torch.Generator().manual_seed(N + K)
    w = torch.randint(-32768, 32767, (N, K), generator=g, dtype=torch.int16)
    out = _lib.pack_weight(w.view(torch.bfloat16).cuda()).view(torch.int16).cpu()
    t = torch.arange(N // 16).view(-1, 1, 1, 1)
    c = torch.arange(K // 32).view(1, -1, 1, 1)
    lane = torch.arange(64).view(1, 1, -1, 1)
    e = torch.arange(8).view(1, 1, 1, -1)
    ref = w[(16 * t + lane % 16), (32 * c + 8 * (lane // 16) + e)]
    assert torch.equal(out.view(-1), ref.reshape(-1))


O_PROJ_CASES = [(1, 3584), (37, 3584), (128, 3584), (200, 3584), (256, 3584), (300, 3584),
                (256, 1536), (256, 4096), (256, 5120), (129, 5120)]


@pytest.mark.parametrize("M,D", O_PROJ_CASES)
def test_o_proj_residual(M, D):
    """The all-rows GEMM over one or two passes (<= 128 rows: one row group, <= 256:
    two, 300: 256 + 44) and the workloads' hidden sizes (1 to 4 K ranges)."""
    g = torch.Generator().manual_seed(M + D)
    K, N = D, D
    o, x, w = rnd(M, K, gen=g), rnd(M, N, gen=g), rnd(N, K, std=0.02, gen=g)
    hp = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ws = zeros_ws(_lib.o_proj_workspace_bytes(M, N, K))
    wp = packed(w)
    _lib.o_proj_residual(o, x, wp, M, K, N, hp, ws)
    mm = mm64(o, w)
    ref = (x.float().cpu() + mm.float()).to(torch.bfloat16)
    close_bf16(hp, ref, scale=ref.float().abs() + mm.float().abs(), atol=acc_bound(o, w))


@pytest.mark.parametrize("M,D", [(256, 3584), (37, 3584), (300, 4096), (256, 5120)])
def test_o_proj_post_norm(M, D):
    """hp as sf_o_proj_residual's (bit for bit), and zn[slot[r]] = bf16(w * bf16(hp[r]
    * rstd)) for the recomputed rows on the kernel's own hp; rows without a slot
    leave zn untouched."""
    g = torch.Generator().manual_seed(7 * M + D)
    o, x, w = rnd(M, D, gen=g), rnd(M, D, gen=g), rnd(D, D, std=0.02, gen=g)
    lnw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
    keep = torch.rand(M, generator=g) < 0.6
    slot = torch.full((M,), -1, dtype=torch.int32)
    slot[keep] = torch.arange(int(keep.sum()), dtype=torch.int32)
    slot = slot.cuda()
    R = int(keep.sum())
    ws = zeros_ws(_lib.o_proj_workspace_bytes(M, D, D))
    wp = packed(w)
    hp = torch.empty(M, D, dtype=torch.bfloat16, device="cuda")
    zn = torch.full((R + 1, D), 7.0, dtype=torch.bfloat16, device="cuda")
    for _ in range(2):  # twice through one workspace
        _lib.o_proj_post_norm(o, x, wp, M, D, D, slot, lnw, 1e-6, hp, zn, ws)
    hp1 = torch.empty_like(hp)
    _lib.o_proj_residual(o, x, wp, M, D, D, hp1, ws)
    torch.cuda.synchronize()
    assert torch.equal(hp, hp1)
    mm = mm64(o, w)
    ref = (x.float().cpu() + mm.float()).to(torch.bfloat16)
    close_bf16(hp, ref, scale=ref.float().abs() + mm.float().abs(), atol=acc_bound(o, w))
    h = hp[keep.cuda()].float()
    z_ref = lnw * (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    close_bf16(zn[:R], z_ref, scale=2 * z_ref.float().abs())
    assert torch.all(zn[R] == 7.0)


@pytest.mark.parametrize("M", [1, 100, 300])
def test_lm_head_rows(M):
    """One row group (<= 128 rows) and two passes (300 rows) of the head GEMM."""
    g = torch.Generator().manual_seed(M)
    D, V = 3584, 16384
    x, w = rnd(M, D, gen=g), rnd(V, D, std=0.02, gen=g)
    logits = torch.empty(M, V, dtype=torch.bfloat16, device="cuda")
    _lib.lm_head(x, M, packed(w), D, V, logits)
    close_bf16(logits, mm64(x, w), atol=acc_bound(x, w))


@pytest.mark.parametrize("B1,N,lo,n,shift", [
    (8, 32, 0, 16, True),      # the first small block and the next: a 128-row pass
    (8, 32, 8, 16, True),
    (8, 32, 24, 8, True),      # the last small block: 64 rows
    (8, 32, 4, 24, False),     # 192 rows: a 256-row pass, unshifted
    (5, 32, 0, 32, True),      # the whole block of 160 rows through the window path
    (8, 64, 16, 32, True),     # 256 rows of 64-row blocks
])
def test_head_logits_rows_window(B1, N, lo, n, shift):
    """sf_head_logits_rows: the window's rows equal the whole head's bit for bit
    (shifted or not), every other row and the padding columns stay untouched;
    V spans whole rounds of 256-column tiles plus a 128-column tail."""
    g = torch.Generator().manual_seed(B1 * 100 + lo + n)
    M, D, V = B1 * N, 1536, 256 * 256 + 384
    x, w = rnd(M, D, gen=g), rnd(V, D, std=0.02, gen=g)
    wp = packed(w)
    full = torch.full((M, V + 8), 7.0, dtype=torch.bfloat16, device="cuda")
    _lib.head_logits(x, M, wp, D, V, full, shift_n=N if shift else 0)
    win = torch.full((M, V + 8), 7.0, dtype=torch.bfloat16, device="cuda")
    _lib.head_logits_rows(x, M, wp, D, V, win, N, shift, lo, n)
    torch.cuda.synchronize()
    inside = torch.zeros(B1, N, dtype=torch.bool)
    inside[:, lo:lo + n] = True
    inside = inside.reshape(M).cuda()
    assert torch.equal(win[inside], full[inside])
    assert torch.all(win[~inside] == 7.0)
    assert torch.all(win[:, V:] == 7.0)
    # and the whole head against the float64 product (its shift: row n from n - 1),
    # on the first main-round columns and the tail tile's
    src = torch.arange(M, device="cuda")
    if shift:
        pos = src % N
        src = torch.where(pos > 0, src - 1, src)
    cols = torch.cat([torch.arange(0, 512), torch.arange(V - 384, V)]).cuda()
    close_bf16(full[:, cols], mm64(x[src], w[cols]), atol=acc_bound(x[src], w[cols]))


@pytest.mark.parametrize("count,D,I,bucket", [(1, 1536, 8960, 256), (39, 1536, 8960, 256),
                                               (117, 1536, 8960, 256), (130, 1536, 8960, 256),
                                               (256, 1536, 8960, 256), (39, 3584, 18944, 256),
                                               (117, 3584, 18944, 128), (300, 1536, 8960, 512),
                                               (64, 1536, 8960, 64)])
def test_ffn_path(count, D, I, bucket):
    """Row counts across the row blocks (64 / 128 / 256 rows per pass, and two
    passes beyond 256), the 1.5B and 7B FFN shapes."""
    g = torch.Generator().manual_seed(count + D)
    BN = max(256, bucket)
    hp = rnd(BN + 1, D, gen=g)
    perm = torch.randperm(BN, generator=g)[:count].sort().values
    rows = torch.full((bucket,), BN, dtype=torch.int32)
    rows[:count] = perm.to(torch.int32)
    rows, cnt = rows.cuda(), torch.tensor([count], dtype=torch.int32).cuda()
    lnw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
    wg, wu, wd = rnd(I, D, std=0.02, gen=g), rnd(I, D, std=0.02, gen=g), rnd(D, I, std=0.02, gen=g)
    zn = torch.zeros(bucket, D, dtype=torch.bfloat16, device="cuda")
    act = torch.zeros(bucket, I, dtype=torch.bfloat16, device="cuda")
    ffn = torch.zeros(BN + 1, D, dtype=torch.bfloat16, device="cuda")
    ws = zeros_ws(max(_lib.gemm_workspace_bytes(bucket, D, I),
                      _lib.gate_up_workspace_bytes(bucket, D, I)))
    _lib.rows_rmsnorm(hp, rows, cnt, bucket, lnw, D, 1e-6, zn)
    for _ in range(2):  # twice through one workspace
        _lib.ffn_gate_up(zn, cnt, bucket, packed(wg), packed(wu), D, I, act, ws)
        _lib.ffn_down_scatter(act, cnt, bucket, rows, packed(wd), I, D, ffn, ws)
    torch.cuda.synchronize()
    r = rows[:count].long()
    x = hp[r].float()
    z_ref = lnw * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    # two roundings (x*rstd, then *w): a flip of the inner one can show as 2 ulps
    close_bf16(zn[:count], z_ref, scale=2 * z_ref.float().abs())
    z = zn[:count]
    gt = mm64(z, wg)
    up = mm64(z, wu)
    act_ref = F.silu(gt) * up
    # x*sigmoid(x) has condition number |1 + x(1 - sigmoid(x))| <= 1 + |x|: a 1-ulp
    # change of the gate GEMM output moves act by up to (1 + |g|) ulps
    close_bf16(act[:count], act_ref, scale=act_ref.float().abs() * (2 + gt.float().abs()),
               atol=(acc_bound(z, wg) + acc_bound(z, wu)) * (1 + up.double().abs()))
    close_bf16(ffn[r], mm64(act[:count], wd), atol=acc_bound(act[:count], wd))
    untouched = torch.ones(BN + 1, dtype=torch.bool)
    untouched[r.cpu()] = False
    assert torch.all(ffn[untouched.cuda()] == 0)


def test_residual_gather_add_and_lm_head():
    g = torch.Generator().manual_seed(5)
    B1, N, D, V = 8, 32, 3584, 152064
    hp, ffn = rnd(B1 * N, D, gen=g), rnd(B1 * N + 1, D, gen=g)
    src = torch.randint(0, B1, (B1 * N,), generator=g, dtype=torch.int32).cuda()
    out = torch.empty(B1 * N, D, dtype=torch.bfloat16, device="cuda")
    _lib.residual_gather_add(hp, ffn, src, B1, N, D, out)
    n = torch.arange(N).repeat(B1).cuda()
    ref = hp + ffn[src.long() * N + n]
    assert torch.equal(out, ref)
    w = rnd(V, D, std=0.02, gen=g)
    logits = torch.empty(B1 * N, V, dtype=torch.bfloat16, device="cuda")
    _lib.lm_head(out, B1 * N, packed(w), D, V, logits)
    close_bf16(logits, mm64(out, w), atol=acc_bound(out, w))
