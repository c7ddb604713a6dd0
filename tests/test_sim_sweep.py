"""Seeded random sweeps of the kernels' own sources in the CPU SIMT simulator, over
shapes the fixed cases of test_sim_attention.py, test_sim_gemm.py and
test_sim_gate.py do not name: attention (prefix length, page size, branches,
block length, head grouping, recomputed rows, causal block), the GEMMs (D, I,
recomputed rows, bucket, static M), the gate with compaction (forests of up
to 32 branches, block lengths, widths, all three gate modes, buckets below, at
and above the recomputed count) and gate -> attention -> chain correction at
random prefix lengths and inputs.  Same checks as the fixed cases.

SF_SIM_SWEEP=<n> sets the number of attention and GEMM shapes (default 4 each;
the gate takes 8x as many cases); SF_SIM_SWEEP_SEED picks another sweep."""

import os
import random
import subprocess

import pytest
import torch

from specfold_amd import _lib
from specfold_amd.engine import build_parent_map
from tests.test_gpu_gate import check_outputs, ref_mask
from tests.test_sim_attention import attn_sim  # noqa: F401  (fixture)
import tests.test_sim_gate as sim_gate
from tests.test_sim_gate import run_gate, sim  # noqa: F401  (fixture)
from tests.test_sim_gemm import gemm_sim  # noqa: F401  (fixture)

COUNT = int(os.environ.get("SF_SIM_SWEEP", "4"))
SEED = int(os.environ.get("SF_SIM_SWEEP_SEED", "2026"))


def attn_cases():
    rng = random.Random(SEED)
    out = []
    for _ in range(COUNT):
        Hkv = rng.choice([1, 2, 4, 8])
        G = rng.randint(1, 8)
        B1 = rng.randint(1, 8)
        N = rng.choice([8, 16, 32])
        P = rng.choice([0, rng.randint(1, 200), rng.randint(1, 1500)])
        out.append((P, rng.choice([16, 32, 64, 128]), B1, N, G * Hkv, Hkv,
                    rng.randint(1, B1 * N), rng.randint(0, 1), rng.randint(1, 10**6)))
    return out


def gemm_cases():
    rng = random.Random(SEED + 1)
    out = []
    for _ in range(COUNT):
        bucket = rng.randint(1, 256)
        out.append((128 * rng.randint(1, 6), 128 * rng.randint(1, 8), rng.randint(1, bucket),
                    bucket, rng.randint(1, 256), rng.randint(1, 10**6)))
    return out


@pytest.mark.parametrize("case", attn_cases(), ids=lambda c: "P%d_ps%d_B%d_N%d_H%d-%d_R%d_c%d" % c[:8])
def test_attention_sweep(attn_sim, case):  # noqa: F811
    r = subprocess.run([str(attn_sim), *map(str, case)], capture_output=True, text=True,
                       timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.parametrize("case", gemm_cases(), ids=lambda c: "D%d_I%d_count%d_bucket%d_M%d" % c[:5])
def test_gemm_sweep(gemm_sim, case):  # noqa: F811
    r = subprocess.run([str(gemm_sim), *map(str, case)], capture_output=True, text=True,
                       timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr


def test_gate_sweep(sim):  # noqa: F811
    rng = random.Random(SEED + 2)
    for _ in range(8 * COUNT):
        seed = rng.randint(0, 10**9)
        gen = torch.Generator().manual_seed(seed)
        B1 = rng.randint(1, 32)
        N = min(rng.choice([4, 8, 16, 32]), 1024 // B1)
        main = torch.randint(0, 5, (N,), generator=gen)
        toks = main.repeat(B1, 1)
        p = rng.choice([0.05, 0.15, 0.4])
        for i in range(1, B1):
            m = torch.rand(N, generator=gen) < p
            toks[i][m] = torch.randint(5, 9, (int(m.sum()),), generator=gen)
        parents = build_parent_map(toks)[0]
        D = 8 * rng.randint(1, 96)
        hidden = torch.zeros(B1, N, D)
        hidden[0] = torch.randn(N, D, generator=gen)
        for i in range(1, B1):
            hidden[i] = hidden[parents[i]] + 0.2 * torch.rand(N, 1, generator=gen) * \
                torch.randn(N, D, generator=gen)
        hidden = hidden.to(torch.bfloat16)
        ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).to(torch.bfloat16)
        delta = rng.random() * 0.2
        mode = rng.choice([_lib.SF_GATE_MODEL_DTYPE, _lib.SF_GATE_FP32_SQUARED, _lib.SF_GATE_ALL])
        rec = ref_mask(hidden, parents, delta, mode)
        nrec = int(rec.sum())
        bucket = rng.choice([None, max(1, nrec - rng.randint(0, 3)),
                             min(B1 * N, nrec + rng.randint(0, 40))])
        out = run_gate(sim, hidden, parents, ln_w, delta, mode, bucket=bucket)
        try:
            check_outputs(out, hidden, parents, rec, ln_w, bucket=bucket)
        except AssertionError as e:
            raise AssertionError(f"seed={seed} B1={B1} N={N} D={D} mode={mode} "
                                 f"delta={delta} bucket={bucket}: {e}") from None


def chain_cases():
    rng = random.Random(SEED + 3)
    return [(rng.randint(0, 600), rng.randint(10, 10**6)) for _ in range(max(1, COUNT // 2))]


@pytest.mark.parametrize("P,seed", chain_cases())
def test_chain_sweep(sim, P, seed):  # noqa: F811
    sim_gate.test_gate_attention_chain(sim, P, seed)
