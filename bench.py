"""Benchmark of SpecFold's folded verify step on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload cfg3_7b] [--no-cpu-baseline]

Workload (default ``cfg3_7b``): Fast-dLLM-v2-7B shape (hidden 3584, 28/4 heads,
hd 128, 28 layers, SwiGLU 18944, vocab 152064), bf16, random-init weights
(seed 2), a 2048-token random prompt prefilled block by block into the paged
KV cache, B=7 drafts from the fixed synthetic draft graph (depth 4 <= D=8,
<= S=3 per level), block 32, small block 8, delta 0.1, threshold 0.9, greedy.

A step is one iteration of the decode loop (generate_with_draft_speculation):
one folded verify step of the 8 branches over the prefix (or a block commit
/ a draft-cache hit), then sampling, drafting and unmasking.  W untimed steps,
then exactly K timed steps between two torch.cuda.synchronize() calls.
``value`` = tokens committed during the K steps / their wall time.

Also reported (same run): the verify step alone (hipEvent median), every HIP
kernel's average duration from HIP events around back-to-back launches on
the launch stream with its algorithmic bytes/flops and roofline fraction
(MI355X peaks: HBM 8 TB/s, dense bf16 MFMA 2.5 PFLOP/s), and the CPU baseline:
the oracle (CPU restatement of the reference PyTorch step) in fp32 on the
host cores, one layer timed and scaled to all layers plus the lm_head.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def parse_args(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--workload", default="cfg3_7b")
    ap.add_argument("--verify-iters", type=int, default=50)
    ap.add_argument("--kernel-iters", type=int, default=200)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-mode-b", dest="mode_b", action="store_false",
                    help="skip the verify step at a fold ratio near 0.62 (synthetic layer "
                         "inputs; reported under 'mode_b', measured by default)")
    ap.add_argument("--lockstep", action="store_true",
                    help="a multi-sequence workload (cfg4) decodes its sequences in lockstep, "
                         "one batched verify step per round (a step = one round)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also time a plain 256 MiB device copy (counter calibration)")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="for rocprofv3 --pmc runs: the model, a prefix cache of random K/V "
                         "(no prefill, no decode loop, no graphs), one eager verify step, a 2 s "
                         "pause, the copy calibration, then every entry point launched once per "
                         "layer in PMC_ORDER (no JSON line)")
    ap.add_argument("--traffic-table", nargs="+", metavar="CSV",
                    help="on the host: build profiles/traffic_<workload>.json from the "
                         "counter_collection.csv files of --pmc-pass runs (FETCH_SIZE, "
                         "WRITE_SIZE, optionally the MFMA counters)")
    return ap.parse_args(argv)


def event_time_ms(fns, iters: int) -> float:
    """Average ms per call on the GPU: ``iters`` back-to-back launches (cycling
    through ``fns``, e.g. one launcher per layer, so each launch streams another
    layer's weights as the verify step does) captured in one HIP graph and
    replayed between two HIP events recorded on the stream the kernels run on
    (no host launch overhead between kernels)."""
    fns = fns if isinstance(fns, (list, tuple)) else [fns]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for fn in fns:
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(iters):
            fns[i % len(fns)]()
    graph.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    graph.replay()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / iters


def kernel_roofline(name, ms, w, R, B1, N, P):
    """Algorithmic bytes / flops per launch of each kernel at the measured R."""
    sh = w.shape
    D, H, Hkv, hd, e = sh.hidden, sh.heads, sh.kv_heads, sh.head_dim, 2
    BN = B1 * N
    nq = (H + 2 * Hkv) * hd
    if name == "gate":
        # fused residual gate: hp rows + the R distinct ffn rows in, h rows + R xn rows out
        by = 2 * BN * D * e + 2 * R * D * e + BN * 21 + R * 4
        fl = 7 * BN * D
    elif name == "qkv":
        bias = nq * e if sh.qkv_bias else 0
        by = nq * D * e + bias + R * D * e + R * nq * e + 2 * N * hd * e
        fl = 2 * R * D * nq
    elif name == "attn":
        # prefix K/V once, the block K/V rows, the recomputed rows' q; O (fp32 + bf16)
        # and (m, Z) of every row (folded rows included)
        by = (2 * Hkv * P * hd * e + BN * 2 * Hkv * hd * e + R * H * hd * e
              + BN * H * hd * (4 + e) + 8 * BN * H)
        fl = 4 * R * H * P * hd + 4 * BN * H * N * hd
    elif name == "append":
        by = 2 * (2 * N * Hkv * hd * e)
        fl = 0
    elif name == "o_proj":
        # o_proj of every row fused with the residual (x in, hp out) and the
        # post-attention RMSNorm of the R recomputed rows (zn out, norm weight)
        by = D * H * hd * e + BN * H * hd * e + 2 * BN * D * e + R * D * e + D * e
        fl = 2 * BN * H * hd * D + BN * D + 4 * R * D
    elif name == "gate_up":
        I = sh.intermediate
        by = 2 * I * D * e + R * D * e + R * I * e
        fl = 4 * R * D * I
    elif name == "down":
        I = sh.intermediate
        by = D * I * e + R * I * e + R * D * e
        fl = 2 * R * I * D
    elif name == "final_norm":
        by = 3 * BN * D * e + R * D * e + D * e
        fl = 5 * BN * D
    elif name == "lm_head":
        V = sh.vocab
        by = V * D * e + BN * D * e + BN * V * e
        fl = 2 * BN * D * V
    else:
        raise KeyError(name)
    s = ms * 1e-3
    t_hbm = by / (HBM_PEAK_GBS * 1e9)
    t_mfma = fl / (BF16_PEAK_TFLOPS * 1e12)
    bound = "mfma" if t_mfma > t_hbm else "hbm"
    if bound == "hbm":
        ach, peak, unit = by / s / 1e9, HBM_PEAK_GBS, "GB/s"
    else:
        ach, peak, unit = fl / s / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s"
    return {"bound": bound, "achieved": round(ach, 3), "peak": peak, "unit": unit,
            "frac": round(ach / peak, 5), "traffic": None, "avg_us": round(ms * 1e3, 3),
            "algorithmic_bytes": int(by), "algorithmic_flops": int(fl),
            "hbm_gbps": round(by / s / 1e9, 2), "mfma_tflops": round(fl / s / 1e12, 3)}


def roofline_entry(k: dict, name: str) -> dict:
    """The bench line's roofline object for the dominant kernel: achieved and frac
    from its average duration inside the verify step, the isolated
    (back-to-back launches) figures kept beside."""
    r = dict(k, kernel=name)
    if "in_step_us" in k:
        r.update(achieved=k["in_step_achieved"], frac=k["in_step_frac"],
                 isolated_achieved=k["achieved"], isolated_frac=k["frac"],
                 isolated_us=k["avg_us"], avg_us=k["in_step_us"],
                 timing="HIP events around the kernel's launches inside an eager verify step")
    return r


# kernels launched once per verify step (the others once per layer)
ONCE_PER_STEP = ("lm_head", "final_norm")


# --pmc-pass launch order and the kernels each entry point runs (name prefixes, after
# stripping "void " and the anonymous namespace), for the verify step's shape
PMC_ORDER = ("qkv", "attn", "o_proj", "gate_up", "down", "final_norm", "lm_head", "gate")
PMC_KERNELS = {
    "qkv": ("sfg::gemm_sk_kernel<1, 0,", "sf_qkv_epilogue_kernel"),
    "attn": ("sf_attn_prefix_kernel", "sf_attn_rows_kernel"),
    "o_proj": ("sfg::gemm_rows_kernel<", "part_residual_norm_kernel"),
    # the SiLU fix-up only follows a stream-K gate/up (narrow intermediates); "?" marks
    # a kernel taken when it is the next dispatch
    "gate_up": ("sfg::gemm_sk_kernel<2, 2,", "?silu_fixup_kernel"),
    "down": ("sfg::gemm_sk_kernel<1, 1,", "down_fixup_kernel"),
    "final_norm": ("sf_gate_rows_kernel",),
    # the head: the whole rounds' 256-column kernel, then (where V leaves a partial
    # round) the 128-column one
    "lm_head": ("head_kernel<8, 1,", "?head_kernel<8, 2,"),
    # the compaction runs in the gated QKV GEMM unless the engine's gated_qkv is off
    "gate": ("sf_gate_rows_kernel", "?sf_gate_compact_kernel"),
}


def _kernel_short(name: str) -> str:
    return name.replace("void ", "").replace("(anonymous namespace)::", "")


def traffic_table(csvs, workload: str) -> dict:
    """Per entry point HBM bytes per launch from --pmc-pass runs: the dispatches after
    the pass's pause are walked in PMC_ORDER (qkv, attn, ... once per layer, the
    once-per-step ones once), FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are summed
    over each launch's kernels and scaled by what the same counters read for the
    plain copy of known size launched first in the pause (y = 2x, 256 MiB fp32).  MFMA
    counters, when collected, give each launch's MFMA busy fraction."""
    import csv as _csv
    from specfold_amd.configs import workload as get_workload

    w = get_workload(workload)
    L = w.shape.layers
    per = {}   # counter -> ordered list of (kernel, value) after the pause
    for path in csvs:
        rows = list(_csv.DictReader(open(path)))
        by_disp = {}
        for r in rows:
            d = by_disp.setdefault(int(r["Dispatch_Id"]), {"name": _kernel_short(r["Kernel_Name"]),
                                                           "t0": int(r["Start_Timestamp"]),
                                                           "grid": int(r["Grid_Size"])})
            if r.get("End_Timestamp"):
                d["DURATION_NS"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        seq = [by_disp[k] for k in sorted(by_disp)]
        # the pause: the largest start-time gap before a torch elementwise dispatch
        # (the calibration copy that opens the counted section)
        gaps = [(seq[i + 1]["t0"] - seq[i]["t0"], i + 1) for i in range(len(seq) - 1)
                if "elementwise_kernel" in seq[i + 1]["name"]]
        start = max(gaps)[1]
        for d in seq[start:]:
            for c, v in d.items():
                if c not in ("name", "t0", "grid") and (c != "DURATION_NS" or c not in per
                                                         or path == csvs[0]):
                    per.setdefault(c, []).append((d["name"], v, d["grid"]))
    out = {"workload": workload, "kernels": {}}
    for counter, seq in per.items():
        # calibration copy first (the largest elementwise dispatch), then PMC_ORDER
        cal = seq[0]
        i = 1
        table = {}
        for name in PMC_ORDER:
            launches = 1 if name in ONCE_PER_STEP else L
            pats = PMC_KERNELS[name]
            vals = []
            for _ in range(launches):
                tot = 0.0
                for pat in pats:
                    if isinstance(pat, str) and pat.startswith("?"):
                        if i < len(seq) and seq[i][0].startswith(pat[1:]):
                            tot += seq[i][1]
                            i += 1
                        continue
                    while i < len(seq) and not seq[i][0].startswith(pat):   # str or tuple
                        i += 1   # kernels of other libraries between ours (e.g. torch copies)
                    if i >= len(seq):
                        raise ValueError(f"{counter}: ran out of dispatches at {name}/{pat}")
                    tot += seq[i][1]
                    i += 1
                vals.append(tot)
            table[name] = sum(vals) / len(vals)
        out.setdefault("raw", {})[counter] = {"calibration": cal[1], **table}
    cal_bytes = 256 << 20
    f = out["raw"].get("FETCH_SIZE")
    wr = out["raw"].get("WRITE_SIZE")
    if f and wr:
        ff = cal_bytes / (f["calibration"] * 1024)
        wf = cal_bytes / (wr["calibration"] * 1024)
        out["calibration"] = {"kernel": "vectorized_elementwise_kernel fp32 y=2x, 256 MiB",
                              "fetch_factor": round(ff, 4), "write_factor": round(wf, 4)}
        for name in PMC_ORDER:
            b = f[name] * 1024 * ff + wr[name] * 1024 * wf
            out["kernels"][name] = {"fetch_kib_raw": round(f[name], 1),
                                    "write_kib_raw": round(wr[name], 1),
                                    "bytes_per_launch": int(b)}
    dur = out["raw"].get("DURATION_NS")
    if dur:
        for name in PMC_ORDER:
            out["kernels"].setdefault(name, {})["pmc_run_us"] = round(dur[name] / 1e3, 3)
    mb = out["raw"].get("SQ_VALU_MFMA_BUSY_CYCLES")
    ga = out["raw"].get("GRBM_GUI_ACTIVE")
    if mb:
        # MFMA busy fraction of all 256 CUs x 4 SIMDs over the launch's own duration
        # at the 2.4 GHz peak engine clock.  GRBM_GUI_ACTIVE is not the denominator:
        # on this part it reads the sum over the 8 XCDs plus the profiler's time around
        # each dispatch (gui_active_per_us, 17k-42k per us against 2.4k per clock)
        simds = 256 * 4
        for name in PMC_ORDER:
            k = out["kernels"].setdefault(name, {})
            if dur and dur[name]:
                k["mfma_busy"] = round(mb[name] / (simds * dur[name] * 2.4), 4)
                if ga:
                    k["gui_active_per_us"] = round(ga[name] / (dur[name] / 1e3), 1)
    mo = out["raw"].get("SQ_INSTS_VALU_MFMA_MOPS_BF16")
    if mo:
        # MOPS counts 512 flops per unit: the MFMA work issued (row tiles padded to 16
        # or to the GEMM's row block), and its rate over the launch's duration
        for name in PMC_ORDER:
            k = out["kernels"].setdefault(name, {})
            k["mfma_bf16_flops"] = int(mo[name] * 512)
            if dur and dur[name]:
                k["mfma_tflops_issued"] = round(mo[name] * 512 / dur[name] / 1e3, 2)
    return out


def load_traffic(workload: str) -> dict:
    """HBM bytes per launch measured by rocprofv3 PMC runs (FETCH_SIZE and
    WRITE_SIZE, scaled by the plain-copy calibration), committed as JSON under
    profiles/; empty when absent."""
    path = ROOT / "profiles" / f"traffic_{workload}.json"
    if not path.exists():
        return {}
    data = json.loads(path.read_text())
    return {k: v.get("bytes_per_launch") for k, v in data.get("kernels", {}).items()}


def copy_calibration(mib: int = 256, reps: int = 8) -> dict:
    """A plain device copy of known size through an ordinary vectorized
    elementwise kernel (y = 2x in fp32): the reference point for the
    FETCH_SIZE / WRITE_SIZE counters, and the copy bandwidth this GPU reaches."""
    n = (mib << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.mul(src, 2.0, out=dst)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        torch.mul(src, 2.0, out=dst)
    e.record()
    e.synchronize()
    us = s.elapsed_time(e) / reps * 1e3
    nbytes = n * 4
    return {"kernel": "vectorized_elementwise_kernel (fp32 y = 2x)", "bytes_read": nbytes,
            "bytes_written": nbytes, "avg_us": round(us, 2), "gbps": round(2 * nbytes / us / 1e3, 1)}


def host_cores() -> dict:
    """The host cores this process may use: the affinity set, capped by a cgroup
    CPU quota when one is set, and the CPU model (lscpu's "Model name", read from
    /proc/cpuinfo)."""
    aff = len(os.sched_getaffinity(0))
    quota = None
    try:
        q, per = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            quota = max(1, int(int(q) / int(per)))
    except (OSError, ValueError):
        pass
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"threads": min(aff, quota) if quota else aff, "affinity": aff, "cgroup_quota": quota,
            "model": model}


def cpu_baseline(w, gen, batched, gpu_counts, tokens_per_step, seconds):
    """The oracle (oracle/folded_reference.py: the CPU restatement of the
    reference's PyTorch folded verify step) on the host cores, replaying the GPU
    step's own work: layer 0 of the GPU model (its bf16 weights copied to the
    host: the reference's model dtype), the step's own batched tokens and their
    embedding, and the cache's layer-0 prefix, so the CPU gate recomputes the
    rows the GPU step recomputed at layer 0 (both counts are reported).  One
    layer is timed and scaled by the layer count, plus the lm_head timed on a
    vocabulary slice and scaled ("extrapolated": true)."""
    import copy

    from oracle.folded_reference import FoldCounters, folded_layer, parent_map, topo_order

    host = host_cores()
    torch.set_num_threads(host["threads"])
    eng = gen._engine
    cache = gen._state["cache"]
    P = cache.length
    B1, N = batched.shape
    sh = w.shape
    toks = batched.cpu()
    parent, counts = parent_map(toks)
    order = topo_order(counts)
    h0 = eng.base.embed_tokens(batched).to("cpu")
    h = [h0[i:i + 1] for i in range(B1)]
    lyr = copy.deepcopy(eng.layers[0]).to("cpu")
    kv = tuple(t.to("cpu") for t in cache[0])
    cos, sin = eng.rope_tables(P + N)
    cos, sin = cos[P:P + N].to("cpu"), sin[P:P + N].to("cpu")
    q_scale = None
    qfn = getattr(gen.model_executor, "q_scale", None)
    if qfn is not None:
        qs = qfn(P, N)
        q_scale = None if qs is None else qs.to("cpu")
    cnt = FoldCounters()

    def one(counters=None):
        folded_layer(lyr, h, parent, order, kv, cos, sin, w.delta, sh.heads, sh.kv_heads,
                     counters=counters, q_scale=q_scale)

    with torch.no_grad():
        one(cnt)
        r_cpu = N + cnt.draft_recomputed          # branch 0 always, plus the recomputed drafts
        times = []
        t_end = time.perf_counter() + seconds
        while len(times) < 2 or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            one()
            times.append(time.perf_counter() - t0)
        t_layer = statistics.median(times)
        vs = 8192
        x = torch.randn(B1 * N, sh.hidden, dtype=torch.bfloat16)
        wh = eng.head.weight[:vs].to("cpu")
        x @ wh.t()
        t0 = time.perf_counter()
        for _ in range(3):
            x @ wh.t()
        t_head = (time.perf_counter() - t0) / 3 * (sh.vocab / vs)
    t_step = t_layer * sh.layers + t_head
    return {"value": round(tokens_per_step / t_step, 5), "unit": "tokens/s",
            "cores": host["threads"], "kind": "port", "extrapolated": True,
            "cpu_model": host["model"], "affinity_cores": host["affinity"],
            "cgroup_quota_cores": host["cgroup_quota"], "dtype": str(h0.dtype).replace("torch.", ""),
            "recomputed_rows_layer0": {"cpu": r_cpu, "gpu": int(gpu_counts[0])},
            "sample": (f"the oracle on the GPU step's own layer-0 input (tokens, embedding, "
                       f"weights, {P}-key prefix): 1 of {sh.layers} layers timed ({len(times)} "
                       f"runs, median {t_layer:.3f}s) x{sh.layers} + lm_head ({t_head:.3f}s, "
                       f"timed on a {vs}-row vocab slice and scaled); {tokens_per_step:.3f} "
                       f"tokens/step from the GPU decode loop"),
            "verify_step_s": round(t_step, 4)}


def kernel_table(w, eng, B1, N, kernel_iters):
    """Every entry point's average duration (HIP events around a graph of
    back-to-back launches on the buffers of the engine's last verify step, one
    launcher per layer in turn) with its algorithmic bytes / flops at that step's
    recomputed-row count; returns (kernels, prefix, rows)."""
    shared = {}
    per_layer = [eng.profile_launchers(li=li, shared=shared) for li in range(eng.L)]
    info = per_layer[-1][1]
    P = info["prefix"]
    R = int(info["count"].item())
    kernels = {}
    for name in ("qkv", "attn", "o_proj", "gate_up", "down", "final_norm", "lm_head", "append",
                 "gate"):
        if name not in per_layer[-1][0]:
            continue
        once = name in ONCE_PER_STEP
        fns = [per_layer[-1][0][name]] if once else [pl[0][name] for pl in per_layer]
        ms = event_time_ms(fns, kernel_iters if not once else max(4, kernel_iters // 10))
        kernels[name] = kernel_roofline(name, ms, w, R, B1, N, P)
        kernels[name]["launches_per_step"] = 1 if once else eng.L
    return kernels, P, R


# The engine's calls into the library per entry point of the kernel table (the
# entry points launched by FoldedVerifyEngine._run_layers and its head).
IN_STEP_CALLS = {"gate": ("fold_gate_residual",), "qkv": ("qkv_rope", "qkv_rope_gated"),
                 "attn": ("attn_rows",), "o_proj": ("o_proj_post_norm",),
                 "gate_up": ("ffn_gate_up",), "down": ("ffn_down_scatter",),
                 "final_norm": ("residual_rmsnorm",), "lm_head": ("head_logits",)}


def in_step_times(run_step, reps: int = 3) -> dict:
    """Each entry point's average GPU time inside the verify step itself, next to
    the kernels it runs between in the step: the step runs eagerly with HIP events
    recorded on the launch stream right before and after every library call the
    engine makes (its _lib functions wrapped for the duration), behind a GPU sleep
    long enough that the host has queued the whole step before the GPU reaches it
    (so the events bracket the kernels, not host launch gaps); the median time of
    an empty event pair queued the same way is subtracted.  Returns {name:
    {"in_step_us": mean - pair, "in_step_us_raw": mean, "launches": n}}."""
    from specfold_amd import _lib
    spans = {k: [] for k in IN_STEP_CALLS}
    saved = {}
    for name, fns in IN_STEP_CALLS.items():
        for fn in fns:
            orig = getattr(_lib, fn)
            saved[fn] = orig

            def wrapped(*a, _orig=orig, _name=name, **k):
                s = torch.cuda.Event(enable_timing=True)
                e = torch.cuda.Event(enable_timing=True)
                s.record()
                _orig(*a, **k)
                e.record()
                spans[_name].append((s, e))
            setattr(_lib, fn, wrapped)
    empty = []
    try:
        for _ in range(reps):
            torch.cuda._sleep(200_000_000)      # ~0.1 s of GPU spin: the host runs ahead
            run_step()
            # the cost of an event pair itself, queued the same way: subtracted below
            for _ in range(32):
                s = torch.cuda.Event(enable_timing=True)
                e = torch.cuda.Event(enable_timing=True)
                s.record()
                e.record()
                empty.append((s, e))
        torch.cuda.synchronize()
    finally:
        for fn, orig in saved.items():
            setattr(_lib, fn, orig)
    pair_us = statistics.median(s.elapsed_time(e) * 1e3 for s, e in empty)
    out = {"_event_pair_us": round(pair_us, 3)}
    for name, ev in spans.items():
        if ev:
            us = [s.elapsed_time(e) * 1e3 for s, e in ev]
            out[name] = {"in_step_us": round(statistics.mean(us) - pair_us, 3),
                         "in_step_us_raw": round(statistics.mean(us), 3), "launches": len(us)}
    return out


def with_in_step(kernels: dict, steps: dict, w, R, B1, N, P) -> None:
    """Adds each kernel's in-step time and the roofline it gives beside the
    isolated (back-to-back launch) figures of the table."""
    for name, k in kernels.items():
        st = steps.get(name)
        if not st:
            continue
        rl = kernel_roofline(name, st["in_step_us"] / 1e3, w, R, B1, N, P)
        k["in_step_us"] = st["in_step_us"]
        k["in_step_us_raw"] = st["in_step_us_raw"]
        k["in_step_frac"] = rl["frac"]
        k["in_step_achieved"] = rl["achieved"]


def mode_b(w, gen, batched, iters, kernel_iters):
    """The verify step at the reference's fold regime: every layer's input is
    replaced by synthetic hidden states in which branch i = its parent's +
    sigma * N(0, 1) per position, sigma 0.2 on a seeded 38% of positions and 0.05
    elsewhere (relative L2 ~ sigma, so at delta 0.1 about 38% of the draft
    positions are recomputed: fold ratio ~0.62, the reference's end-to-end figure,
    README.md:55-59).  The step runs eagerly (a replaced layer input leaves the
    captured graph); its per-kernel table is measured like the main one."""
    from specfold_amd.engine import StepStats, build_parent_map
    from specfold_amd.synthetic import perturbed_hidden
    eng = gen._engine
    cache = gen._state["cache"]
    B1, N = batched.shape
    parents, _ = build_parent_map(batched)
    g = torch.Generator().manual_seed(w.seed + 1000)
    teacher = {li: perturbed_hidden(parents, N, w.shape.hidden, g).to(eng.device)
               for li in range(eng.L)}
    qfn = getattr(gen.model_executor, "q_scale", None)
    qs = qfn(cache.length, N) if qfn is not None else None
    st = StepStats()
    lat = []
    for i in range(iters + 2):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        eng.forward(batched, cache, w.delta, teacher=teacher, stats=st, q_scale=qs)
        e.record()
        e.synchronize()
        if i >= 2:
            lat.append(s.elapsed_time(e))
    counts = st.counts
    R = sum(counts) / len(counts)
    kernels, P, R_last = kernel_table(w, eng, B1, N, kernel_iters)
    steps = in_step_times(lambda: eng.forward(batched, cache, w.delta, teacher=teacher,
                                              q_scale=qs))
    with_in_step(kernels, steps, w, R_last, B1, N, P)
    fold = 1 - (sum(counts) - len(counts) * N) / ((B1 - 1) * N * len(counts))
    dominant = max((n for n in kernels if n != "append"),
                   key=lambda n: kernels[n].get("in_step_us", kernels[n]["avg_us"])
                   * kernels[n]["launches_per_step"])
    return {"verify_step_ms_eager": round(statistics.median(lat), 4),
            "recomputed_rows_mean": round(R, 2), "recomputed_rows_last_layer": R_last,
            "fold_ratio": round(fold, 4), "prefix": P,
            "roofline": roofline_entry(kernels[dominant], dominant), "kernels": kernels,
            "data": "synthetic layer inputs (branch = parent + sigma N(0,1)), every layer"}


@torch.no_grad()
def pmc_pass(w) -> int:
    """The program counted by rocprofv3 --pmc runs.  Few dispatches and no graph
    replays: the workload's model and engine, the sequence's paged cache filled
    with N(0, 1) K/V at the workload's prefix (no prefill), one eager verify step
    of the draft tree (so the engine's buffers hold a real step: rows, counts,
    src), then, after a 2 s pause (the parser finds it by the gap), one plain copy
    of known size and every entry point once per layer in PMC_ORDER on the buffers
    of that step."""
    from specfold_amd.synthetic import draft_tree_block, TREE_DIFFS
    gens, _ = make_decoders(w)
    gen = gens[0]
    ex = gen.model_executor
    cache = ex.new_cache()
    g = torch.Generator(device="cuda").manual_seed(w.seed)
    shp = (1, cache.Hkv, w.prefix, cache.hd)
    kv = [(torch.randn(shp, generator=g, device="cuda").to(torch.bfloat16),
           torch.randn(shp, generator=g, device="cuda").to(torch.bfloat16))
          for _ in range(cache.num_layers)]
    cache.load_dense(kv)
    del kv
    gen._pack_layer_weights()
    eng = gen._engine
    eng.use_graphs = False
    tokens = draft_tree_block(w.block, w.shape.vocab, torch.Generator().manual_seed(w.seed),
                              diffs=TREE_DIFFS[:w.branches]).to("cuda")
    gen._batched_block_forward(tokens, cache)
    counts = gen.last_stats.counts
    R = round(sum(counts) / len(counts))
    n = (256 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    shared = {}
    per_layer = [eng.profile_launchers(li=li, shared=shared) for li in range(eng.L)]
    torch.cuda.synchronize()
    time.sleep(2.0)
    torch.mul(src, 2.0, out=dst)
    for name in PMC_ORDER:
        if name in ONCE_PER_STEP:
            per_layer[-1][0][name]()
        else:
            for pl in per_layer:
                pl[0][name]()
    torch.cuda.synchronize()
    print(f"[bench] pmc pass done ({w.name}, P {cache.length}, R {R})", file=sys.stderr,
          flush=True)
    return 0



def make_decoders(w):
    """One generator per sequence of the workload (sharing one executor, so the
    weights and packed weights exist once) and each sequence's random prompt."""
    from specfold_amd.configs import draft_graph
    max_len = w.prefix + w.gen_tokens
    page_order = "shuffled" if w.shuffled_pages else "sequential"
    graph = draft_graph(w.budget_B)
    if w.family == "fastdllm":
        from specfold_amd.generate import FastDLLMModelExecutor, SpecFoldHIPFastDLLMV2Generation
        if w.batch != 1:
            raise ValueError("the Fast-dLLM v2 generator decodes one sequence")
        ex = FastDLLMModelExecutor.synthetic(
            w.shape, w.seed, device="cuda", block_length=w.block, max_length=max_len + 4 * w.block,
            page_size=w.page_size, page_order=page_order, page_seed=w.seed)
        gens = [SpecFoldHIPFastDLLMV2Generation(
            block_length=w.block, model_executor=ex, calibration_graph=graph,
            threshold=w.threshold, small_block_size=w.small_block, max_new_tokens=w.gen_tokens,
            max_length=max_len, delta=w.delta)]
    else:
        from specfold_amd.generate import NLDModelExecutor, SpecFoldHIPNLDGeneration
        ex = NLDModelExecutor.synthetic(
            w.shape, w.seed, device="cuda", block_length=w.block, max_length=max_len + 4 * w.block,
            page_size=w.page_size, page_order=page_order, page_seed=w.seed)
        gens = [SpecFoldHIPNLDGeneration(
            block_length=w.block, model_executor=ex, calibration_graph=graph,
            threshold=w.threshold, max_new_tokens=w.gen_tokens, max_length=max_len,
            delta=w.delta) for _ in range(w.batch)]
    g = torch.Generator().manual_seed(w.seed)
    prompts = [torch.randint(0, w.shape.vocab - 1, (1, w.prefix), generator=g)
               for _ in range(len(gens))]
    return gens, prompts


@torch.no_grad()
def main(argv=None) -> int:
    args = parse_args(argv)
    if args.traffic_table:
        import subprocess
        tab = traffic_table(args.traffic_table, args.workload)
        try:
            tab["commit"] = subprocess.run(["git", "rev-parse", "--short=12", "HEAD"], cwd=ROOT,
                                           capture_output=True, text=True).stdout.strip() or None
        except OSError:
            tab["commit"] = None
        tab["sources"] = [str(Path(c)) for c in args.traffic_table]
        path = ROOT / "profiles" / f"traffic_{args.workload}.json"
        path.write_text(json.dumps(tab, indent=1) + "\n")
        print(f"wrote {path.relative_to(ROOT)}")
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the verify step is a single-GPU path in this build "
              "(multi-GPU sharding is design-only); run with --gpus 1", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    from specfold_amd.configs import workload

    torch.cuda.set_device(0)
    w = workload(args.workload)
    if args.pmc_pass:
        return pmc_pass(w)
    t_build = time.time()
    gens, prompts = make_decoders(w)
    torch.cuda.synchronize()
    build_s = time.time() - t_build
    print(f"[bench] model + engine ready in {build_s:.1f}s ({w.family}, {len(gens)} sequence(s))",
          file=sys.stderr, flush=True)

    # decode loops (one per sequence, stepped round-robin; or, with --lockstep, all
    # sequences per round with their verify steps batched): prefill, W warmup
    # steps, K timed steps
    lockstep = args.lockstep and len(gens) > 1
    if args.lockstep and not lockstep:
        print("--lockstep needs a multi-sequence workload", file=sys.stderr)
        return 2
    t0 = time.time()
    if lockstep:
        from specfold_amd.generate.lockstep import LockstepDecoder
        dec = LockstepDecoder(gens)
        rounds = dec.rounds(prompts)
        first = next(rounds)      # every sequence's prefill, then the first batched step
        assert [e["kind"] for _, e in first["events"]] == ["prefill"] * len(gens)

        def advance(i):
            try:
                r = next(rounds)
            except StopIteration:
                raise SystemExit("the decode loops ended before the timed steps did: "
                                 "lower --steps / --warmup") from None
            return r["committed"], [e["kind"] for _, e in r["events"]]
    else:
        loops = [g.decode_steps(p) for g, p in zip(gens, prompts)]
        for lp in loops:
            ev = next(lp)
            assert ev["kind"] == "prefill"

        def advance(i):
            ev = next(loops[i % len(loops)])
            return ev["committed"], [ev["kind"]]
    torch.cuda.synchronize()
    prefill_s = time.time() - t0
    print(f"[bench] prefill {len(gens)} x {w.prefix} tokens in {prefill_s:.2f}s", file=sys.stderr,
          flush=True)
    # start-up work of a serving engine: the verify step's graph for every branch
    # count the draft graph can produce, captured against each sequence's cache
    t0 = time.time()
    warmed = sum(g.warm_graphs() for g in gens if hasattr(g, "warm_graphs")) if not lockstep else 0
    torch.cuda.synchronize()
    warm_s = time.time() - t0
    if warmed:
        print(f"[bench] {warmed} verify-step graphs captured in {warm_s:.2f}s", file=sys.stderr,
              flush=True)
    for i in range(args.warmup):
        advance(i)
    kinds = {}
    committed = 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        c, ks = advance(i)
        committed += c
        for k in ks:
            kinds[k] = kinds.get(k, 0) + 1
    torch.cuda.synchronize()
    timed_s = time.perf_counter() - t0
    tps = committed / timed_s
    print(f"[bench] {args.steps} decode steps in {timed_s:.3f}s: {committed} tokens, {kinds}",
          file=sys.stderr, flush=True)

    # the verify step alone, on a B+1-branch draft batch of the last block at the
    # current prefix of sequence 0
    gen = gens[0]
    cache = gen._state["cache"]
    x_cur = gen._state["x_t"] if w.family == "fastdllm" else gen._state["x_accum"]
    from specfold_amd.synthetic import TREE_DIFFS
    diffs = TREE_DIFFS[:w.branches]
    gsel = torch.Generator().manual_seed(123)
    repl = torch.randint(0, w.shape.vocab - 1, (7,), generator=gsel).to(x_cur.device)

    def tree_batch(x):
        """The draft tree's B+1 branches over the last block of token state x."""
        b = x[:, -w.block:].repeat(len(diffs), 1)
        for i, d in enumerate(diffs):
            for k in d:
                b[i, k] = repl[k]
        return b

    batched = tree_batch(x_cur)
    lat = []
    for i in range(args.verify_iters + 3):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        gen._batched_block_forward(batched, cache)
        e.record()
        e.synchronize()
        if i >= 3:
            lat.append(s.elapsed_time(e))
    verify_ms = statistics.median(lat)
    counts = gen.last_stats.counts
    # the same step as the decode loop runs it: the head only on the rows the loop
    # reads (a small block and the next one: the generator's head_rows window)
    win_ms = None
    if hasattr(gen, "head_rows") and w.family == "fastdllm":
        sbs = gen.small_block_size
        gen.head_rows = (0, min(2 * sbs, w.block))
        lat_w = []
        try:
            for i in range(args.verify_iters + 3):
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                gen._batched_block_forward(batched, cache)
                e.record()
                e.synchronize()
                if i >= 3:
                    lat_w.append(s.elapsed_time(e))
        finally:
            gen.head_rows = None
        win_ms = statistics.median(lat_w)
        print(f"[bench] verify step with the decode window's head rows (2 small blocks) "
              f"median {win_ms:.3f} ms", file=sys.stderr, flush=True)
    R = round(sum(counts) / len(counts))
    B1, N = batched.shape
    fold_ratio_step = 1 - (sum(counts) - len(counts) * N) / ((B1 - 1) * N * len(counts))
    print(f"[bench] verify step median {verify_ms:.3f} ms, mean R {R}", file=sys.stderr,
          flush=True)
    batched_step = None
    if lockstep:
        # the batched verify step alone: every sequence's B+1-branch batch at its own
        # prefix, in one step (as a lockstep round runs it)
        reqs = [(tree_batch(g._state["x_t"] if w.family == "fastdllm" else g._state["x_accum"]),
                 g._state["cache"]) for g in gens]
        lat_b = []
        for i in range(args.verify_iters + 3):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            dec.forward_many(reqs)
            e.record()
            e.synchronize()
            if i >= 3:
                lat_b.append(s.elapsed_time(e))
        ms_b = statistics.median(lat_b)
        batched_step = {"ms": round(ms_b, 4), "sequences": len(reqs),
                        "branches_each": len(diffs), "pad_to": dec.pad_to,
                        "ms_per_sequence": round(ms_b / len(reqs), 4)}
        print(f"[bench] batched verify step ({len(reqs)} sequences) median {ms_b:.3f} ms",
              file=sys.stderr, flush=True)

    # per-kernel timings on the buffers of the last verify step, cycling through the
    # layers (weights and cache slices) as the step does
    eng = gen._engine
    kernels, P, R_last = kernel_table(w, eng, B1, N, args.kernel_iters)
    traffic = load_traffic(w.name)
    for name, k in kernels.items():
        k["traffic"] = traffic.get(name)
    # the same entry points inside the verify step (eager, events around each call)
    eng.use_graphs = False
    try:
        steps = in_step_times(lambda: gen._batched_block_forward(batched, cache))
    finally:
        eng.use_graphs = True
    with_in_step(kernels, steps, w, R_last, B1, N, P)
    print(f"[bench] kernels isolated {json.dumps({k: v['avg_us'] for k, v in kernels.items()})}"
          f"\n[bench] kernels in step "
          f"{json.dumps({k: v.get('in_step_us') for k, v in kernels.items()})}",
          file=sys.stderr, flush=True)
    # the dominant kernel: largest GPU time per verify step (in the step)
    dominant = max((n for n in kernels if n != "append"),
                   key=lambda n: kernels[n].get("in_step_us", kernels[n]["avg_us"])
                   * kernels[n]["launches_per_step"])
    copy = copy_calibration() if args.copy_calibration else None

    # tokens per sequence's decode step (a lockstep round steps every sequence)
    tokens_per_step = committed / max(1, args.steps * (len(gens) if lockstep else 1))
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(w, gen, batched, counts, tokens_per_step, args.cpu_seconds)
        print(f"[bench] cpu baseline {cpu}", file=sys.stderr, flush=True)

    mb = None
    if args.mode_b:
        mb = mode_b(w, gen, batched, max(3, args.verify_iters // 5), args.kernel_iters)
        print(f"[bench] mode B: R {mb['recomputed_rows_mean']}, kernels "
              f"{json.dumps({k: v['avg_us'] for k, v in mb['kernels'].items()})}",
              file=sys.stderr, flush=True)

    out = {
        "metric": "decode tokens/sec on 1 GPU; folded verify-step latency; attention HBM GB/s",
        "value": round(tps, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(timed_s / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": (f"synthetic (random-init weights, random-token prompt, synthetic draft graph; "
                 f"{w.batch} independent sequence(s) "
                 + ("decoded in lockstep, one batched verify step per round; a step = one "
                    "round)" if lockstep else "stepped round-robin)")),
        "config": {"workload": w.name, "hidden": w.shape.hidden, "layers": w.shape.layers,
                   "heads": w.shape.heads, "kv_heads": w.shape.kv_heads,
                   "intermediate": w.shape.intermediate, "vocab": w.shape.vocab,
                   "prefix": w.prefix, "branches": w.branches, "block": w.block,
                   "small_block": w.small_block if w.family == "fastdllm" else None,
                   "delta": w.delta, "threshold": w.threshold, "batch": w.batch,
                   "family": w.family, "shuffled_pages": w.shuffled_pages,
                   "lockstep": lockstep,
                   "parallelism": "none (1 GPU)"},
        "verify_step_ms": round(verify_ms, 4),
        "verify_step_ms_decode_window": None if win_ms is None else round(win_ms, 4),
        "verify_step_batched": batched_step,
        "verify_step_prefix": P,
        "verify_recomputed_rows_mean": R,
        "verify_fold_ratio": round(fold_ratio_step, 4),
        "decode_step_kinds": kinds,
        "tokens_per_step": round(tokens_per_step, 4),
        "prefill_s": round(prefill_s, 3),
        "graph_warmup": {"graphs": warmed, "s": round(warm_s, 3)},
        "roofline": roofline_entry(kernels[dominant], dominant),
        "kernels": kernels,
        "in_step_event_pair_us": steps.get("_event_pair_us"),
        "copy_calibration": copy,
        "cpu_baseline": cpu,
        "mode_b": mb,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
