"""bench.py's host-side pieces (CPU only): the contract's refusals, the
per-kernel algorithmic bytes/flops against the per-unit figures they are built
from, the traffic table, and the workloads' draft graphs."""

import json

import pytest

import bench
from specfold_amd.configs import SYNTHETIC_DRAFT_GRAPH, WORKLOADS, draft_graph, workload


def test_more_than_one_gpu_is_refused(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err


def test_defaults_finish_within_minutes():
    a = bench.parse_args([])
    assert a.gpus == 1 and a.workload == "cfg3_7b"
    assert a.steps * 10 <= 1000 and a.warmup <= a.steps


@pytest.mark.parametrize("name", ["cfg3_7b", "cfg5_14b_16k"])
def test_roofline_bytes_follow_the_unit_figures(name):
    """Weight bytes dominate each GEMM's figure; attention's is the prefix K/V plus
    the block; frac = achieved / peak with the bound the larger time picks."""
    w = workload(name)
    sh = w.shape
    D, I, H, Hkv, hd = sh.hidden, sh.intermediate, sh.heads, sh.kv_heads, sh.head_dim
    R, B1, N, P = 39, 8, 32, w.prefix
    k = bench.kernel_roofline("gate_up", 0.05, w, R, B1, N, P)
    assert k["algorithmic_bytes"] == 2 * I * D * 2 + R * D * 2 + R * I * 2
    assert k["algorithmic_flops"] == 4 * R * D * I
    assert k["bound"] == "hbm"
    assert k["frac"] == pytest.approx(k["algorithmic_bytes"] / 50e-6 / 8e12, rel=1e-3)
    a = bench.kernel_roofline("attn", 0.05, w, R, B1, N, P)
    BN = B1 * N
    assert a["algorithmic_bytes"] == (2 * Hkv * P * hd * 2 + BN * 2 * Hkv * hd * 2
                                      + R * H * hd * 2 + BN * H * hd * (4 + 2) + 8 * BN * H)
    assert a["algorithmic_flops"] == 4 * R * H * P * hd + 4 * BN * H * N * hd
    q = bench.kernel_roofline("qkv", 0.02, w, R, B1, N, P)
    nq = (H + 2 * Hkv) * hd
    bias = nq * 2 if sh.qkv_bias else 0
    assert q["algorithmic_bytes"] == nq * D * 2 + bias + R * D * 2 + R * nq * 2 + 2 * N * hd * 2
    with pytest.raises(KeyError):
        bench.kernel_roofline("nope", 1.0, w, R, B1, N, P)


def _launched(name, optional):
    """The kernel names one launch of entry point `name` dispatches: each pattern's
    last alternative; optional ("?") kernels only when `optional`."""
    out = []
    for pat in bench.PMC_KERNELS[name]:
        pat = pat if isinstance(pat, str) else pat[-1]
        if pat.startswith("?"):
            if optional:
                out.append(pat[1:])
        else:
            out.append(pat)
    return out


def _pmc_csv(path, w, fetch_kib, write_kib, cal_kib, optional=True):
    """A counter_collection.csv as rocprofv3 --pmc writes it for one --pmc-pass run:
    the verify steps before the pause, then the calibration copy and PMC_ORDER's
    launches (one per layer, the once-per-step ones once), with a torch copy
    between two of them."""
    import csv
    rows, disp, t = [], 0, 0

    def emit(name, kib_f, kib_w, gap=1000):
        nonlocal disp, t
        disp += 1
        t += gap
        for c, v in (("FETCH_SIZE", kib_f), ("WRITE_SIZE", kib_w)):
            rows.append({"Dispatch_Id": disp, "Kernel_Name": "void " + name,
                         "Start_Timestamp": t, "Grid_Size": 256, "Counter_Name": c,
                         "Counter_Value": v})

    L = w.shape.layers
    n_after = 1 + sum(len(bench.PMC_KERNELS[n]) * (1 if n in bench.ONCE_PER_STEP else L)
                      for n in bench.PMC_ORDER) + 1
    for _ in range(n_after + 5):
        emit("warmup_kernel", 7.0, 3.0)
    emit("vectorized_elementwise_kernel", cal_kib, cal_kib, gap=10 ** 9)   # the pause
    for name in bench.PMC_ORDER:
        for li in range(1 if name in bench.ONCE_PER_STEP else L):
            for j, pat in enumerate(_launched(name, optional)):
                emit(pat + "x>(int)", fetch_kib[name] + li + j, write_kib[name])
            if name == "attn" and li == 0:
                emit("elementwise_kernel_copy", 1e6, 1e6)
    with open(path, "w", newline="") as f:
        wr = csv.DictWriter(f, fieldnames=list(rows[0]))
        wr.writeheader()
        wr.writerows(rows)


@pytest.mark.parametrize("optional", [True, False])
def test_traffic_table_scales_each_launch_by_the_copy_calibration(tmp_path, optional):
    """Bytes per launch = mean over layers of the sum over the launch's kernels of
    FETCH_SIZE and WRITE_SIZE (KiB), times 256 MiB / the calibration copy's reading;
    kernels of other libraries between ours are skipped; an optional kernel ("?":
    gate/up's SiLU fix-up) counts where it was launched and is not looked for
    further on where it was not."""
    w = workload("cfg3_7b")
    L = w.shape.layers
    fetch = {n: 100.0 * (i + 1) for i, n in enumerate(bench.PMC_ORDER)}
    write = {n: 10.0 * (i + 1) for i, n in enumerate(bench.PMC_ORDER)}
    cal = (256 << 20) / 1024 / 2.0          # the counter reads half the copy's bytes
    p = tmp_path / "counter_collection.csv"
    _pmc_csv(p, w, fetch, write, cal, optional)
    out = bench.traffic_table([str(p)], "cfg3_7b")
    assert out["calibration"]["fetch_factor"] == pytest.approx(2.0)
    for name in bench.PMC_ORDER:
        k = len(_launched(name, optional))
        n = 1 if name in bench.ONCE_PER_STEP else L
        f_mean = sum(fetch[name] * k + k * li + k * (k - 1) / 2 for li in range(n)) / n
        want = (f_mean + write[name] * k) * 1024 * 2.0
        assert out["kernels"][name]["bytes_per_launch"] == int(want), name
    assert bench.load_traffic("no_such_workload") == {}


@pytest.mark.parametrize("B", [1, 4, 7])
def test_draft_graphs_are_trees(B):
    """Every node's (position rank, vocab rank) set extends an earlier node's set
    by one pair (or is a root), at most 3 nodes per depth, depth <= 8."""
    g = draft_graph(B)
    nodes = [set(map(tuple, n["ij_set"])) for n in g["selected_nodes"]]
    assert len(nodes) == B
    per_depth = {}
    for i, s in enumerate(nodes):
        per_depth[len(s)] = per_depth.get(len(s), 0) + 1
        assert len(s) == 1 or any(len(p) == len(s) - 1 and p < s for p in nodes[:i])
    assert max(per_depth.values()) <= 3 and max(per_depth) <= 8
    assert g["selected_nodes"][0] is not SYNTHETIC_DRAFT_GRAPH["selected_nodes"][0]
    with pytest.raises(ValueError):
        draft_graph(8)


def test_workloads_cover_the_baseline_configs():
    assert {"cfg1_1p5b_layer", "cfg2_1p5b", "cfg3_7b", "cfg4_8b_x4", "cfg5_14b_16k"} <= set(WORKLOADS)
    assert workload("cfg4_8b_x4").family == "nld" and workload("cfg4_8b_x4").batch == 4
    assert workload("cfg5_14b_16k").shuffled_pages and workload("cfg5_14b_16k").prefix == 16384
    assert workload("cfg3_7b").family == "fastdllm" and workload("cfg3_7b").branches == 8
