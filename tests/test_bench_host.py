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
    assert a["algorithmic_bytes"] == (2 * Hkv * P * hd * 2 + B1 * N * 2 * Hkv * hd * 2
                                      + 2 * R * H * hd * 2 + 8 * R * H)
    assert a["algorithmic_flops"] == 4 * R * H * (P + N) * hd
    q = bench.kernel_roofline("qkv", 0.02, w, R, B1, N, P)
    nq = (H + 2 * Hkv) * hd
    bias = nq * 2 if sh.qkv_bias else 0
    assert q["algorithmic_bytes"] == nq * D * 2 + bias + R * D * 2 + R * nq * 2 + 2 * N * hd * 2
    with pytest.raises(KeyError):
        bench.kernel_roofline("nope", 1.0, w, R, B1, N, P)


def test_committed_traffic_table_is_per_launch_bytes():
    t = bench.load_traffic("cfg3_7b")
    assert t["gate_up"] > 2.7e8                      # the 271 MB weight stream, read once
    raw = json.loads((bench.ROOT / "profiles" / "traffic_cfg3_7b.json").read_text())
    for name, v in raw["kernels"].items():
        assert v["bytes_per_launch"] == t[name]
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
