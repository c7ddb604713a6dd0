"""The whole HIP verify step on the CPU: FoldedVerifyEngine.forward (both model
families) with every kernel it launches compiled from its own source for the
SIMT simulator of tests/sim (tests/simlib.py), stage by stage against the oracle
with the same checks and tolerances as the GPU parity tests
(tests/test_gpu_engine_parity.py: integer outputs bit-exact, q/k/v and hidden
states within bf16 rounding, attention state within fp32 attention rounding).

Test infrastructure: the engine refuses a model outside the GPU
(FoldedVerifyEngine._check_device); the subclass below lifts that check for the
simulated library only, and runs without HIP graphs."""

import pytest
import torch

from oracle.folded_reference import StepTrace, folded_verify_step, llama4_q_scale
from specfold_amd.engine import FoldedVerifyEngine
from specfold_amd.kv_cache import PagedKVCache
from tests.helpers import SHAPE_G2, SHAPE_G7, SHAPE_N4, err_stats, make_case, make_nld_case
from tests.simlib import build_sim_library, compiler, use_sim_library
from tests.test_gpu_engine_parity import check_layers


class SimEngine(FoldedVerifyEngine):
    """The engine over CPU tensors, for the simulated kernels only."""

    @staticmethod
    def _check_device(device):
        if device.type != "cpu":
            raise ValueError("SimEngine runs the simulated kernels on CPU tensors")


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    if compiler() is None:
        pytest.skip("no clang++ (the simulator needs clang's vector extensions)")
    path = build_sim_library(tmp_path_factory.mktemp("simlib"))
    with use_sim_library(path) as lib:
        yield lib


def run(case, q_scale=None):
    tr = StepTrace()
    ref_logits = folded_verify_step(case.model_cpu, case.tokens, case.kv, case.delta, trace=tr,
                                    shift=False, q_scale=q_scale)
    eng = SimEngine(case.model_cpu)
    eng.use_graphs = False
    cache = None
    if case.kv is not None:
        cache = PagedKVCache(len(case.kv), case.kv[0][0].shape[1], 128, 512, page_size=16,
                             device="cpu", page_order="shuffled", seed=5)
        cache.load_dense(case.kv)
    trace = []
    tf = {li: lt.h_in for li, lt in enumerate(tr.layers)}
    logits = eng.forward(case.tokens, cache, case.delta, trace=trace, teacher=tf, q_scale=q_scale)
    return tr, ref_logits, trace, logits


@pytest.mark.parametrize("name,shape,seed,P,delta", [
    ("g2_p100", SHAPE_G2, 1, 100, 0.1),
    ("g7_p300", SHAPE_G7, 3, 300, 0.05),
])
def test_fastdllm_layers_teacher_forced(sim, name, shape, seed, P, delta):
    case = make_case(shape, seed, P=P, delta=delta)
    tr, ref_logits, trace, logits = run(case)
    check_layers(case, shape, tr, trace)
    st = err_stats(logits.float(), ref_logits.float())
    print(f"{name} logits (teacher-forced last layer): {st}")
    assert st["max_abs"] <= 2e-2 * max(1.0, st["ref_absmax"])


@pytest.mark.parametrize("name,shape,seed,P,delta,omax", [
    ("n4_p100", SHAPE_N4, 1, 100, 0.1, 64),    # llama-4 q scale active
    ("n4_p0", SHAPE_N4, 3, 0, 0.1, 16),
])
def test_nld_layers_teacher_forced(sim, name, shape, seed, P, delta, omax):
    case = make_nld_case(shape, seed, P=P, delta=delta, omax=omax)
    qs = llama4_q_scale(case.model_cpu.config, P, case.tokens.shape[1])
    assert (qs is not None) == (P + case.tokens.shape[1] > omax)
    tr, ref_logits, trace, logits = run(case, q_scale=qs)
    check_layers(case, shape, tr, trace)
