"""The benchmark's own checks, on the GPU: the full-output validation that precedes every timed
run must count wrong outputs (a planted error, NaN, a transposed operand), and the hipBLASLt
comparison's candidate search must bind one of its candidates and give the same product."""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    if REPO not in sys.path:
        sys.path.insert(0, REPO)
    import bench as b

    return b


def test_validate_step_counts_wrong_outputs(bench, mm, cuda):
    torch = cuda
    M, N, K = 300, 264, 520
    A = torch.empty((M, K), dtype=torch.float16, device="cuda")
    B = torch.empty((K, N), dtype=torch.float16, device="cuda")
    mm.fill_uniform(A, 13, 0)
    mm.fill_uniform(B, 13, 1)
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")
    truth = lambda: mm.gemm_truth(A, B)
    good = bench.validate_step(torch, mm.bind_gemm(A, B, C), C, truth)
    assert good["outputs"] == M * N and good["violations"] == 0 and good["worst_err_over_S"] < 1e-5

    def planted():
        mm.gemm(A, B, C)
        C[7, 11] += 0.01 * float(C.abs().max())

    bad = bench.validate_step(torch, planted, C, truth)
    assert bad["violations"] >= 1 and bad["worst_err_over_S"] > 1e-3

    def nan():
        mm.gemm(A, B, C)
        C[0, 0] = float("nan")

    assert bench.validate_step(torch, nan, C, truth)["violations"] == 1
    # a launch that never writes C leaves the NaN the check fills it with: every output fails
    assert bench.validate_step(torch, lambda: None, C, truth)["violations"] == M * N
    # B's rows in reverse order (a plausible indexing mistake)
    Bf = B.flip(0).contiguous()
    wrong = bench.validate_step(torch, lambda: mm.gemm(A, Bf, C), C, truth)
    assert wrong["violations"] > M * N // 2


@pytest.mark.parametrize("shape", [(256, 256, 256), (1000, 777, 320)])
def test_hipblaslt_tuning_binds_a_candidate(orc, mm, cuda, shape):
    torch = cuda
    M, N, K = shape
    A = orc.uniform_f16((M, K), 6, 0)
    B = orc.uniform_f16((K, N), 6, 1)
    Ad = torch.from_numpy(A).cuda()
    Bd = torch.from_numpy(B).cuda()
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    launch = mm.bind_witness_hipblaslt(Ad, Bd, C)
    t = launch.tuning
    assert 1 <= t["algos"] <= 16 and 0 <= t["best_index"] < t["algos"]
    assert len(t["ms"]) == t["algos"]
    timed = [x for x in t["ms"] if x > 0]
    assert timed and t["ms"][t["best_index"]] == min(timed)
    assert launch.plan.info() == (t["algos"], t["best_index"])
    C.fill_(float("nan"))
    launch()
    torch.cuda.synchronize()
    T, S = orc.gemm_f64(A, B)
    bad, worst = orc.check_tol(C.cpu().numpy(), T, S)
    assert bad == 0, worst
