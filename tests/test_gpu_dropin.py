"""The C++ drop-in at the reference's own call sites, on the GPU.

`rdna4-gemm-wmma_amd/lib/dropin_callsite` (built from `examples/dropin_callsite.cpp` by the
library's Makefile) is the reference's benchmark program shape -- `_Float16*` host and device
buffers, hipMemcpy in, one warm-up, timed launches on the null stream, hipMemcpy out
(mmm.cpp:1441-1500; mmmTensor.cpp:345-371) -- with the kernel launch replaced by
`mmm::WMMA_Swizzled_Full<2,2,4,4>(dA, dB, dC, DIM_I, DIM_J, DIM_K)` and
`mmm::WMMA_Tensor(dG, d_Input, d_Output, mt, bt, rt, nt, rt_l)` from include/mmm.hpp (and, by name
on its command line, the lineage's WMMA_Templated_Base / WMMA_LDS_Padded / WMMA_LDS_Swizzled and
GEMM_Naive).  Its
outputs are checked here against the CPU oracle: within the tolerance against the fp64 truth on
the seeded configuration-1 inputs, bit for bit on integer-valued inputs.
"""
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(REPO, "rdna4-gemm-wmma_amd", "lib", "dropin_callsite")


def _run(args, tmp_path):
    assert os.path.exists(EXE), f"{EXE} is not built (make -C rdna4-gemm-wmma_amd)"
    print(f"[dropin] {' '.join(map(str, args))}", flush=True)
    r = subprocess.run([EXE, *map(str, args)], capture_output=True, text=True, timeout=120, cwd=tmp_path)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


def _gemm(tmp_path, A, B, kernel="WMMA_Swizzled_Full"):
    M, K = A.shape
    N = B.shape[1]
    a, b, c = tmp_path / "A.bin", tmp_path / "B.bin", tmp_path / "C.bin"
    np.ascontiguousarray(A, dtype=np.float16).tofile(a)
    np.ascontiguousarray(B, dtype=np.float16).tofile(b)
    out = _run(["gemm", M, N, K, a, b, c, kernel], tmp_path)
    assert out.startswith(f"gemm {M}x{N}x{K} {kernel} best ")
    C = np.fromfile(c, dtype=np.float32)
    assert C.size == M * N
    return C.reshape(M, N)


def test_callsite_gemm_config1(orc, tmp_path):
    """Configuration 1 (256^3, U[-1,1) seed 0) through the reference's template spelling
    <2,2,4,4>: every output within 1e-3 * sum|a*b| of the fp64 truth and of the CPU restatement
    of the reference kernel's arithmetic."""
    A = orc.uniform_f16((256, 256), 0, 0)
    B = orc.uniform_f16((256, 256), 0, 1)
    C = _gemm(tmp_path, A, B)
    T, S = orc.gemm_f64(A, B)
    bad, worst = orc.check_tol(C, T, S)
    assert bad == 0, f"{bad} outputs outside tolerance (worst {worst:.3g})"
    R = orc.gemm_refkernel_f32(A, B)
    bad, worst = orc.check_tol(C, R.astype(np.float64), S)
    assert bad == 0, f"{bad} outputs outside tolerance of the reference-kernel restatement (worst {worst:.3g})"


@pytest.mark.parametrize("kernel", ["WMMA_Templated_Base", "WMMA_LDS_Padded", "WMMA_LDS_Swizzled"])
def test_callsite_lineage_names(orc, tmp_path, kernel):
    """The reference's earlier names for the same GEMM (mmm.cpp:694-1198), spelled <2,2,4,4> at
    configuration 1: every output within 1e-3 * sum|a*b| of the fp64 truth."""
    A = orc.uniform_f16((256, 256), 0, 0)
    B = orc.uniform_f16((256, 256), 0, 1)
    C = _gemm(tmp_path, A, B, kernel)
    T, S = orc.gemm_f64(A, B)
    bad, worst = orc.check_tol(C, T, S)
    assert bad == 0, f"{kernel}: {bad} outputs outside tolerance (worst {worst:.3g})"


def test_callsite_gemm_naive(orc, tmp_path):
    """mmm::GEMM_Naive at the reference's GEMM_Naive call shape (mmm.cpp:52-62): bit for bit the
    oracle's restatement of its fp32, k-ascending sum, on configuration 1 and on a ragged shape."""
    for M, N, K, seed in ((256, 256, 256, 0), (37, 141, 203, 8)):
        A = orc.uniform_f16((M, K), seed, 0)
        B = orc.uniform_f16((K, N), seed, 1)
        C = _gemm(tmp_path, A, B, "GEMM_Naive")
        R = orc.gemm_naive_f32(A, B)
        assert np.array_equal(C, R), f"{M}x{N}x{K}: {int((C != R).sum())} outputs differ from the k-ascending sum"


def test_callsite_gemm_exact_ragged(orc, tmp_path):
    """A shape the reference's unmasked kernel cannot run (no dimension a multiple of its 128x128
    tile) on integer-valued inputs: C equals the int64 product bit for bit."""
    rng = np.random.default_rng(31)
    M, N, K = 301, 203, 357
    A = rng.integers(-4, 5, size=(M, K)).astype(np.float16)
    B = rng.integers(-4, 5, size=(K, N)).astype(np.float16)
    C = _gemm(tmp_path, A, B)
    assert np.array_equal(C, (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("dims", [(4, 96, 16, 3, 40), (2, 160, 64, 2, 128)], ids=lambda d: "-".join(map(str, d)))
def test_callsite_tensor(orc, tmp_path, dims):
    """The tensor program (G[r][n][m][l], Input[b][n][l] -> Out[m][b][r], mmmTensor.cpp:20-28,
    246-252, 329-340) through mmm::WMMA_Tensor: within tolerance of the oracle's 5-D loop nest on
    seeded inputs, and bit for bit on integer inputs."""
    mt, bt, rt, nt, rt_l = dims
    g, i, o = tmp_path / "G.bin", tmp_path / "In.bin", tmp_path / "Out.bin"

    def run(G, In):
        G.tofile(g)
        In.tofile(i)
        out = _run(["tensor", mt, bt, rt, nt, rt_l, g, i, o], tmp_path)
        assert out.startswith(f"tensor mt={mt} bt={bt} rt={rt} nt={nt} rt_l={rt_l} best ")
        Out = np.fromfile(o, dtype=np.float32).reshape(mt, bt, rt)
        return np.ascontiguousarray(Out.transpose(0, 2, 1).reshape(mt * rt, bt))  # rows m*rt + r

    G = orc.uniform_f16((rt, nt, mt, rt_l), 5, 0)
    In = orc.uniform_f16((bt, nt, rt_l), 5, 1)
    T, S = orc.contract_reference_f64(G, In)
    bad, worst = orc.check_tol(run(G, In), T, S)
    assert bad == 0, f"{bad} outputs outside tolerance (worst {worst:.3g})"

    rng = np.random.default_rng(32)
    Gi = rng.integers(-4, 5, size=(rt, nt, mt, rt_l)).astype(np.float16)
    Ii = rng.integers(-4, 5, size=(bt, nt, rt_l)).astype(np.float16)
    Ti, _ = orc.contract_reference_f64(Gi, Ii)
    assert np.array_equal(run(Gi, Ii), Ti.astype(np.float32))
