"""On-device cross-check kernels (mmm_gemm_naive_f16f32, mmm_gemm_truth_f64,
mmm_contract5d_truth_f64) and full-output validation of every configuration with them.

The cross-check kernels are pinned bit for bit against the CPU oracle:
  * the fp32 naive kernel against the oracle's GEMM_Naive restatement (mmm.cpp:52-62), on small
    shapes;
  * the fp64 truth and scale against the oracle's fp64 loops (products of fp16 values are
    exact in fp64 and both sum in ascending k, so they agree exactly), on small shapes in full
    and at every configuration's full size on a sampled sub-grid.
Pinned that way, they validate every element of the full-size outputs on the device with the
tolerance |C - T| <= 1e-3 * S, S = sum_k |a*b|, instead of a sampled sub-grid.
"""
import numpy as np
import pytest

from conftest import to_dev

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _violations(C, T, S):
    """(count of elements with NOT |C - T| <= TOL * S, worst |C - T| / S); NaN counts as bad."""
    d = (C.double() - T).abs()
    ok = d <= TOL * S
    worst = (d / S.clamp_min(1e-300)).max().item() if d.numel() else 0.0
    return int((~ok).sum().item()), worst


# ------------------------------------------------------------------------------ pinning
@pytest.mark.parametrize("shape", [(300, 264, 200), (67, 129, 1000), (1, 1, 1), (33, 65, 31)],
                         ids=lambda s: "x".join(map(str, s)))
def test_naive_matches_oracle_bitwise(mm, cuda, orc, shape):
    M, N, K = shape
    A = orc.uniform_f16((M, K), 21, 0)
    B = orc.uniform_f16((K, N), 21, 1)
    got = mm.gemm_naive(to_dev(cuda, A), to_dev(cuda, B)).cpu().numpy()
    want = orc.gemm_naive_f32(A, B)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_naive_leading_dimensions(mm, cuda, orc):
    M, N, K = 70, 90, 150
    Aw = orc.uniform_f16((M, K + 13), 22, 0)
    Bw = orc.uniform_f16((K, N + 7), 22, 1)
    Cw = cuda.full((M, N + 5), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm_naive(to_dev(cuda, Aw)[:, :K], to_dev(cuda, Bw)[:, :N], Cw[:, :N])
    got = Cw.cpu().numpy()
    want = orc.gemm_naive_f32(np.ascontiguousarray(Aw[:, :K]), np.ascontiguousarray(Bw[:, :N]))
    assert np.array_equal(got[:, :N], want)
    assert np.isnan(got[:, N:]).all(), "wrote outside the [M][N] window"


def test_naive_zero_k(mm, cuda):
    A = cuda.empty((5, 0), dtype=cuda.float16, device="cuda")
    B = cuda.empty((0, 9), dtype=cuda.float16, device="cuda")
    C = cuda.full((5, 9), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm_naive(A, B, C)
    assert (C == 0).all().item()


@pytest.mark.parametrize("shape", [(300, 264, 200), (67, 129, 1000)], ids=lambda s: "x".join(map(str, s)))
def test_truth_matches_oracle_bitwise(mm, cuda, orc, shape):
    M, N, K = shape
    A = orc.normal_f16((M, K), 23, 0, 0.1)
    B = orc.normal_f16((K, N), 23, 1, 0.1)
    T, S = mm.gemm_truth(to_dev(cuda, A), to_dev(cuda, B))
    Tw, Sw = orc.gemm_f64(A, B)
    assert np.array_equal(T.cpu().numpy(), Tw)
    assert np.array_equal(S.cpu().numpy(), Sw)


@pytest.mark.parametrize("shape", [(4097, 4095, 4111), (8192, 2048, 2048), (16, 8192, 8192), (8192, 8192, 8192)],
                         ids=lambda s: "x".join(map(str, s)))
def test_truth_matches_oracle_at_full_size(mm, cuda, orc, shape):
    """The fp64 truth kernel at the configurations' full sizes, bit for bit against the oracle on a
    sampled sub-grid (first, last and spread rows and columns): the every-output checks of those
    configurations rest on this kernel, so it is pinned at their sizes, not only at small ones."""
    M, N, K = shape
    A = orc.uniform_f16((M, K), 29, 0)
    B = orc.uniform_f16((K, N), 29, 1)
    T, S = mm.gemm_truth(to_dev(cuda, A), to_dev(cuda, B))
    rows = np.unique(np.r_[0, 1, M - 1, np.linspace(0, M - 1, 24).astype(np.int64)])
    cols = np.unique(np.r_[0, N - 1, np.linspace(0, N - 1, 40).astype(np.int64)])
    Tw, Sw = orc.gemm_f64(A, B, rows=rows, cols=cols)
    r, c = cuda.as_tensor(rows, device="cuda"), cuda.as_tensor(cols, device="cuda")
    assert np.array_equal(T[r][:, c].cpu().numpy(), Tw)
    assert np.array_equal(S[r][:, c].cpu().numpy(), Sw)


def test_truth_without_scale(mm, cuda, orc):
    A = orc.uniform_f16((40, 50), 24, 0)
    B = orc.uniform_f16((50, 60), 24, 1)
    T, S = mm.gemm_truth(to_dev(cuda, A), to_dev(cuda, B), with_scale=False)
    assert S is None
    assert np.array_equal(T.cpu().numpy(), orc.gemm_f64(A, B)[0])


def test_contract_truth_reference_layout_bitwise(mm, cuda, orc):
    mt, bt, rt, nt, rt_l = 4, 40, 8, 3, 24
    G = orc.uniform_f16((rt, nt, mt, rt_l), 25, 0)
    In = orc.uniform_f16((bt, nt, rt_l), 25, 1)
    T = cuda.empty((mt, bt, rt), dtype=cuda.float64, device="cuda")
    S = cuda.empty_like(T)
    mm.contract_truth(mm.contract_desc_reference(mt, bt, rt, nt, rt_l), to_dev(cuda, G), to_dev(cuda, In), T, S)
    Tw, Sw = orc.contract_reference_f64(G, In)  # [m*rt + r][b]
    got_T = T.cpu().numpy().transpose(0, 2, 1).reshape(mt * rt, bt)
    got_S = S.cpu().numpy().transpose(0, 2, 1).reshape(mt * rt, bt)
    assert np.array_equal(got_T, Tw)
    assert np.array_equal(got_S, Sw)


def test_contract_truth_baseline_bitwise(mm, cuda, orc):
    b, i, k, l, j = 2, 30, 3, 20, 50
    A = orc.normal_f16((b, i, k, l), 26, 0, 0.1)
    B = orc.normal_f16((k, l, j), 26, 1, 0.1)
    T = cuda.empty((b, i, j), dtype=cuda.float64, device="cuda")
    S = cuda.empty_like(T)
    mm.contract_truth(mm.contract_desc_baseline(b, i, k, l, j), to_dev(cuda, A), to_dev(cuda, B), T, S)
    Tw, Sw = orc.contract_baseline_f64(A, B)  # [b*i][j]
    assert np.array_equal(T.cpu().numpy().reshape(b * i, j), Tw)
    assert np.array_equal(S.cpu().numpy().reshape(b * i, j), Sw)


def test_cross_check_invalid_arguments(mm, cuda):
    A = cuda.zeros((4, 4), dtype=cuda.float16, device="cuda")
    L = mm.lib()
    assert L.mmm_gemm_naive_f16f32(None, None, None, 4, 4, 4, 4, 4, 4, None) != 0
    assert L.mmm_gemm_truth_f64(A.data_ptr(), A.data_ptr(), None, None, 4, 4, 4, 4, 4, 4, None) != 0
    assert L.mmm_gemm_truth_f64(A.data_ptr(), A.data_ptr(), A.data_ptr(), None, 4, 4, 4, 3, 4, 4, None) != 0
    assert L.mmm_contract5d_truth_f64(None, None, None, None, None, None) != 0


# ------------------------------------------------------------------------------ full outputs
def _full_gemm_check(mm, cuda, M, N, K, seed, fill="uniform"):
    A = cuda.empty((M, K), dtype=cuda.float16, device="cuda")
    B = cuda.empty((K, N), dtype=cuda.float16, device="cuda")
    if fill == "uniform":
        mm.fill_uniform(A, seed, 0)
        mm.fill_uniform(B, seed, 1)
    else:
        mm.fill_normal(A, seed, 0, 0.1)
        mm.fill_normal(B, seed, 1, 0.1)
    C = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm(A, B, C)
    T, S = mm.gemm_truth(A, B)
    bad, worst = _violations(C, T, S)
    assert bad == 0, f"{M}x{N}x{K}: {bad} of {M * N} outputs out of tolerance (worst {worst:.3g})"
    return A, B, T, S, worst


def test_config2_8192_every_output(mm, cuda):
    """C2 (8192^3, U[-1,1), seed 1): all 67M outputs within tolerance; the fp32 naive too."""
    A, B, T, S, worst = _full_gemm_check(mm, cuda, 8192, 8192, 8192, 1)
    assert worst < 1e-4
    Cn = mm.gemm_naive(A, B)
    bad, _ = _violations(Cn, T, S)
    assert bad == 0


def test_config3_ragged_every_output(mm, cuda):
    _full_gemm_check(mm, cuda, 4097, 4095, 4111, 2)


def test_config5_skinny_every_output(mm, cuda):
    _full_gemm_check(mm, cuda, 16, 8192, 8192, 4)


def test_config4_contraction_every_output(mm, cuda):
    b, i, k, l, j = 8, 1024, 32, 64, 2048
    A = cuda.empty((b, i, k, l), dtype=cuda.float16, device="cuda")
    B = cuda.empty((k, l, j), dtype=cuda.float16, device="cuda")
    mm.fill_normal(A, 3, 0, 0.1)
    mm.fill_normal(B, 3, 1, 0.1)
    d = mm.contract_desc_baseline(b, i, k, l, j)
    C = cuda.full((b, i, j), float("nan"), dtype=cuda.float32, device="cuda")
    mm.contract(d, A, B, C)
    T = cuda.empty((b, i, j), dtype=cuda.float64, device="cuda")
    S = cuda.empty_like(T)
    mm.contract_truth(d, A, B, T, S)
    bad, worst = _violations(C, T, S)
    assert bad == 0, f"{bad} outputs out of tolerance (worst {worst:.3g})"


def test_reference_contraction_every_output(mm, cuda):
    """The reference's tensor program at its own size (mmmTensor.cpp:20-28), every output."""
    mt, bt, rt, nt, rt_l = 128, 8192, 64, 64, 128
    G = cuda.empty((rt, nt, mt, rt_l), dtype=cuda.float16, device="cuda")
    In = cuda.empty((bt, nt, rt_l), dtype=cuda.float16, device="cuda")
    mm.fill_uniform(G, 5, 0)
    mm.fill_uniform(In, 5, 1)
    d = mm.contract_desc_reference(mt, bt, rt, nt, rt_l)
    Out = cuda.full((mt, bt, rt), float("nan"), dtype=cuda.float32, device="cuda")
    mm.contract(d, G, In, Out)
    T = cuda.empty((mt, bt, rt), dtype=cuda.float64, device="cuda")
    S = cuda.empty_like(T)
    mm.contract_truth(d, G, In, T, S)
    bad, worst = _violations(Out, T, S)
    assert bad == 0, f"{bad} outputs out of tolerance (worst {worst:.3g})"


@pytest.mark.parametrize("tile", ["256x256", "256x128", "128x256", "128x128", "64x64", "192x192"])
def test_every_tile_every_output(mm, cuda, tile):
    M, N, K = 2000, 1500, 1032
    A = cuda.empty((M, K), dtype=cuda.float16, device="cuda")
    B = cuda.empty((K, N), dtype=cuda.float16, device="cuda")
    mm.fill_uniform(A, 27, 0)
    mm.fill_uniform(B, 27, 1)
    C = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm(A, B, C, tile=tile)
    T, S = mm.gemm_truth(A, B)
    bad, worst = _violations(C, T, S)
    assert bad == 0, f"{tile}: {bad} outputs out of tolerance (worst {worst:.3g})"
