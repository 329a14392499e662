"""Pins the CPU oracle (no GPU).

The reference has no golden vectors (its only check is a run-time rocBLAS
comparison), so each oracle function is pinned by something independent of it:
numpy's IEEE conversions, exact integer arithmetic, numpy/einsum in fp64, published
splitmix64 output, the reference's own index formulas evaluated by brute force, and
planted mistakes that the checks must catch.
"""
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ------------------------------------------------------------------------------ conversions
def test_f16_to_f32_every_value(orc):
    h = np.arange(65536, dtype=np.uint16).view(np.float16)
    got = orc.f16_to_f32(h)
    ref = h.astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne(orc):
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(400_000) * np.exp(rng.uniform(-28, 13, 400_000))).astype(np.float32)
    # exact halfway cases between adjacent fp16 values, normal and subnormal, plus edges
    h = np.arange(1, 0x7bff, 97, dtype=np.uint16).view(np.float16).astype(np.float64)
    h_next = (np.arange(1, 0x7bff, 97, dtype=np.uint16) + 1).view(np.float16).astype(np.float64)
    ties = ((h + h_next) / 2).astype(np.float32)
    edges = np.array([65504, 65519.99, 65520, 1e9, 2 ** -24, 2 ** -25, 2 ** -25 * 1.0001, 2 ** -26, 0.0, -0.0,
                      np.inf, -np.inf], dtype=np.float32)
    for v in (x, ties, -ties, edges):
        with np.errstate(over="ignore"):
            ref = v.astype(np.float16)
        assert np.array_equal(orc.f32_to_f16(v).view(np.uint16), ref.view(np.uint16))


def test_f64_to_f16_single_rounding(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(300_000) * np.exp(rng.uniform(-28, 12, 300_000))
    # fp16 values in [1, 2) have ulp 2^-10; h + 2^-11 is a tie.  h + 2^-11 + 2^-40 lies just
    # above the tie: one rounding from fp64 goes up, but via fp32 (ulp 2^-23) it would first
    # become the tie and then round to even -- a double-rounding mistake this catches.
    h = np.arange(0x3c00, 0x4000, dtype=np.uint16).view(np.float16).astype(np.float64)
    just_above_tie = h + 2.0 ** -11 + 2.0 ** -40
    for v in (x, just_above_tie, -just_above_tie):
        with np.errstate(over="ignore"):
            ref = v.astype(np.float16)
        assert np.array_equal(orc.f64_to_f16(v).view(np.uint16), ref.view(np.uint16))
    via_f32 = just_above_tie.astype(np.float32).astype(np.float16)
    assert not np.array_equal(via_f32.view(np.uint16), orc.f64_to_f16(just_above_tie).view(np.uint16))


# ------------------------------------------------------------------------------ generator
def test_splitmix64_published_output(orc):
    # splitmix64 with state 0: first output 0xE220A8397B1DCDAF (Steele, Lea, Flood 2014;
    # the reference value used by every splitmix64 implementation's self-test).
    assert orc.splitmix64(0) == 0xE220A8397B1DCDAF


def test_generator_known_answers(orc):
    kat = json.load(open(os.path.join(GOLDEN, "prng_kat.json")))
    for name, e in kat.items():
        if e["dist"] == "uniform":
            v = orc.uniform_f16((16,), e["seed"], e["tensor_id"])
        else:
            v = orc.normal_f16((16,), e["seed"], e["tensor_id"], 0.1)
        assert [int(x) for x in v.view(np.uint16)] == e["bits"], name


def test_generator_distributions(orc):
    n = 2_000_000
    u = orc.uniform_f16((n,), 1, 0).astype(np.float64)
    assert u.min() >= -1.0 and u.max() <= 1.0
    assert abs(u.mean()) < 3e-3 and abs(u.var() - 1 / 3) < 3e-3
    g = orc.normal_f16((n,), 3, 0, 0.1).astype(np.float64)
    assert abs(g.mean()) < 3e-4 and abs(g.std() - 0.1) < 3e-4
    # streams for different tensors / seeds differ
    assert not np.array_equal(orc.uniform_f16((64,), 1, 0), orc.uniform_f16((64,), 1, 1))
    assert not np.array_equal(orc.uniform_f16((64,), 1, 0), orc.uniform_f16((64,), 2, 0))


# ------------------------------------------------------------------------------ GEMM truth
def test_gemm_f64_matches_numpy(orc):
    A = orc.uniform_f16((70, 90), 0, 0)
    B = orc.uniform_f16((90, 50), 0, 1)
    C, S = orc.gemm_f64(A, B)
    A64, B64 = A.astype(np.float64), B.astype(np.float64)
    assert np.allclose(C, A64 @ B64, rtol=0, atol=1e-12)
    assert np.allclose(S, np.abs(A64) @ np.abs(B64), rtol=1e-14, atol=0)
    # row/column sub-grids and the TN layout give the same numbers
    rows, cols = np.array([0, 7, 69]), np.array([3, 49])
    Cs, Ss = orc.gemm_f64(A, B, rows=rows, cols=cols)
    assert np.array_equal(Cs, C[np.ix_(rows, cols)]) and np.array_equal(Ss, S[np.ix_(rows, cols)])
    Ct, St = orc.gemm_f64(A, np.ascontiguousarray(B.T), b_layout="nk")
    assert np.array_equal(Ct, C) and np.array_equal(St, S)


def test_gemm_golden_small(orc):
    g = np.load(os.path.join(GOLDEN, "gemm_small.npz"))
    C, S = orc.gemm_f64(g["A"], g["B"])
    assert np.array_equal(C, g["C"]) and np.array_equal(S, g["S"])


def test_c1_golden_record(orc):
    """Configuration C1 (256^3, seed 0): the seeded inputs and the fp64 result match the
    committed hashes and sample values."""
    import hashlib

    rec = json.load(open(os.path.join(GOLDEN, "c1_256.json")))
    A = orc.uniform_f16((256, 256), 0, 0)
    B = orc.uniform_f16((256, 256), 0, 1)
    C, S = orc.gemm_f64(A, B)
    h = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    assert h(A.view(np.uint16)) == rec["sha256"]["A_f16_bits"]
    assert h(B.view(np.uint16)) == rec["sha256"]["B_f16_bits"]
    assert h(C) == rec["sha256"]["C_f64"] and h(S) == rec["sha256"]["S_f64"]
    assert C[0, 0] == rec["samples"]["C[0][0]"] and C[255, 255] == rec["samples"]["C[255][255]"]
    assert C[17, 200] == rec["samples"]["C[17][200]"]


def test_fp32_restatements_exact_on_integers(orc):
    rng = np.random.default_rng(3)
    A = rng.integers(-4, 5, size=(33, 70)).astype(np.float16)
    B = rng.integers(-4, 5, size=(70, 45)).astype(np.float16)
    truth = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32)
    assert np.array_equal(orc.gemm_naive_f32(A, B), truth)
    assert np.array_equal(orc.gemm_refkernel_f32(A, B), truth)
    assert np.array_equal(orc.cpu_gemm_f16f32(A, B), truth)


def test_fp32_restatements_within_tolerance(orc):
    A = orc.uniform_f16((40, 3000), 4, 0)
    B = orc.uniform_f16((3000, 30), 4, 1)
    T, S = orc.gemm_f64(A, B)
    for C in (orc.gemm_naive_f32(A, B), orc.gemm_refkernel_f32(A, B), orc.cpu_gemm_f16f32(A, B)):
        bad, worst = orc.check_tol(C, T, S)
        assert bad == 0 and worst < 1e-5


def test_refkernel_blocking_differs_from_naive(orc):
    """The restatement sums 16-term WMMA steps into the accumulator (mmm.cpp:1323-1353), which
    is not the same fp32 arithmetic as GEMM_Naive's running sum (mmm.cpp:57-58)."""
    A = orc.uniform_f16((16, 4096), 7, 0)
    B = orc.uniform_f16((4096, 16), 7, 1)
    assert not np.array_equal(orc.gemm_naive_f32(A, B), orc.gemm_refkernel_f32(A, B))


def _np_naive_f32(A, B):
    """GEMM_Naive's order (mmm.cpp:57-58) in numpy float32: one running sum per output, k
    ascending, every addition rounded to fp32 (the fp16 x fp16 products are exact in fp32)."""
    a, b = A.astype(np.float32), B.astype(np.float32)
    acc = np.zeros((A.shape[0], B.shape[1]), dtype=np.float32)
    for k in range(A.shape[1]):
        acc = acc + np.outer(a[:, k], b[k]).astype(np.float32)
    return acc


def _np_refkernel_f32(A, B, tile=32, step=16):
    """WMMA_Swizzled_Full's order (mmm.cpp:1309-1356) in numpy float32: K walked in 32-deep
    LDS tiles of two 16-deep WMMA steps; each step's 16 products are summed in ascending k
    from zero, then added to the accumulator; past K the operands are zero (mmmTensor.cpp:137-175)."""
    M, K = A.shape
    N = B.shape[1]
    kp = -(-K // tile) * tile
    a = np.zeros((M, kp), dtype=np.float32)
    b = np.zeros((kp, N), dtype=np.float32)
    a[:, :K], b[:K] = A, B
    acc = np.zeros((M, N), dtype=np.float32)
    for k0 in range(0, kp, step):
        s = np.zeros((M, N), dtype=np.float32)
        for k in range(k0, k0 + step):
            s = s + np.outer(a[:, k], b[k]).astype(np.float32)
        acc = acc + s
    return acc


def test_fp32_orders_match_numpy_restatements(orc):
    """Both fp32 restatements reproduce, bit for bit on non-integer inputs (where the order of
    the additions decides the rounding), an independent float32 restatement of their order:
    the naive running sum and the reference kernel's 16-deep steps (K 203, so the last 32-deep
    tile is partly past K)."""
    A = orc.uniform_f16((9, 203), 11, 0)
    B = orc.uniform_f16((203, 7), 11, 1)
    assert np.array_equal(orc.gemm_naive_f32(A, B).view(np.uint32), _np_naive_f32(A, B).view(np.uint32))
    assert np.array_equal(orc.gemm_refkernel_f32(A, B).view(np.uint32), _np_refkernel_f32(A, B).view(np.uint32))
    # the TN layout of the reference's tensor kernel walks K the same way
    Bt = np.ascontiguousarray(B.T)
    assert np.array_equal(orc.gemm_refkernel_f32(A, Bt, b_layout="nk").view(np.uint32),
                          _np_refkernel_f32(A, B).view(np.uint32))


def test_fp32_order_checks_catch_wrong_orders(orc):
    """The numpy restatements tell plausible mistakes apart: K blocked by 8 instead of 16,
    and a running sum without the 16-deep steps, both give other bits on these inputs."""
    A = orc.uniform_f16((9, 203), 11, 0)
    B = orc.uniform_f16((203, 7), 11, 1)
    ref = orc.gemm_refkernel_f32(A, B).view(np.uint32)
    assert not np.array_equal(ref, _np_refkernel_f32(A, B, step=8).view(np.uint32))
    assert not np.array_equal(ref, _np_naive_f32(A, B).view(np.uint32))
    desc = _np_naive_f32(A[:, ::-1], B[::-1])  # k descending
    assert not np.array_equal(orc.gemm_naive_f32(A, B).view(np.uint32), desc.view(np.uint32))


def test_refkernel_zero_fills_k_tail(orc):
    """K not a multiple of 32: elements past K contribute nothing (mmmTensor.cpp:137-175)."""
    rng = np.random.default_rng(8)
    A = rng.integers(-4, 5, size=(5, 37)).astype(np.float16)
    B = rng.integers(-4, 5, size=(37, 6)).astype(np.float16)
    assert np.array_equal(orc.gemm_refkernel_f32(A, B), (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32))


def test_check_tol_catches_planted_errors(orc):
    A = orc.uniform_f16((20, 500), 2, 0)
    B = orc.uniform_f16((500, 20), 2, 1)
    T, S = orc.gemm_f64(A, B)
    C = T.astype(np.float32)
    assert orc.check_tol(C, T, S)[0] == 0
    planted = C.copy()
    planted[3, 4] += np.float32(2e-3 * S[3, 4])
    assert orc.check_tol(planted, T, S)[0] == 1
    nan = C.copy()
    nan[0, 0] = np.nan
    assert orc.check_tol(nan, T, S)[0] == 1
    # a dropped k term (a plausible indexing mistake) is caught
    dropped = (A[:, 1:].astype(np.float64) @ B[1:].astype(np.float64)).astype(np.float32)
    assert orc.check_tol(dropped, T, S)[0] > 0
    # a transposed operand is caught
    Bt = np.ascontiguousarray(B.T)
    wrong = (A.astype(np.float64)[:, :20] @ Bt.astype(np.float64)[:, :20]).astype(np.float32)
    assert orc.check_tol(wrong, T, S)[0] > 0


def test_tolerance_bound_holds_for_fp32_summation(orc):
    """Worst-case fp32 recursive summation error gamma_K*S < 1e-3*S at K = 8192 (K*2^-24 = 4.9e-4)."""
    K = 8192
    assert K * 2.0 ** -24 / (1 - K * 2.0 ** -24) < 1e-3


# ------------------------------------------------------------------------------ contractions
def test_contract_baseline_matches_einsum(orc):
    A = orc.normal_f16((2, 9, 3, 5), 3, 0, 0.1)
    B = orc.normal_f16((3, 5, 11), 3, 1, 0.1)
    C, S = orc.contract_baseline_f64(A, B)
    E = np.einsum("bikl,klj->bij", A.astype(np.float64), B.astype(np.float64)).reshape(18, 11)
    ES = np.einsum("bikl,klj->bij", np.abs(A.astype(np.float64)), np.abs(B.astype(np.float64))).reshape(18, 11)
    assert np.allclose(C, E, rtol=0, atol=1e-14) and np.allclose(S, ES, rtol=1e-14, atol=0)
    # equals the GEMM of the folded operands (the fold the library uses)
    Cg, Sg = orc.gemm_f64(A.reshape(18, 15), B.reshape(15, 11))
    assert np.allclose(C, Cg, rtol=0, atol=1e-14)


def test_contract_baseline_golden_small(orc):
    """The benchmark contraction's layout at a size small enough to commit: the seeded inputs
    and the fp64 loop nest reproduce the fixture exactly."""
    g = np.load(os.path.join(GOLDEN, "contract_baseline_small.npz"))
    assert np.array_equal(orc.normal_f16((2, 3, 4, 5), 11, 0, 0.1).view(np.uint16), g["A"].view(np.uint16))
    assert np.array_equal(orc.normal_f16((4, 5, 6), 11, 1, 0.1).view(np.uint16), g["B"].view(np.uint16))
    C, S = orc.contract_baseline_f64(g["A"], g["B"])
    assert np.array_equal(C, g["C"]) and np.array_equal(S, g["S"])


def test_contract_reference_matches_einsum_and_pack(orc):
    g = np.load(os.path.join(GOLDEN, "contract_ref_small.npz"))
    G, In = g["G"], g["In"]
    rt, nt, mt, rt_l = G.shape
    bt = In.shape[0]
    C, S = orc.contract_reference_f64(G, In)
    E = np.einsum("rnml,bnl->mrb", G.astype(np.float64), In.astype(np.float64)).reshape(mt * rt, bt)
    assert np.allclose(C, E, rtol=0, atol=1e-14)
    assert np.allclose(C.reshape(mt, rt, bt).transpose(0, 2, 1), g["Out"], rtol=0, atol=0)
    # the reference's host pack (mmmTensor.cpp:329-340) followed by its TN GEMM
    hA = orc.pack_reference_G(G)
    assert hA.shape == (mt * rt, nt * rt_l)
    for m, r, n, l in [(0, 0, 0, 0), (1, 3, 2, 7), (0, 2, 1, 5)]:
        assert hA[m * rt + r, n * rt_l + l] == G[r, n, m, l]
    Cp, _ = orc.gemm_f64(hA, In.reshape(bt, nt * rt_l), b_layout="nk")
    assert np.allclose(Cp, C, rtol=0, atol=1e-14)


# ------------------------------------------------------------------------------ reference remap
def _remap_image(orc, gx, gy):
    seen = {}
    for by in range(gy):
        for bx in range(gx):
            t = orc.ref_block_remap(bx, by, gx, gy)
            seen[t] = seen.get(t, 0) + 1
    return seen


@pytest.mark.parametrize("grid", [(2, 2), (16, 64), (32, 33), (64, 64)])
def test_reference_remap_bijective_at_config_grids(orc, grid):
    gx, gy = grid
    seen = _remap_image(orc, gx, gy)
    assert len(seen) == gx * gy and max(seen.values()) == 1


def test_reference_remap_defect(orc):
    """mmm.cpp:1219-1236 skips tiles when gridDim.x > 32 is not a multiple of 32."""
    seen = _remap_image(orc, 33, 4)
    missing = 33 * 4 - len(seen)
    dup = sum(v - 1 for v in seen.values() if v > 1)
    assert missing == 2 and dup == 2


def test_cpu_gemm_ragged(orc):
    A = orc.uniform_f16((131, 77), 6, 0)
    B = orc.uniform_f16((77, 101), 6, 1)
    T, S = orc.gemm_f64(A, B)
    bad, worst = orc.check_tol(orc.cpu_gemm_f16f32(A, B, threads=3), T, S)
    assert bad == 0
