"""GPU parity tests: the HIP library (through its C ABI) against the CPU oracle.

Tolerance (BASELINE): |C - C_ref| <= 1e-3 * S elementwise, S = sum_k |a_ik * b_kj|,
against the fp64 truth and against the CPU restatement of the reference kernel's fp32
arithmetic.  Integer-valued inputs (|a|, |b| <= 4, 16*K < 2^24) make every fp32 partial
sum exact in any order, so those cases must match an int64 product bit for bit.
At full size, outputs are checked on sampled rows/columns plus row and column checksums
(C 1 = A (B 1), 1^T C = (1^T A) B, each within the summed tolerance).
"""
import ctypes as C

import numpy as np
import pytest

from conftest import to_dev

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _int_inputs(rng, M, N, K):
    A = rng.integers(-4, 5, size=(M, K)).astype(np.float16)
    B = rng.integers(-4, 5, size=(K, N)).astype(np.float16)
    truth = A.astype(np.int64) @ B.astype(np.int64)
    return A, B, truth.astype(np.float32)


def _check_sampled(orc, A, B, C, rows, cols, label):
    T, S = orc.gemm_f64(A, B, rows=rows)
    bad, worst = orc.check_tol(np.ascontiguousarray(C[rows]), T, S, TOL)
    assert bad == 0, f"{label}: {bad} row-sample violations (worst |d|/S = {worst:.3g})"
    T, S = orc.gemm_f64(A, B, cols=cols)
    bad2, worst2 = orc.check_tol(np.ascontiguousarray(C[:, cols]), T, S, TOL)
    assert bad2 == 0, f"{label}: {bad2} column-sample violations (worst |d|/S = {worst2:.3g})"
    return max(worst, worst2)


def _check_refkernel(orc, A, B, C, rows, cols, label):
    """Sampled rows and columns against the CPU restatement of the reference kernel's fp32
    arithmetic (K blocked 32 -> 16-deep steps, zero fill past K; mmm.cpp:1309-1356,
    mmmTensor.cpp:135-178), within the same BASELINE tolerance."""
    R = orc.gemm_refkernel_f32(A, B, rows=rows)
    _, S = orc.gemm_f64(A, B, rows=rows)
    d = np.abs(np.ascontiguousarray(C[rows]).astype(np.float64) - R)
    assert np.all(d <= TOL * S), f"{label}: rows vs reference-kernel math off by {np.max(d / S):.3g} of S"
    R = orc.gemm_refkernel_f32(A, B, cols=cols)
    _, S = orc.gemm_f64(A, B, cols=cols)
    d = np.abs(np.ascontiguousarray(C[:, cols]).astype(np.float64) - R)
    assert np.all(d <= TOL * S), f"{label}: columns vs reference-kernel math off by {np.max(d / S):.3g} of S"


def _check_checksums(A, B, C, label):
    A64 = A.astype(np.float64)
    B64 = B.astype(np.float64)
    C64 = C.astype(np.float64)
    r_true = A64 @ B64.sum(axis=1)
    r_bound = np.abs(A64) @ np.abs(B64).sum(axis=1)
    r_err = np.abs(C64.sum(axis=1) - r_true)
    assert np.all(r_err <= TOL * r_bound), f"{label}: row checksum off by {np.max(r_err / r_bound):.3g} of bound"
    c_true = A64.sum(axis=0) @ B64
    c_bound = np.abs(A64).sum(axis=0) @ np.abs(B64)
    c_err = np.abs(C64.sum(axis=0) - c_true)
    assert np.all(c_err <= TOL * c_bound), f"{label}: column checksum off by {np.max(c_err / c_bound):.3g} of bound"


def _sample(n, k, rng, must=()):
    s = set(int(x) for x in rng.choice(n, size=min(k, n), replace=False))
    s.update(int(m) % n for m in must)
    return np.array(sorted(s), dtype=np.int64)


# ------------------------------------------------------------------------------ configs
def test_config1_256_full(orc, mm, cuda):
    """C1: 256^3, U[-1,1], seed 0; every output vs fp64 and vs the reference-kernel restatement."""
    A = orc.uniform_f16((256, 256), 0, 0)
    B = orc.uniform_f16((256, 256), 0, 1)
    C = mm.gemm(to_dev(cuda, A), to_dev(cuda, B)).cpu().numpy()
    T, S = orc.gemm_f64(A, B)
    bad, worst = orc.check_tol(C, T, S, TOL)
    assert bad == 0, f"{bad} violations vs fp64 (worst {worst:.3g})"
    R = orc.gemm_refkernel_f32(A, B)
    assert np.all(np.abs(C.astype(np.float64) - R) <= TOL * S), "violations vs the reference kernel's fp32 math"
    N32 = orc.gemm_naive_f32(A, B)
    assert np.all(np.abs(C.astype(np.float64) - N32) <= TOL * S), "violations vs GEMM_Naive's fp32 math"


def test_config1_golden_record(mm, cuda):
    """C1's inputs from the on-device generator hash to the committed record, and the GEMM's
    sample outputs are within tolerance of the committed fp64 values."""
    import hashlib
    import json
    import os

    rec = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "c1_256.json")))
    A = cuda.empty((256, 256), dtype=cuda.float16, device="cuda")
    B = cuda.empty((256, 256), dtype=cuda.float16, device="cuda")
    mm.fill_uniform(A, 0, 0)
    mm.fill_uniform(B, 0, 1)
    h = lambda t: hashlib.sha256(t.cpu().numpy().view(np.uint16).tobytes()).hexdigest()
    assert h(A) == rec["sha256"]["A_f16_bits"] and h(B) == rec["sha256"]["B_f16_bits"]
    C = mm.gemm(A, B).cpu().numpy()
    _, S = mm.gemm_truth(A, B)
    S = S.cpu().numpy()
    for (i, j), key in [((0, 0), "C[0][0]"), ((255, 255), "C[255][255]"), ((17, 200), "C[17][200]")]:
        assert abs(float(C[i, j]) - rec["samples"][key]) <= TOL * S[i, j], key


def test_config2_8192_sampled(orc, mm, cuda):
    """C2: 8192^3, U[-1,1], seed 1; sampled rows/cols vs fp64, plus row/column checksums."""
    n = 8192
    A = orc.uniform_f16((n, n), 1, 0)
    B = orc.uniform_f16((n, n), 1, 1)
    C = mm.gemm(to_dev(cuda, A), to_dev(cuda, B))
    cuda.cuda.synchronize()
    C = C.cpu().numpy()
    rng = np.random.default_rng(11)
    rows = _sample(n, 24, rng, must=(0, 255, 256, n - 1))
    cols = _sample(n, 8, rng, must=(0, n - 1))
    _check_sampled(orc, A, B, C, rows, cols, "8192^3")
    _check_refkernel(orc, A, B, C, rows, cols, "8192^3")
    _check_checksums(A, B, C, "8192^3")


def test_config3_ragged(orc, mm, cuda):
    """C3: 4097 x 4095 x 4111 (no dimension a tile multiple, rows only 2-byte aligned), seed 2."""
    M, N, K = 4097, 4095, 4111
    A = orc.uniform_f16((M, K), 2, 0)
    B = orc.uniform_f16((K, N), 2, 1)
    Cd = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm(to_dev(cuda, A), to_dev(cuda, B), Cd)
    C = Cd.cpu().numpy()
    assert not np.isnan(C).any(), "unwritten outputs remain"
    rng = np.random.default_rng(12)
    rows = _sample(M, 20, rng, must=(0, 127, 128, 255, 256, M - 2, M - 1))
    cols = _sample(N, 12, rng, must=(0, 127, 128, N - 2, N - 1))
    _check_sampled(orc, A, B, C, rows, cols, "ragged")
    _check_refkernel(orc, A, B, C, rows, cols, "ragged")
    _check_checksums(A, B, C, "ragged")


def test_config4_contraction_baseline(orc, mm, cuda):
    """C4: C[b,i,j] = sum_{k,l} A[b,i,k,l] B[k,l,j], b=8 i=1024 k=32 l=64 j=2048, N(0,1)*0.1, seed 3."""
    b, i, k, l, j = 8, 1024, 32, 64, 2048
    A = orc.normal_f16((b, i, k, l), 3, 0, 0.1)
    B = orc.normal_f16((k, l, j), 3, 1, 0.1)
    desc = mm.contract_desc_baseline(b, i, k, l, j)
    Cd = cuda.full((b, i, j), float("nan"), dtype=cuda.float32, device="cuda")
    mm.contract(desc, to_dev(cuda, A), to_dev(cuda, B), Cd)
    C = Cd.cpu().numpy()
    rng = np.random.default_rng(13)
    bi = _sample(b * i, 24, rng, must=(0, i - 1, i, b * i - 1))
    T, S = orc.contract_baseline_f64(A, B, bi)  # 5-D loop nest, no fold
    Cs = np.ascontiguousarray(C.reshape(b * i, j)[bi])
    bad, worst = orc.check_tol(Cs, T, S, TOL)
    assert bad == 0, f"{bad} violations vs the 5-D loop nest (worst {worst:.3g})"
    # the second reference: the reference kernel's fp32 math on the folded GEMM (M = b*i, K = k*l)
    A2, B2, C2 = A.reshape(b * i, k * l), B.reshape(k * l, j), C.reshape(b * i, j)
    cols = _sample(j, 12, rng, must=(0, j - 1))
    _check_refkernel(orc, A2, B2, C2, bi, cols, "contraction")
    _check_checksums(A2, B2, C2, "contraction")


def test_config5_skinny_full(orc, mm, cuda):
    """C5: 16 x 8192 x 8192, U[-1,1], seed 4; every output vs fp64."""
    M, N, K = 16, 8192, 8192
    A = orc.uniform_f16((M, K), 4, 0)
    B = orc.uniform_f16((K, N), 4, 1)
    C = mm.gemm(to_dev(cuda, A), to_dev(cuda, B)).cpu().numpy()
    T, S = orc.gemm_f64(A, B)
    bad, worst = orc.check_tol(C, T, S, TOL)
    assert bad == 0, f"{bad} violations vs fp64 (worst {worst:.3g})"
    R = orc.gemm_refkernel_f32(A, B, cols=np.arange(0, N, 64))
    assert np.all(np.abs(C[:, ::64].astype(np.float64) - R) <= TOL * S[:, ::64])


# ------------------------------------------------------------------------------ exact / edges
EXACT_SHAPES = [
    (256, 256, 256),   # aligned, direct-to-LDS path, one tile
    (300, 264, 200),   # direct-to-LDS path with M/N edge tiles, K tail of 8
    (257, 129, 77),    # odd K and N: masked last K tile
    (513, 1000, 1032), # several tiles, K tail 8
    (33, 40, 16),      # smaller than one tile
    (1, 1, 1),
]


@pytest.mark.parametrize("shape", EXACT_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_exact_integer(mm, cuda, shape):
    M, N, K = shape
    rng = np.random.default_rng(M * 7919 + N * 31 + K)
    A, B, truth = _int_inputs(rng, M, N, K)
    C = mm.gemm(to_dev(cuda, A), to_dev(cuda, B)).cpu().numpy()
    assert np.array_equal(C, truth), f"max |diff| {np.abs(C - truth).max()}"


@pytest.mark.parametrize("tile", ["256x256", "128x256", "256x128", "128x128", "64x64", "192x192"])
@pytest.mark.parametrize("K", [264, 263])
def test_exact_every_tile(mm, cuda, tile, K):
    """Every instantiated tile, with whole K tiles (K=264) and a last K tile whose chunks across K
    and N are patched (K=263, odd N): the direct-to-LDS path (the register-staged one has its own
    test)."""
    M, N = 333, (520 if K % 8 == 0 else 517)
    rng = np.random.default_rng(K)
    A, B, truth = _int_inputs(rng, M, N, K)
    C = mm.gemm(to_dev(cuda, A), to_dev(cuda, B), tile=tile).cpu().numpy()
    assert np.array_equal(C, truth)


def _odd_copy(cuda, X):
    """X's bytes on the device at an odd byte address: (buffer, address).  fp16 data there can only
    be read by the register-staged kernels (the direct-to-LDS loads need 2-byte alignment)."""
    raw = np.ascontiguousarray(X).view(np.uint8).ravel()
    buf = cuda.zeros(raw.size + 1, dtype=cuda.uint8, device="cuda")
    buf[1:].copy_(cuda.from_numpy(raw))
    return buf, buf.data_ptr() + 1


@pytest.mark.parametrize("tile", [None, "256x256", "192x192", "128x256", "256x128", "128x128", "64x64"])
def test_exact_register_staged_path(mm, cuda, tile):
    """A and B at odd byte addresses: the planner sends them to the register-staged kernels
    (element-wise masked loads through VGPRs) on every tile; exact on integer inputs."""
    import ctypes as C

    M, N, K = 333, 517, 263
    assert mm.gemm_plan(M, N, K, A=3)["direct_to_lds"] == 0
    A, B, truth = _int_inputs(np.random.default_rng(263), M, N, K)
    abuf, pa = _odd_copy(cuda, A)
    bbuf, pb = _odd_copy(cuda, B)
    Cd = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    L = mm.lib()
    st = C.c_void_p(cuda.cuda.current_stream().cuda_stream)
    if tile is None:
        e = L.mmm_gemm_f16f32(C.c_void_p(pa), C.c_void_p(pb), C.c_void_p(Cd.data_ptr()), M, N, K, K, N, N, st)
    else:
        wm, wn, wi, wj = mm.TILES[tile]
        e = L.mmm_gemm_f16f32_tiled(C.c_void_p(pa), C.c_void_p(pb), C.c_void_p(Cd.data_ptr()), M, N, K, K, N, N,
                                    wm, wn, wi, wj, None, 0, st)
    assert e == 0
    got = Cd.cpu().numpy()
    del abuf, bbuf
    assert np.array_equal(got, truth), f"{int((got != truth).sum())} mismatches"


@pytest.mark.parametrize("tile", [None, "128x128"])
def test_exact_ragged_full_size(mm, cuda, tile):
    """The ragged configuration's shape with integer inputs: every output bit-exact.  Rows of
    A and B are only 2-byte aligned (unaligned direct-to-LDS loads) and the last K tile's chunks
    across K and N are patched.  fp64 BLAS is exact here (all partial sums below 2^53)."""
    M, N, K = 4097, 4095, 4111
    rng = np.random.default_rng(4111)
    A = rng.integers(-4, 5, size=(M, K)).astype(np.float16)
    B = rng.integers(-4, 5, size=(K, N)).astype(np.float16)
    truth = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    C = mm.gemm(to_dev(cuda, A), to_dev(cuda, B), tile=tile).cpu().numpy()
    assert np.array_equal(C, truth), f"{int((C != truth).sum())} mismatches"


TAIL_PADDING = [
    ((333, 517, 263, 5, 3), None),       # 64x64 tiles; chunks across K and across N in B's row K-1
    ((333, 517, 263, 5, 3), "256x256"),  # the same through every tile shape
    ((333, 517, 263, 5, 3), "192x192"),
    ((333, 517, 263, 5, 3), "256x128"),
    ((333, 517, 263, 5, 3), "128x256"),
    ((333, 517, 263, 5, 3), "128x128"),
    ((100, 300, 37, 3, 3), None),        # one K tile: the prologue publishes the patched tile
    ((333, 520, 264, 3, 0), "256x256"),  # unaligned rows, K and N multiples of 8: nothing to patch
    ((333, 517, 256, 3, 3), None),       # K a multiple of 64 (last tile full), B's chunk across N
    ((333, 517, 256, 3, 3), "256x256"),
    ((300, 1023, 1024, 0, 1), "192x192"),
    ((257, 129, 77, 5, 3), "256x256"),   # B rows narrower than the tile: gathered through VGPRs
    ((300, 40, 77, 5, 3), "64x64"),      # the same on the 64x64 tile (its loads go out together)
    ((2000, 40, 4097, 1, 1), None),      # ... with the K split of a small grid
    ((333, 517, 8191, 5, 3), None),      # 128x128 tiles split 16 ways: the last split patches
    ((1000, 777, 6151, 1, 1), None),     # a 4-way split of the partial last round
]


@pytest.mark.parametrize("case", TAIL_PADDING, ids=lambda c: "x".join(map(str, c[0])) + "-" + str(c[1]))
def test_exact_tail_padding(mm, cuda, case):
    """Rows of A and B padded past K and N with NaN (lda = K + pa, ldb = N + pb).  The last K
    tile's chunks across K read that padding (or the next row) before the kernel overwrites them
    from its gathered copy; a value left there would meet B's zero rows past K as NaN * 0.  The
    chunks across N in B's padding only reach columns that are never stored.  Exact on integer
    inputs."""
    (M, N, K, pa, pb), tile = case
    rng = np.random.default_rng(M + 5 * N + 11 * K)
    A, B, truth = _int_inputs(rng, M, N, K)
    Ap = np.full((M, K + pa), np.nan, dtype=np.float16)
    Ap[:, :K] = A
    Bp = np.full((K, N + pb), np.nan, dtype=np.float16)
    Bp[:, :N] = B
    Ad, Bd = to_dev(cuda, Ap), to_dev(cuda, Bp)
    C = mm.gemm(Ad[:, :K], Bd[:, :N], tile=tile).cpu().numpy()
    assert np.array_equal(C, truth), f"{int((C != truth).sum())} mismatches, {int(np.isnan(C).sum())} NaN"


@pytest.mark.parametrize("shape", [(300, 270, 1001), (129, 65, 2055), (64, 4100, 515)], ids=lambda s: "x".join(map(str, s)))
def test_exact_unaligned_rows(mm, cuda, shape):
    """Odd leading dimensions across many K tiles (unaligned direct-to-LDS rows)."""
    M, N, K = shape
    rng = np.random.default_rng(M + 3 * N + 7 * K)
    A, B, truth = _int_inputs(rng, M, N, K)
    C = mm.gemm(to_dev(cuda, A), to_dev(cuda, B)).cpu().numpy()
    assert np.array_equal(C, truth)


@pytest.mark.parametrize("shape", [(16, 8192, 8192), (5, 1000, 2000), (16, 96, 72), (1, 64, 8), (11, 520, 4104)],
                         ids=lambda s: "x".join(map(str, s)))
def test_exact_skinny(mm, cuda, shape):
    """M <= 16 runs on the streaming kernel's 16-row variant (fixed-order reductions)."""
    M, N, K = shape
    rng = np.random.default_rng(M * 13 + N + K)
    A = rng.integers(-4, 5, size=(M, K)).astype(np.float16)
    B = rng.integers(-4, 5, size=(K, N)).astype(np.float16)
    truth = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    Cd = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm(to_dev(cuda, A), to_dev(cuda, B), Cd)
    C = Cd.cpu().numpy()
    assert np.array_equal(C, truth), f"{int((C != truth).sum())} mismatches"


@pytest.mark.parametrize("shape", [(3, 1001, 777), (16, 4095, 4111), (9, 130, 2050), (1, 4095, 4111)],
                         ids=lambda s: "x".join(map(str, s)))
def test_exact_skinny_unaligned(mm, cuda, shape):
    """Streaming kernel on odd N/K (unaligned rows; last K slot gathered element-wise)."""
    M, N, K = shape
    rng = np.random.default_rng(M * 31 + N + 7 * K)
    A = rng.integers(-4, 5, size=(M, K)).astype(np.float16)
    B = rng.integers(-4, 5, size=(K, N)).astype(np.float16)
    truth = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    Cd = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm(to_dev(cuda, A), to_dev(cuda, B), Cd)
    C = Cd.cpu().numpy()
    assert np.array_equal(C, truth), f"{int((C != truth).sum())} mismatches"


@pytest.mark.parametrize("shape", [(16, 8192, 8192), (3, 1001, 777), (16, 4095, 4111), (9, 130, 2050),
                                   (1, 4095, 4111), (16, 96, 64), (5, 33, 8)],
                         ids=lambda s: "x".join(map(str, s)))
def test_exact_skinny_no_workspace(mm, cuda, shape):
    """M <= 16 without a workspace: one workgroup streams its column strip over all of K and
    reduces its waves' K ranges in LDS (aligned, odd N and K, gathered last slot)."""
    M, N, K = shape
    A, B, truth = _exact_case(np.random.default_rng(M * 7 + N + 3 * K), M, N, K)
    Cd = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm(to_dev(cuda, A), to_dev(cuda, B), Cd, workspace=False)
    C = Cd.cpu().numpy()
    assert np.array_equal(C, truth), f"{int((C != truth).sum())} mismatches"


@pytest.mark.parametrize("case", [
    (4095, 4111, 4095, 0, 0), (4096, 5120, 4096, 0, 0), (4096, 5121, 4096, 0, 0), (17, 1, 17, 0, 0),
    (9, 129, 9, 0, 0), (8, 8, 8, 0, 0), (7, 300, 8, 0, 0), (3, 50, 3, 0, 0), (4801, 2000, 4801, 1, 1),
    (4095, 4111, 4103, 1, 0), (16 * 300 + 5, 127, 16 * 300 + 8, 0, 1), (60000, 4096, 60000, 0, 0)],
    ids=lambda c: "N{}-K{}-ldb{}-A{}-B{}".format(*c))
@pytest.mark.parametrize("ws", [None, False], ids=["workspace", "no_workspace"])
def test_exact_one_row(mm, cuda, case, ws):
    """M = 1 (decode-shaped GEMV, the ragged configuration's remainder row) on the streaming
    kernels: N and K tails (odd K: A's last element shares a dword with the byte after A), B rows
    padded with NaN (ldb > N), A and B starting one element past a 16-byte boundary, N below one
    strip, several rounds of strips, with and without a workspace, C confined to its view.
    Integer inputs, bit-exact against the int64 product."""
    torch = cuda
    N, K, ldb, a_off, b_off = case
    rng = np.random.default_rng(N + 3 * K + ldb)
    A = rng.integers(-4, 5, size=(1, K)).astype(np.float16)
    B = rng.integers(-4, 5, size=(K, N)).astype(np.float16)
    truth = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32)
    Abuf = torch.zeros(K + a_off, dtype=torch.float16, device="cuda")
    Abuf[a_off:] = to_dev(torch, A)[0]
    Ad = Abuf[a_off:].view(1, K)
    Bbuf = torch.full((K * ldb + b_off,), float("nan"), dtype=torch.float16, device="cuda")
    Bd = Bbuf[b_off:].view(K, ldb)[:, :N]
    Bd.copy_(to_dev(torch, B))
    Cbuf = torch.full((N + 8,), -1.0, dtype=torch.float32, device="cuda")
    Cv = Cbuf[4:4 + N].view(1, N)
    print(f"[one_row] N={N} K={K} ldb={ldb} A+{a_off} B+{b_off} ws={ws is None} plan {mm.gemm_plan(1, N, K, ldb=ldb)}",
          flush=True)
    mm.gemm(Ad, Bd, Cv, workspace=ws)
    torch.cuda.synchronize()
    Cb = Cbuf.cpu().numpy()
    assert np.all(Cb[:4] == -1.0) and np.all(Cb[4 + N:] == -1.0), "wrote outside the C view"
    C = Cb[4:4 + N].reshape(1, N)
    assert np.array_equal(C, truth), f"{int((C != truth).sum())} mismatches"


@pytest.mark.parametrize("shape", [(16 * 256 + 1, 4096, 264), (16 * 256 + 40, 4096, 264), (16 * 256 + 64, 4096, 1000),
                                   (16 * 256 + 17, 4095, 523)],
                         ids=lambda s: "x".join(map(str, s)))
def test_exact_row_remainder_split(mm, cuda, shape):
    """M = 256*k + r (r <= 64): the r rows run on the streaming kernel, the rest on the tile kernel."""
    M, N, K = shape
    plan = mm.gemm_plan(M, N, K)
    assert plan["kernel"] == "tile+stream" and plan["stream_rows"] == M % 256
    rng = np.random.default_rng(M + N + K)
    A = rng.integers(-4, 5, size=(M, K)).astype(np.float16)
    B = rng.integers(-4, 5, size=(K, N)).astype(np.float16)
    truth = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    Cd = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm(to_dev(cuda, A), to_dev(cuda, B), Cd)
    C = Cd.cpu().numpy()
    assert np.array_equal(C, truth), f"{int((C != truth).sum())} mismatches"


def _exact_case(rng, M, N, K):
    A = rng.integers(-4, 5, size=(M, K)).astype(np.float16)
    B = rng.integers(-4, 5, size=(K, N)).astype(np.float16)
    return A, B, (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)


# (M, N, K) -> K ranges the streaming kernel reduces across workgroups (0: within one workgroup),
# columns per workgroup strip
STREAM_SPLITS = [((16, 8192, 8192), 8, 256), ((1, 16384, 8192), 4, 256), ((13, 8200, 8192), 7, 256),
                 ((9, 8200, 8197), 7, 256), ((7, 16384, 4096), 2, 128), ((16, 4096, 8192), 8, 128),
                 ((5, 1024, 8192), 16, 128), ((16, 32768, 512), 1, 128), ((3, 2000, 4000), 15, 128),
                 ((16, 4095, 4111), 0, 32), ((16, 6001, 4111), 0, 32), ((16, 8191, 4111), 4, 128),
                 ((16, 2047, 4111), 16, 128), ((1, 130, 9000), 16, 128), ((16, 8192, 256), 0, 32), ((2, 264, 200), 0, 32)]


@pytest.mark.parametrize("case", STREAM_SPLITS, ids=lambda c: "x".join(map(str, c[0])) + f"-s{c[1]}-n{c[2]}")
def test_exact_stream_splits(mm, cuda, case):
    """The streaming kernel at every K-split count and strip width (256-column strips with a
    ragged last strip and a gathered K tail among them), the unsplit wide launch and the
    in-workgroup split; exact against int64 (the partial sums are integers, so any order is
    exact)."""
    (M, N, K), splits, cols = case
    plan = mm.gemm_plan(M, N, K)
    assert plan["stream_splits"] == splits and plan["stream_columns"] == cols
    A, B, truth = _exact_case(np.random.default_rng(M * 7 + N + K), M, N, K)
    Cd = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm(to_dev(cuda, A), to_dev(cuda, B), Cd)
    C = Cd.cpu().numpy()
    assert np.array_equal(C, truth), f"{int((C != truth).sum())} mismatches"


# 17 <= M <= 64: 32- and 64-row variants of the split streaming kernel -> K splits, columns per strip
STREAM_ROWS = [((17, 8192, 8192), 4, 128), ((24, 14336, 4096), 2, 128), ((32, 4095, 4111), 8, 128),
               ((33, 1000, 3000), 11, 128), ((48, 130, 9000), 16, 128), ((64, 8192, 1024), 4, 128),
               ((63, 28672, 512), 1, 128), ((40, 128, 64), 1, 128), ((64, 264, 200), 1, 128),
               ((57, 777, 1031), 4, 128), ((20, 16384, 8192), 4, 256), ((29, 16200, 8195), 4, 256),
               ((57, 16200, 9001), 4, 256), ((40, 8192, 16384), 8, 256), ((61, 16520, 8195), 3, 256)]


@pytest.mark.parametrize("case", STREAM_ROWS, ids=lambda c: "x".join(map(str, c[0])) + f"-s{c[1]}-n{c[2]}")
def test_exact_stream_rows(mm, cuda, case):
    """Up to 64 rows on the streaming kernel (two or four 16-row groups sharing every B
    fragment), split and unsplit, aligned and gathered tails, 256-column strips for 17-64 rows
    (with ragged last strips and gathered K tails; 64 rows sum their partials in two passes):
    exact against int64."""
    (M, N, K), splits, cols = case
    plan = mm.gemm_plan(M, N, K)
    assert plan["kernel"] == "stream" and plan["stream_splits"] == splits and plan["stream_columns"] == cols
    A, B, truth = _exact_case(np.random.default_rng(M * 5 + N + 3 * K), M, N, K)
    Cd = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm(to_dev(cuda, A), to_dev(cuda, B), Cd)
    C = Cd.cpu().numpy()
    assert np.array_equal(C, truth), f"{int((C != truth).sum())} mismatches"


def test_stream_split_repeat_and_resize(mm, cuda):
    """Shapes with different strip and split counts alternate on one stream and reuse one
    per-stream workspace (no clearing between calls); every call stays exact."""
    rng = np.random.default_rng(5)
    cases = [_exact_case(rng, *shp) for shp in [(16, 8192, 2048), (4, 1024, 4096), (16, 4096, 1024)]]
    dev = [(to_dev(cuda, A), to_dev(cuda, B), truth) for A, B, truth in cases]
    for _ in range(3):
        for A, B, truth in dev:
            assert np.array_equal(mm.gemm(A, B).cpu().numpy(), truth)


def test_stream_split_concurrent_streams(mm, cuda):
    """Two streams run split launches at the same time; each stream has its own workspace."""
    rng = np.random.default_rng(6)
    A1, B1, t1 = _exact_case(rng, 16, 8192, 4096)
    A2, B2, t2 = _exact_case(rng, 8, 8192, 4096)
    A1, B1, A2, B2 = (to_dev(cuda, x) for x in (A1, B1, A2, B2))
    s1, s2 = cuda.cuda.Stream(), cuda.cuda.Stream()
    outs = []
    cuda.cuda.synchronize()
    for _ in range(4):
        with cuda.cuda.stream(s1):
            C1 = mm.gemm(A1, B1)
        with cuda.cuda.stream(s2):
            C2 = mm.gemm(A2, B2)
        outs.append((C1, C2))
    cuda.cuda.synchronize()
    for C1, C2 in outs:
        assert np.array_equal(C1.cpu().numpy(), t1)
        assert np.array_equal(C2.cpu().numpy(), t2)


@pytest.mark.parametrize("rows", [16, 40])
@pytest.mark.parametrize("ws", [None, False], ids=["workspace", "no-workspace"])
def test_stream_graph_capture(mm, cuda, rows, ws):
    """Captured into a HIP graph, with the wrapper's per-stream workspace (the K split) or none
    (the in-workgroup kernel for 16 rows, one K range per workgroup for 40); every replay, with
    eager work in between, matches eager."""
    rng = np.random.default_rng(8)
    A, B, truth = _exact_case(rng, rows, 8192, 2048)
    A, B = to_dev(cuda, A), to_dev(cuda, B)
    C = cuda.full((rows, 8192), float("nan"), dtype=cuda.float32, device="cuda")
    g = cuda.cuda.CUDAGraph()
    with cuda.cuda.graph(g):
        mm.gemm(A, B, C, workspace=ws)
    for i in range(3):
        C.fill_(float("nan"))
        g.replay()
        cuda.cuda.synchronize()
        assert np.array_equal(C.cpu().numpy(), truth), f"replay {i}"
        assert np.array_equal(mm.gemm(A, B).cpu().numpy(), truth)


@pytest.mark.parametrize("shape", [(2048, 2048, 2048), (8192, 4096, 512), (1024, 1024, 8192), (3000, 3070, 1031)],
                         ids=lambda s: "x".join(map(str, s)))
def test_tile_graph_capture(mm, cuda, shape):
    """The tile kernels' store paths captured into a HIP graph: one round with write-through
    whole-line stores (2048^3), a persistent grid with non-temporal whole-line stores (8192 x 4096
    x 512, two rounds), a K split with write-through partial tiles and the reduction launch
    (1024^2 x 8192), and the 192x192 tile with edge tiles (3000 x 3070 x 1031).  Every replay, with
    eager work and synchronisation in between, equals the eager result bit for bit."""
    M, N, K = shape
    A = cuda.empty((M, K), dtype=cuda.float16, device="cuda")
    B = cuda.empty((K, N), dtype=cuda.float16, device="cuda")
    mm.fill_uniform(A, 11, 0)
    mm.fill_uniform(B, 11, 1)
    eager = mm.gemm(A, B)
    C = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    g = cuda.cuda.CUDAGraph()
    with cuda.cuda.graph(g):
        mm.gemm(A, B, C)
    for i in range(3):
        C.fill_(float("nan"))
        g.replay()
        cuda.cuda.synchronize()
        assert cuda.equal(C, eager), f"replay {i}"
        assert cuda.equal(mm.gemm(A, B), eager)


# shapes whose launch splits K: streaming (16 and 40 rows), one small round of tiles, a partly
# filled last round (with a masked K tail), and the 128x128 tile
WS_SHAPES = [(16, 8192, 2048), (40, 4096, 4096), (1024, 1024, 8192), (4357, 4095, 8191), (300, 264, 4096)]


@pytest.mark.parametrize("shape", WS_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_workspace_entry_point(mm, cuda, shape):
    """mmm_gemm_f16f32_ws through the C ABI: a workspace of the queried size (K split), one
    byte short and none (both unsplit) all give exact results, and nothing past the queried
    size is written."""
    M, N, K = shape
    A, B, truth = _exact_case(np.random.default_rng(M + 2 * N + K), M, N, K)
    A, B = to_dev(cuda, A), to_dev(cuda, B)
    L = mm.lib()
    st = C.c_void_p(cuda.cuda.current_stream().cuda_stream)
    need = C.c_size_t(0)
    Cd = cuda.empty((M, N), dtype=cuda.float32, device="cuda")
    assert L.mmm_gemm_workspace_f16f32(A.data_ptr(), B.data_ptr(), Cd.data_ptr(), M, N, K, K, N, N,
                                       C.byref(need)) == 0
    assert need.value > 0
    guard = 4096
    ws = cuda.full((need.value + guard,), 0x5A, dtype=cuda.uint8, device="cuda")
    for nbytes in (need.value, need.value - 1, 0):
        Cd.fill_(float("nan"))
        ptr = C.c_void_p(ws.data_ptr()) if nbytes else None
        assert L.mmm_gemm_f16f32_ws(A.data_ptr(), B.data_ptr(), Cd.data_ptr(), M, N, K, K, N, N, ptr, nbytes, st) == 0
        got = Cd.cpu().numpy()
        assert np.array_equal(got, truth), f"workspace {nbytes} of {need.value}: {int((got != truth).sum())} mismatches"
        assert bool((ws[need.value:] == 0x5A).all()), "wrote past the queried workspace size"


# (M, N, K, C row padding): whole interior 256x256 (or 192x192) tiles over several rounds run on the
# persistent kernel (256 workgroups looping over tiles, next tile's loads issued before this tile's stores)
PERSISTENT = [(8192, 8192, 8192, 0), (8192, 8192, 2048, 0), (4608, 4096, 192, 0), (2560, 16384, 1024, 0),
              (4608, 4096, 576, 3), (6144, 6144, 2048, 0), (3072, 6144, 1024, 3)]


@pytest.mark.parametrize("case", PERSISTENT, ids=lambda c: "x".join(map(str, c[:3])) + f"-pad{c[3]}")
def test_exact_persistent(mm, cuda, case):
    """The persistent tile kernel (256x256 tiles, and 192x192 in the last two cases): exact against
    the on-device fp64 truth (integer inputs), three calls in a row, with padded C row strides."""
    M, N, K, pad = case
    plan = mm.gemm_plan(M, N, K, ldc=N + pad)
    assert plan["kernel"] == "tile" and plan["tile_persistent"] == 1
    g = cuda.Generator(device="cuda").manual_seed(M + N + K + pad)
    A = cuda.randint(-4, 5, (M, K), device="cuda", generator=g).half()
    B = cuda.randint(-4, 5, (K, N), device="cuda", generator=g).half()
    T, _ = mm.gemm_truth(A, B, with_scale=False)
    for _ in range(3):
        Cbuf = cuda.full((M, N + pad), float("nan"), dtype=cuda.float32, device="cuda")
        C = Cbuf[:, :N]
        mm.gemm(A, B, C)
        assert cuda.equal(C.double(), T), f"{int((C.double() != T).sum())} mismatches"
        if pad:
            assert bool(cuda.isnan(Cbuf[:, N:]).all()), "wrote past the row"


# (M, N, K) -> (tile, K splits, split tiles): the last round of 256 workgroups is less than half
# full, so its tiles run as K ranges while the rest run over all of K (0 split tiles: declined,
# the reduction would cost more than the round it saves)
TAIL_SPLITS = [((6144, 6144, 4096), ("256x256", 4, 64)), ((1792, 5120, 8192), ("256x128", 10, 24)),
               ((1408, 6656, 8192), ("128x256", 8, 30)), ((1344, 7168, 4096), ("192x192", 8, 10)),
               ((4608, 4608, 8192), ("256x256", 3, 68)), ((7168, 7168, 7168), ("256x256", 14, 16)),
               ((4357, 4095, 8191), ("256x256", 8, 32)), ((2304, 2304, 8192), ("256x256", 3, 81)),
               ((6150, 6144, 1030), ("256x256", 1, 0))]


@pytest.mark.parametrize("shape", [(3072, 3072, 3072), (3072, 3072, 8192), (3000, 3070, 1031)],
                         ids=lambda s: "x".join(map(str, s)))
def test_exact_192_full_round(mm, cuda, shape):
    """Shapes the library runs as one round of 192x192 tiles (16 x 16 of them at 3072^2; edges
    and a masked K tail in the last case): exact against the on-device fp64 truth."""
    M, N, K = shape
    plan = mm.gemm_plan(M, N, K)
    assert (plan["kernel"], plan["block_m"], plan["block_n"], plan["tile_splits"]) == ("tile", 192, 192, 1)
    g = cuda.Generator(device="cuda").manual_seed(M + N + K)
    A = cuda.randint(-4, 5, (M, K), device="cuda", generator=g).half()
    B = cuda.randint(-4, 5, (K, N), device="cuda", generator=g).half()
    T, _ = mm.gemm_truth(A, B, with_scale=False)
    for _ in range(2):
        C = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
        mm.gemm(A, B, C)
        assert cuda.equal(C.double(), T), f"{int((C.double() != T).sum())} mismatches"


@pytest.mark.parametrize("case", TAIL_SPLITS, ids=lambda c: "x".join(map(str, c[0])))
def test_exact_tail_split(mm, cuda, case):
    """Whole tiles and K-split last-round tiles in one launch, then the ordered reduction: exact
    against the on-device fp64 truth (integer inputs; every partial sum is exact), twice."""
    (M, N, K), (tile, splits, split_tiles) = case
    plan = mm.gemm_plan(M, N, K)
    assert plan["kernel"] == "tile" and f"{plan['block_m']}x{plan['block_n']}" == tile
    assert (plan["tile_splits"], plan["tile_split_tiles"]) == (splits, split_tiles)
    g = cuda.Generator(device="cuda").manual_seed(M + N + K)
    A = cuda.randint(-4, 5, (M, K), device="cuda", generator=g).half()
    B = cuda.randint(-4, 5, (K, N), device="cuda", generator=g).half()
    T, _ = mm.gemm_truth(A, B, with_scale=False)
    for _ in range(2):
        C = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
        mm.gemm(A, B, C)
        assert cuda.equal(C.double(), T), f"{int((C.double() != T).sum())} mismatches"


# (M, N, K, tile or None) -> K splits of the tile kernel
TILE_SPLITS = [((1024, 1024, 8192, None), 4), ((65, 4096, 4096, None), 8), ((300, 264, 2048, "128x128"), 4),
               ((65, 128, 4096, None), 8), ((100, 200, 3000, "64x64"), 5), ((400, 500, 3000, "192x192"), 5),
               ((100, 200, 1001, None), 1), ((256, 512, 4096, "256x256"), 8), ((256, 512, 2048, "256x128"), 4),
               ((200, 300, 3000, "128x256"), 5), ((2000, 2000, 512, None), 1)]


@pytest.mark.parametrize("case", TILE_SPLITS, ids=lambda c: "x".join(map(str, c[0][:3])) + f"-{c[0][3]}-s{c[1]}")
def test_exact_tile_splits(mm, cuda, case):
    """K split across workgroups on every tile (and with a masked last K tile): exact."""
    (M, N, K, tile), splits = case
    if tile is None:
        assert mm.gemm_plan(M, N, K)["tile_splits"] == splits
    A, B, truth = _exact_case(np.random.default_rng(M + 3 * N + K), M, N, K)
    Cd = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm(to_dev(cuda, A), to_dev(cuda, B), Cd, tile=tile)
    C = Cd.cpu().numpy()
    assert np.array_equal(C, truth), f"{int((C != truth).sum())} mismatches"


# Grids of several rounds of workgroups, on every tile, with row/column edges and a K tail.
LARGE_GRIDS = [((8192, 4096, 128), "256x256"), ((8190, 4104, 200), "256x256"), ((8192, 4096, 520), "256x128"),
           ((4096, 8192, 64), "128x256"), ((4096, 4096, 192), "128x128"), ((4000, 4100, 136), "128x128"),
           ((2048, 2048, 192), "64x64"), ((2000, 1100, 136), "64x64"), ((6144, 3072, 192), "192x192"),
           ((4000, 4100, 136), "192x192")]


@pytest.mark.parametrize("case", LARGE_GRIDS, ids=lambda c: "x".join(map(str, c[0])) + "-" + c[1])
def test_exact_large_grids(mm, cuda, case):
    """Multi-round tile grids on every tile: exact on integer inputs."""
    (M, N, K), tile = case
    A, B, truth = _exact_case(np.random.default_rng(M + N + 5 * K), M, N, K)
    Cd = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm(to_dev(cuda, A), to_dev(cuda, B), Cd, tile=tile)
    C = Cd.cpu().numpy()
    assert np.array_equal(C, truth), f"{int((C != truth).sum())} mismatches"


@pytest.mark.parametrize("pad", [1, 2, 3])
@pytest.mark.parametrize("case", [((1000, 1999, 777), None), ((4097, 1000, 520), "256x256"),
                                  ((513, 700, 1032), "128x256"), ((700, 300, 4000), None)],
                         ids=lambda c: "x".join(map(str, c[0])) + f"-{c[1]}")
def test_exact_c_row_alignment(mm, cuda, case, pad):
    """C rows only 4-byte aligned (ldc = N + pad): 16-byte stores of unaligned rows, on the
    tile epilogue and the split reduction; nothing outside the [M][N] window is written."""
    (M, N, K), tile = case
    A, B, truth = _exact_case(np.random.default_rng(M + N + K + pad), M, N, K)
    Cw = cuda.full((M, N + pad), float("nan"), dtype=cuda.float32, device="cuda")
    mm.gemm(to_dev(cuda, A), to_dev(cuda, B), Cw[:, :N], tile=tile)
    C = Cw.cpu().numpy()
    assert np.array_equal(C[:, :N], truth), f"{int((C[:, :N] != truth).sum())} mismatches"
    assert np.isnan(C[:, N:]).all(), "wrote outside the [M][N] window"


def test_tile_split_deterministic_and_graph(mm, cuda, orc):
    """A split launch is bitwise reproducible, and a captured graph's replays match it."""
    A = to_dev(cuda, orc.uniform_f16((1024, 8192), 9, 0))
    B = to_dev(cuda, orc.uniform_f16((8192, 1024), 9, 1))
    C1 = mm.gemm(A, B).cpu().numpy()
    C2 = mm.gemm(A, B).cpu().numpy()
    assert np.array_equal(C1.view(np.uint32), C2.view(np.uint32))
    C = cuda.full((1024, 1024), float("nan"), dtype=cuda.float32, device="cuda")
    g = cuda.cuda.CUDAGraph()
    with cuda.cuda.graph(g):
        mm.gemm(A, B, C)
    T, S = mm.gemm_truth(A, B)
    for i in range(3):
        C.fill_(float("nan"))
        g.replay()
        cuda.cuda.synchronize()
        d = (C.double() - T).abs()
        assert bool((d <= 1e-3 * S).all()), f"replay {i}"


def test_concurrent_host_threads(mm, cuda):
    """Six host threads, each with its own stream, issue split launches (tile K splits, the
    streaming split, the tile+stream split) at the same time (ctypes releases the GIL during a
    call, so the calls overlap inside the library): each stream gets its own workspace, results
    exact.  (mmm_gemm_f16f32_noalloc is left out: its calls share one scratch array per GPU, and
    overlapping calls on one GPU race by contract.)"""
    import threading

    rng = np.random.default_rng(12)
    cases = [_exact_case(rng, *shp) for shp in [(16, 8192, 2048), (1024, 512, 4096), (8, 4096, 4096), (300, 264, 4096),
                                                (4097, 512, 300), (2304, 2304, 1024)]]
    dev = [(to_dev(cuda, A), to_dev(cuda, B), truth) for A, B, truth in cases]
    results, errors = {}, []

    def worker(i):
        try:
            A, B, _ = dev[i]
            s = cuda.cuda.Stream()
            outs = []
            with cuda.cuda.stream(s):
                for _ in range(3):
                    outs.append(mm.gemm(A, B))
            s.synchronize()
            results[i] = [o.cpu().numpy() for o in outs]
        except Exception as e:  # reported below
            errors.append(repr(e))

    cuda.cuda.synchronize()
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(dev))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i, (_, _, truth) in enumerate(dev):
        for o in results[i]:
            assert np.array_equal(o, truth)


def test_skinny_deterministic(mm, cuda, orc):
    A = to_dev(cuda, orc.uniform_f16((16, 8192), 4, 0))
    B = to_dev(cuda, orc.uniform_f16((8192, 8192), 4, 1))
    C1 = mm.gemm(A, B).cpu().numpy()
    C2 = mm.gemm(A, B).cpu().numpy()
    assert np.array_equal(C1.view(np.uint32), C2.view(np.uint32))


def test_identity(mm, cuda, orc):
    """A = I gives C = float(B) exactly."""
    n = 384
    A = np.eye(n, dtype=np.float16)
    B = orc.uniform_f16((n, 640), 5, 1)
    C = mm.gemm(to_dev(cuda, A), to_dev(cuda, B)).cpu().numpy()
    assert np.array_equal(C, B.astype(np.float32))


def test_all_ones(mm, cuda):
    """All-ones inputs give C = K exactly."""
    M, N, K = 200, 300, 4100
    A = np.ones((M, K), dtype=np.float16)
    B = np.ones((K, N), dtype=np.float16)
    C = mm.gemm(to_dev(cuda, A), to_dev(cuda, B)).cpu().numpy()
    assert np.all(C == K)


def test_leading_dimensions(mm, cuda):
    """Sub-matrix views: padded lda/ldb/ldc (aligned and unaligned) and a misaligned base."""
    rng = np.random.default_rng(5)
    M, N, K = 190, 270, 136
    A, B, truth = _int_inputs(rng, M, N, K)
    for pad_a, pad_b, off in [(8, 10, 0), (3, 5, 0), (8, 10, 1)]:
        Abig = np.zeros((M, K + pad_a + off), dtype=np.float16)
        Abig[:, off:off + K] = A
        Bbig = np.zeros((K, N + pad_b), dtype=np.float16)
        Bbig[:, :N] = B
        Ad = to_dev(cuda, Abig)[:, off:off + K]
        Bd = to_dev(cuda, Bbig)[:, :N]
        Cbig = cuda.full((M, N + 7), -1.0, dtype=cuda.float32, device="cuda")
        mm.gemm(Ad, Bd, Cbig[:, :N])
        C = Cbig.cpu().numpy()
        assert np.array_equal(C[:, :N], truth), f"pads {pad_a},{pad_b} offset {off}"
        assert np.all(C[:, N:] == -1.0), "wrote outside the C view"


def test_degenerate_sizes(mm, cuda):
    A = cuda.zeros((5, 0), dtype=cuda.float16, device="cuda")
    B = cuda.zeros((0, 7), dtype=cuda.float16, device="cuda")
    C = cuda.full((5, 7), 3.0, dtype=cuda.float32, device="cuda")
    mm.gemm(A, B, C)
    assert (C.cpu() == 0).all(), "K == 0 must write zeros"
    A = cuda.zeros((0, 9), dtype=cuda.float16, device="cuda")
    B = cuda.zeros((9, 4), dtype=cuda.float16, device="cuda")
    C = mm.gemm(A, B)
    assert C.shape == (0, 4)


def test_invalid_arguments(mm, cuda):
    import ctypes as C

    L = mm.lib()
    null = C.c_void_p(0)
    assert L.mmm_gemm_f16f32(null, null, null, 4, 4, 4, 4, 4, 4, null) == mm.HIP_ERROR_INVALID_VALUE
    A = cuda.zeros((4, 4), dtype=cuda.float16, device="cuda")
    Cd = cuda.zeros((4, 4), dtype=cuda.float32, device="cuda")
    p = C.c_void_p(A.data_ptr())
    assert L.mmm_gemm_f16f32(p, p, C.c_void_p(Cd.data_ptr()), 4, 4, 4, 3, 4, 4, null) == mm.HIP_ERROR_INVALID_VALUE
    assert L.mmm_gemm_f16f32(p, p, C.c_void_p(Cd.data_ptr()), -1, 4, 4, 4, 4, 4, null) == mm.HIP_ERROR_INVALID_VALUE
    assert L.mmm_gemm_f16f32_tiled(p, p, C.c_void_p(Cd.data_ptr()), 4, 4, 4, 4, 4, 4, 2, 2, 4, 4, null, 0, null) == \
        mm.HIP_ERROR_INVALID_VALUE


# ------------------------------------------------------------------------------ contractions
def test_contraction_baseline_exact(mm, cuda):
    b, i, k, l, j = 2, 33, 3, 40, 70
    rng = np.random.default_rng(21)
    A = rng.integers(-4, 5, size=(b, i, k, l)).astype(np.float16)
    B = rng.integers(-4, 5, size=(k, l, j)).astype(np.float16)
    truth = np.einsum("bikl,klj->bij", A.astype(np.int64), B.astype(np.int64)).astype(np.float32)
    C = cuda.full((b, i, j), float("nan"), dtype=cuda.float32, device="cuda")
    mm.contract(mm.contract_desc_baseline(b, i, k, l, j), to_dev(cuda, A), to_dev(cuda, B), C)
    assert np.array_equal(C.cpu().numpy(), truth)


@pytest.mark.parametrize("dims", [(4, 40, 8, 3, 24), (3, 130, 32, 5, 16)], ids=lambda d: "x".join(map(str, d)))
def test_contraction_reference_layout_exact(mm, cuda, orc, dims):
    """Reference layout Out[m][b][r] = sum_{n,l} G[r][n][m][l] In[b][n][l] (mmmTensor.cpp)."""
    mt, bt, rt, nt, rt_l = dims
    rng = np.random.default_rng(sum(dims))
    G = rng.integers(-4, 5, size=(rt, nt, mt, rt_l)).astype(np.float16)
    In = rng.integers(-4, 5, size=(bt, nt, rt_l)).astype(np.float16)
    truth = np.einsum("rnml,bnl->mbr", G.astype(np.int64), In.astype(np.int64)).astype(np.float32)
    Out = cuda.full((mt, bt, rt), float("nan"), dtype=cuda.float32, device="cuda")
    mm.contract(mm.contract_desc_reference(mt, bt, rt, nt, rt_l), to_dev(cuda, G), to_dev(cuda, In), Out)
    got = Out.cpu().numpy()
    assert np.array_equal(got, truth)
    # the same numbers as the reference's own route: host pack + TN GEMM + remap
    hA = orc.pack_reference_G(G).astype(np.int64)
    gemm = hA @ In.reshape(bt, nt * rt_l).astype(np.int64).T  # [(m*rt+r)][b]
    assert np.array_equal(got, gemm.reshape(mt, rt, bt).transpose(0, 2, 1).astype(np.float32))


# bt = 301 and 258: n_lo = bt not a multiple of 4, so the epilogue stores element by element;
# rt = 6: rows of 6; 32 x 8448 x 64: 264 tiles of 256 x 256 (two rounds, the second partly filled)
@pytest.mark.parametrize("dims", [(8, 300, 64, 3, 128), (4, 520, 32, 2, 64), (8, 301, 64, 3, 128), (4, 258, 32, 2, 64),
                                  (8, 300, 6, 3, 128), (32, 8448, 64, 2, 64)],
                         ids=lambda d: "x".join(map(str, d)))
def test_contraction_reference_layout_dma_exact(mm, cuda, orc, dims):
    """Reference layout on the direct-to-LDS fold path (K tiles inside one n block): bit-exact."""
    mt, bt, rt, nt, rt_l = dims
    rng = np.random.default_rng(sum(dims) + 1)
    G = rng.integers(-4, 5, size=(rt, nt, mt, rt_l)).astype(np.float16)
    In = rng.integers(-4, 5, size=(bt, nt, rt_l)).astype(np.float16)
    hA = orc.pack_reference_G(G).astype(np.float64)
    truth = (hA @ In.reshape(bt, nt * rt_l).astype(np.float64).T).reshape(mt, rt, bt).transpose(0, 2, 1)
    Out = cuda.full((mt, bt, rt), float("nan"), dtype=cuda.float32, device="cuda")
    mm.contract(mm.contract_desc_reference(mt, bt, rt, nt, rt_l), to_dev(cuda, G), to_dev(cuda, In), Out)
    assert np.array_equal(Out.cpu().numpy(), truth.astype(np.float32))


# rt_l a multiple of 8 but not of 64 (K tiles cross n blocks; each lane tracks its own chunk's
# block): rt_l = 8 crosses eight blocks per K tile, 200 at most one; bt = 301 stores element by
# element; rt = 6 rows of 6; 32 x 8448 x 64 runs two rounds of tiles.  The last five end K
# inside the last K tile (K = 120, 24 -- one partial tile --, 360, 200 with a single n block,
# and 72)
@pytest.mark.parametrize("dims", [(8, 300, 64, 24, 8), (4, 520, 32, 8, 24), (8, 301, 64, 8, 40), (8, 300, 6, 8, 120),
                                  (32, 8448, 64, 8, 72), (8, 300, 64, 8, 200), (8, 300, 64, 5, 24), (8, 301, 64, 3, 8),
                                  (32, 8448, 64, 3, 120), (8, 300, 6, 1, 200), (4, 40, 8, 3, 24)],
                         ids=lambda d: "x".join(map(str, d)))
def test_contraction_reference_layout_lane_k_exact(mm, cuda, orc, dims):
    """Reference layout on the direct-to-LDS fold path with per-lane K blocks: bit-exact."""
    mt, bt, rt, nt, rt_l = dims
    assert rt_l % 8 == 0 and rt_l % 64
    rng = np.random.default_rng(sum(dims) + 2)
    G = rng.integers(-4, 5, size=(rt, nt, mt, rt_l)).astype(np.float16)
    In = rng.integers(-4, 5, size=(bt, nt, rt_l)).astype(np.float16)
    hA = orc.pack_reference_G(G).astype(np.float64)
    truth = (hA @ In.reshape(bt, nt * rt_l).astype(np.float64).T).reshape(mt, rt, bt).transpose(0, 2, 1)
    Out = cuda.full((mt, bt, rt), float("nan"), dtype=cuda.float32, device="cuda")
    mm.contract(mm.contract_desc_reference(mt, bt, rt, nt, rt_l), to_dev(cuda, G), to_dev(cuda, In), Out)
    assert np.array_equal(Out.cpu().numpy(), truth.astype(np.float32))


# Folds off the direct-to-LDS path, on the register-staged kernel's grouped gathers: rt_l = 100,
# 50 and 25 give groups of 4, 2 and 1 elements; G or Input placed 4 or 2 elements into its buffer
# narrows the group by its alignment (G 8-byte aligned: groups of 4 for A, 8 for Input)
@pytest.mark.parametrize("dims,g_off,in_off", [((8, 300, 64, 3, 100), 0, 0), ((8, 301, 64, 3, 50), 0, 0),
                                               ((4, 258, 32, 3, 25), 0, 0), ((8, 300, 64, 3, 128), 4, 0),
                                               ((8, 300, 64, 3, 100), 0, 2), ((32, 8448, 64, 2, 100), 0, 0)],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_contraction_reference_layout_gathers_exact(mm, cuda, orc, dims, g_off, in_off):
    """Reference layout on the register-staged fold kernel (grouped gathers): bit-exact."""
    mt, bt, rt, nt, rt_l = dims
    rng = np.random.default_rng(sum(dims) + 3 + g_off + in_off)
    G = rng.integers(-4, 5, size=(rt, nt, mt, rt_l)).astype(np.float16)
    In = rng.integers(-4, 5, size=(bt, nt, rt_l)).astype(np.float16)
    hA = orc.pack_reference_G(G).astype(np.float64)
    truth = (hA @ In.reshape(bt, nt * rt_l).astype(np.float64).T).reshape(mt, rt, bt).transpose(0, 2, 1)
    Gbuf = to_dev(cuda, np.concatenate([np.zeros(g_off, np.float16), G.ravel()]))
    Ibuf = to_dev(cuda, np.concatenate([np.zeros(in_off, np.float16), In.ravel()]))
    Gd = Gbuf[g_off:].view(rt, nt, mt, rt_l)
    Id = Ibuf[in_off:].view(bt, nt, rt_l)
    Out = cuda.full((mt, bt, rt), float("nan"), dtype=cuda.float32, device="cuda")
    mm.contract(mm.contract_desc_reference(mt, bt, rt, nt, rt_l), Gd, Id, Out)
    assert np.array_equal(Out.cpu().numpy(), truth.astype(np.float32))


def test_contraction_reference_layout_dma_unaligned_out(mm, cuda, orc):
    """Out 4-byte but not 16-byte aligned."""
    mt, bt, rt, nt, rt_l = 8, 300, 64, 3, 128
    rng = np.random.default_rng(77)
    G = rng.integers(-4, 5, size=(rt, nt, mt, rt_l)).astype(np.float16)
    In = rng.integers(-4, 5, size=(bt, nt, rt_l)).astype(np.float16)
    hA = orc.pack_reference_G(G).astype(np.float64)
    truth = (hA @ In.reshape(bt, nt * rt_l).astype(np.float64).T).reshape(mt, rt, bt).transpose(0, 2, 1)
    buf = cuda.full((mt * bt * rt + 1,), float("nan"), dtype=cuda.float32, device="cuda")
    Out = buf[1:].view(mt, bt, rt)
    mm.contract(mm.contract_desc_reference(mt, bt, rt, nt, rt_l), to_dev(cuda, G), to_dev(cuda, In), Out)
    assert np.array_equal(Out.cpu().numpy(), truth.astype(np.float32))
    assert np.isnan(buf[0].item())


def test_contraction_reference_layout_full_size(mm, cuda, orc):
    """The reference's own contraction size (mmmTensor.cpp:20-28): M = N = K = 8192."""
    mt, bt, rt, nt, rt_l = 128, 8192, 64, 64, 128
    G = cuda.empty((rt, nt, mt, rt_l), dtype=cuda.float16, device="cuda")
    In = cuda.empty((bt, nt, rt_l), dtype=cuda.float16, device="cuda")
    mm.fill_uniform(G, 5, 0)
    mm.fill_uniform(In, 5, 1)
    Out = cuda.full((mt, bt, rt), float("nan"), dtype=cuda.float32, device="cuda")
    mm.contract(mm.contract_desc_reference(mt, bt, rt, nt, rt_l), G, In, Out)
    got = Out.cpu().numpy()
    assert not np.isnan(got).any()
    Gh, Inh = G.cpu().numpy(), In.cpu().numpy()
    rng = np.random.default_rng(15)
    mr = _sample(mt * rt, 16, rng, must=(0, 63, 64, mt * rt - 1))
    T, S = orc.contract_reference_f64(Gh, Inh, mr)
    Cs = np.ascontiguousarray(got.transpose(0, 2, 1).reshape(mt * rt, bt)[mr])
    bad, worst = orc.check_tol(Cs, T, S, TOL)
    assert bad == 0, f"{bad} violations (worst {worst:.3g})"


def test_contraction_reference_layout_tolerance(mm, cuda, orc):
    mt, bt, rt, nt, rt_l = 16, 512, 64, 8, 128
    G = orc.normal_f16((rt, nt, mt, rt_l), 6, 0, 0.1)
    In = orc.normal_f16((bt, nt, rt_l), 6, 1, 0.1)
    Out = cuda.full((mt, bt, rt), float("nan"), dtype=cuda.float32, device="cuda")
    mm.contract(mm.contract_desc_reference(mt, bt, rt, nt, rt_l), to_dev(cuda, G), to_dev(cuda, In), Out)
    got = Out.cpu().numpy()
    rng = np.random.default_rng(14)
    mr = _sample(mt * rt, 32, rng, must=(0, mt * rt - 1))
    T, S = orc.contract_reference_f64(G, In, mr)
    Cs = np.ascontiguousarray(got.transpose(0, 2, 1).reshape(mt * rt, bt)[mr])
    bad, worst = orc.check_tol(Cs, T, S, TOL)
    assert bad == 0, f"{bad} violations (worst {worst:.3g})"


# ------------------------------------------------------------------------------ input generator
def test_fill_uniform_matches_oracle(mm, cuda, orc):
    n = 1_000_003
    t = cuda.empty(n, dtype=cuda.float16, device="cuda")
    mm.fill_uniform(t, 7, 1)
    assert np.array_equal(t.cpu().numpy().view(np.uint16), orc.uniform_f16((n,), 7, 1).view(np.uint16))


def test_fill_normal_matches_oracle(mm, cuda, orc):
    n = 1_000_003
    t = cuda.empty(n, dtype=cuda.float16, device="cuda")
    mm.fill_normal(t, 3, 0, 0.1)
    got = t.cpu().numpy()
    ref = orc.normal_f16((n,), 3, 0, 0.1)
    diff = got.view(np.uint16) != ref.view(np.uint16)
    # device and host libm (log, cos) may differ in the last fp64 bit; after the single
    # rounding to fp16 that can flip at most a rare halfway case by one ulp.
    assert diff.mean() < 1e-4
    if diff.any():
        ulps = np.abs(got[diff].view(np.uint16).astype(np.int32) - ref[diff].view(np.uint16).astype(np.int32))
        assert ulps.max() <= 1


# ------------------------------------------------------------------------------ bound launchers
@pytest.mark.parametrize("shape,ws", [((16, 8192, 2048), None), ((16, 4095, 4111), False), ((300, 264, 4096), None),
                                      ((1024, 1024, 1024), None)],
                         ids=["skinny-split", "skinny-no-workspace", "tile-split", "tile"])
def test_bind_gemm(mm, cuda, shape, ws):
    """mmm.bind_gemm: the launcher bound once gives gemm()'s exact result on every call, and sees
    new contents of its operands (it binds storage, not values)."""
    M, N, K = shape
    rng = np.random.default_rng(M + N + K + 5)
    A, B, truth = _exact_case(rng, M, N, K)
    Ad, Bd = to_dev(cuda, A), to_dev(cuda, B)
    Cd = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    launch = mm.bind_gemm(Ad, Bd, Cd, workspace=ws)
    for _ in range(2):
        Cd.fill_(float("nan"))
        launch()
        assert np.array_equal(Cd.cpu().numpy(), truth)
    Ad.neg_()
    launch()
    assert np.array_equal(Cd.cpu().numpy(), -truth)


def test_bind_contract(mm, cuda, orc):
    """mmm.bind_contract on the baseline fold and the reference layout: exact, repeatable."""
    b, i, k, l, j = 2, 33, 3, 40, 70
    rng = np.random.default_rng(22)
    A = rng.integers(-4, 5, size=(b, i, k, l)).astype(np.float16)
    B = rng.integers(-4, 5, size=(k, l, j)).astype(np.float16)
    truth = np.einsum("bikl,klj->bij", A.astype(np.int64), B.astype(np.int64)).astype(np.float32)
    C = cuda.full((b, i, j), float("nan"), dtype=cuda.float32, device="cuda")
    launch = mm.bind_contract(mm.contract_desc_baseline(b, i, k, l, j), to_dev(cuda, A), to_dev(cuda, B), C)
    for _ in range(2):
        C.fill_(float("nan"))
        launch()
        assert np.array_equal(C.cpu().numpy(), truth)
    mt, bt, rt, nt, rt_l = 8, 300, 64, 3, 128
    G = rng.integers(-4, 5, size=(rt, nt, mt, rt_l)).astype(np.float16)
    In = rng.integers(-4, 5, size=(bt, nt, rt_l)).astype(np.float16)
    truth = np.einsum("rnml,bnl->mbr", G.astype(np.int64), In.astype(np.int64)).astype(np.float32)
    Out = cuda.full((mt, bt, rt), float("nan"), dtype=cuda.float32, device="cuda")
    desc = mm.contract_desc_reference(mt, bt, rt, nt, rt_l)
    launch = mm.bind_contract(desc, to_dev(cuda, G), to_dev(cuda, In), Out)
    del desc  # the launcher holds its own copy of the descriptor
    for _ in range(2):
        Out.fill_(float("nan"))
        launch()
        assert np.array_equal(Out.cpu().numpy(), truth)


def _fold_case(rng, ext, order_a, order_b, order_c):
    """Integer-valued operands laid out with the given axis orders over the sub-indices
    mh, ml (rows), nh, nl (columns), kh, kl (reduction), and the descriptor that addresses them in
    place (element strides read off the arrays)."""
    import mmm

    def make(order, dtype, fill=True):
        shape = tuple(ext[a] for a in order)
        x = rng.integers(-4, 5, size=shape).astype(dtype) if fill else np.zeros(shape, dtype)
        return x, {a: x.strides[i] // x.itemsize for i, a in enumerate(order)}

    A, sa = make(order_a, np.float16)
    B, sb = make(order_b, np.float16)
    Cz, sc = make(order_c, np.float32, fill=False)
    d = mmm.ContractDesc()
    d.m_ext[0], d.m_ext[1] = ext["mh"], ext["ml"]
    d.n_ext[0], d.n_ext[1] = ext["nh"], ext["nl"]
    d.k_ext[0], d.k_ext[1] = ext["kh"], ext["kl"]
    d.a_m_stride[0], d.a_m_stride[1] = sa["mh"], sa["ml"]
    d.a_k_stride[0], d.a_k_stride[1] = sa["kh"], sa["kl"]
    d.b_k_stride[0], d.b_k_stride[1] = sb["kh"], sb["kl"]
    d.b_n_stride[0], d.b_n_stride[1] = sb["nh"], sb["nl"]
    d.c_m_stride[0], d.c_m_stride[1] = sc["mh"], sc["ml"]
    d.c_n_stride[0], d.c_n_stride[1] = sc["nh"], sc["nl"]
    spec = lambda order: "".join({"mh": "a", "ml": "b", "nh": "c", "nl": "d", "kh": "e", "kl": "f"}[x] for x in order)
    truth = np.einsum(f"{spec(order_a)},{spec(order_b)}->{spec(order_c)}", A.astype(np.int64), B.astype(np.int64))
    return d, A, B, Cz.shape, truth.astype(np.float32)


@pytest.mark.parametrize("seed", range(8))
def test_contraction_random_folds_lane_k_exact(mm, cuda, seed):
    """Random 2-level folds with the K sub-index innermost in both operands and a k_lo that is a
    multiple of 8 (so every stride is too): the direct-to-LDS fold kernel, mostly with K tiles
    crossing k blocks and K ending inside a tile; the other sub-indices in random memory orders.
    Integer inputs, bit-exact against an int64 einsum."""
    rng = np.random.default_rng(2000 + seed)
    kl = int(rng.choice([8, 16, 24, 40, 56, 72, 96, 120, 128]))
    ext = {"mh": int(rng.integers(2, 6)), "ml": int(rng.integers(3, 70)), "nh": int(rng.integers(2, 6)),
           "nl": int(rng.integers(3, 70)), "kh": int(rng.integers(1, 6)), "kl": kl}
    order_a = list(rng.permutation(["mh", "ml", "kh"])) + ["kl"]
    order_b = list(rng.permutation(["kh", "nh", "nl"])) + ["kl"]
    order_c = list(rng.permutation(["mh", "ml", "nh", "nl"]))
    d, A, B, cshape, truth = _fold_case(rng, ext, order_a, order_b, order_c)
    Cd = cuda.full(cshape, float("nan"), dtype=cuda.float32, device="cuda")
    mm.contract(d, to_dev(cuda, A), to_dev(cuda, B), Cd)
    got = Cd.cpu().numpy()
    assert np.array_equal(got, truth), f"{ext} {order_a} {order_b} {order_c}: {int((got != truth).sum())} mismatches"


@pytest.mark.parametrize("seed", range(6))
def test_contraction_random_folds_exact(mm, cuda, seed):
    """Random 2-level folds: every operand's four sub-indices in a random memory order (the generic
    gathering kernel, or the direct-to-LDS fold kernel when the K sub-index happens to be
    contiguous in both operands), integer inputs, bit-exact against an int64 einsum."""
    rng = np.random.default_rng(1000 + seed)
    ext = {"mh": int(rng.integers(2, 6)), "ml": int(rng.integers(3, 40)), "nh": int(rng.integers(2, 6)),
           "nl": int(rng.integers(3, 40)), "kh": int(rng.integers(1, 5)), "kl": int(rng.integers(1, 80))}
    order_a = list(rng.permutation(["mh", "ml", "kh", "kl"]))
    order_b = list(rng.permutation(["kh", "kl", "nh", "nl"]))
    order_c = list(rng.permutation(["mh", "ml", "nh", "nl"]))
    d, A, B, cshape, truth = _fold_case(rng, ext, order_a, order_b, order_c)
    Cd = cuda.full(cshape, float("nan"), dtype=cuda.float32, device="cuda")
    mm.contract(d, to_dev(cuda, A), to_dev(cuda, B), Cd)
    got = Cd.cpu().numpy()
    assert np.array_equal(got, truth), f"{ext} {order_a} {order_b} {order_c}: {int((got != truth).sum())} mismatches"


@pytest.mark.parametrize("seed", range(8))
def test_contraction_random_large_folds(mm, cuda, seed):
    """Random 2-level folds over grids of many tiles: even seeds with the K sub-index innermost in
    both operands and k_lo a multiple of 8 (the direct-to-LDS fold kernel; K tiles mostly cross k
    blocks; M and N up to 4000, K up to 2048), odd seeds with every sub-index in a random memory
    order (the gathering kernel unless K happens to be contiguous; up to 1500 x 1500 x 1000).
    C's sub-indices in a random order too.  Integer inputs, bit-exact against a device fp64
    product of the operands permuted to [M][K] x [K][N]; C starts as NaN and every element is
    compared."""
    torch = cuda
    rng = np.random.default_rng(3000 + seed)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3000 + seed)
    if seed % 2 == 0:
        kl = int(rng.choice([8, 16, 24, 40, 56, 72, 96, 120, 128, 192, 256]))
        ext = {"mh": int(rng.integers(2, 9)), "ml": int(rng.integers(100, 501)), "nh": int(rng.integers(2, 9)),
               "nl": int(rng.integers(100, 501)), "kh": int(rng.integers(1, 9)), "kl": kl}
        order_a = [str(a) for a in rng.permutation(["mh", "ml", "kh"])] + ["kl"]
        order_b = [str(a) for a in rng.permutation(["kh", "nh", "nl"])] + ["kl"]
    else:
        ext = {"mh": int(rng.integers(2, 6)), "ml": int(rng.integers(50, 301)), "nh": int(rng.integers(2, 6)),
               "nl": int(rng.integers(50, 301)), "kh": int(rng.integers(1, 6)), "kl": int(rng.integers(1, 201))}
        order_a = [str(a) for a in rng.permutation(["mh", "ml", "kh", "kl"])]
        order_b = [str(a) for a in rng.permutation(["kh", "kl", "nh", "nl"])]
    order_c = [str(a) for a in rng.permutation(["mh", "ml", "nh", "nl"])]

    def make(order, operand):
        shape = tuple(ext[a] for a in order)
        if operand:
            x = torch.randint(-4, 5, shape, generator=gen, device="cuda", dtype=torch.int8).to(torch.float16)
        else:
            x = torch.full(shape, float("nan"), dtype=torch.float32, device="cuda")
        return x, {a: x.stride(i) for i, a in enumerate(order)}

    A, sa = make(order_a, True)
    B, sb = make(order_b, True)
    Cd, sc = make(order_c, False)
    d = mm.ContractDesc()
    for f, h, l in (("m_ext", "mh", "ml"), ("n_ext", "nh", "nl"), ("k_ext", "kh", "kl")):
        getattr(d, f)[0], getattr(d, f)[1] = ext[h], ext[l]
    for f, s, h, l in (("a_m_stride", sa, "mh", "ml"), ("a_k_stride", sa, "kh", "kl"), ("b_k_stride", sb, "kh", "kl"),
                       ("b_n_stride", sb, "nh", "nl"), ("c_m_stride", sc, "mh", "ml"), ("c_n_stride", sc, "nh", "nl")):
        getattr(d, f)[0], getattr(d, f)[1] = s[h], s[l]
    M, N, K = ext["mh"] * ext["ml"], ext["nh"] * ext["nl"], ext["kh"] * ext["kl"]
    where = f"{ext} A {order_a} B {order_b} C {order_c} (M {M} N {N} K {K})"
    print(f"[random_large_fold] {where}", flush=True)
    mm.contract(d, A, B, Cd)
    torch.cuda.synchronize()
    A2 = A.permute(*[order_a.index(a) for a in ("mh", "ml", "kh", "kl")]).reshape(M, K).double()
    B2 = B.permute(*[order_b.index(a) for a in ("kh", "kl", "nh", "nl")]).reshape(K, N).double()
    T = (A2 @ B2).reshape(ext["mh"], ext["ml"], ext["nh"], ext["nl"])
    T = T.permute(*[("mh", "ml", "nh", "nl").index(a) for a in order_c]).float()
    same = torch.equal(Cd, T)
    assert same, f"{where}: {int((Cd != T).sum().item())} outputs differ"
    del A, B, Cd, A2, B2, T
    torch.cuda.empty_cache()


def test_contraction_fold_dma_path_exact(mm, cuda):
    """A fold whose K sub-index is contiguous in both operands, in whole 64-deep tiles (the
    direct-to-LDS fold kernel) with permuted M and N sub-indices and a permuted C."""
    rng = np.random.default_rng(77)
    ext = {"mh": 5, "ml": 72, "nh": 3, "nl": 100, "kh": 3, "kl": 128}
    d, A, B, cshape, truth = _fold_case(rng, ext, ["kh", "mh", "ml", "kl"], ["nl", "kh", "nh", "kl"],
                                        ["nh", "mh", "nl", "ml"])
    Cd = cuda.full(cshape, float("nan"), dtype=cuda.float32, device="cuda")
    mm.contract(d, to_dev(cuda, A), to_dev(cuda, B), Cd)
    assert np.array_equal(Cd.cpu().numpy(), truth)


@pytest.mark.parametrize("seed", range(12))
def test_exact_random_views(mm, cuda, seed):
    """Random shapes (1..700 per side, some past 256 for multi-tile grids), random row pitches of
    A, B and C, random element offsets of each base (2- to 16-byte alignment), and the planner's
    tile or a random forced one: bit-exact on integer inputs, nothing written outside C's view."""
    rng = np.random.default_rng(4242 + seed)
    M, N, K = (int(x) for x in rng.integers(1, 701, size=3))
    A, B, truth = _int_inputs(rng, M, N, K)
    pa, pb, pc = (int(x) for x in rng.integers(0, 12, size=3))
    oa, ob, oc = (int(x) for x in rng.integers(0, 8, size=3))
    Abig = np.zeros((M, K + pa + oa), dtype=np.float16)
    Abig[:, oa:oa + K] = A
    Bbig = np.zeros((K, N + pb + ob), dtype=np.float16)
    Bbig[:, ob:ob + N] = B
    Ad = to_dev(cuda, Abig)[:, oa:oa + K]
    Bd = to_dev(cuda, Bbig)[:, ob:ob + N]
    Cbig = cuda.full((M, N + pc + oc), -1.0, dtype=cuda.float32, device="cuda")
    Cv = Cbig[:, oc:oc + N]
    tile = [None, None, "256x256", "192x192", "128x256", "256x128", "128x128", "64x64"][seed % 8]
    mm.gemm(Ad, Bd, Cv, tile=tile)
    C = Cbig.cpu().numpy()
    where = f"{M}x{N}x{K} pads {pa},{pb},{pc} offsets {oa},{ob},{oc} tile {tile}"
    assert np.array_equal(C[:, oc:oc + N], truth), where
    assert np.all(C[:, :oc] == -1.0) and np.all(C[:, oc + N:] == -1.0), "wrote outside the C view: " + where


@pytest.mark.parametrize("seed", range(10))
def test_exact_random_skinny(mm, cuda, seed):
    """Random M <= 64 problems (the streaming kernels and the tile+stream split), random N and K,
    row pitches and base offsets, with the wrapper's workspace or none: bit-exact, confined to C."""
    rng = np.random.default_rng(777 + seed)
    M = int(rng.integers(1, 65))
    N, K = (int(x) for x in rng.integers(1, 3001, size=2))
    A, B, truth = _int_inputs(rng, M, N, K)
    pa, pb, pc = (int(x) for x in rng.integers(0, 12, size=3))
    oa, ob, oc = (int(x) for x in rng.integers(0, 8, size=3))
    Abig = np.zeros((M, K + pa + oa), dtype=np.float16)
    Abig[:, oa:oa + K] = A
    Bbig = np.zeros((K, N + pb + ob), dtype=np.float16)
    Bbig[:, ob:ob + N] = B
    Ad = to_dev(cuda, Abig)[:, oa:oa + K]
    Bd = to_dev(cuda, Bbig)[:, ob:ob + N]
    Cbig = cuda.full((M, N + pc + oc), -1.0, dtype=cuda.float32, device="cuda")
    ws = None if seed % 2 == 0 else False
    mm.gemm(Ad, Bd, Cbig[:, oc:oc + N], workspace=ws)
    C = Cbig.cpu().numpy()
    where = f"{M}x{N}x{K} pads {pa},{pb},{pc} offsets {oa},{ob},{oc} workspace {ws is None}"
    assert np.array_equal(C[:, oc:oc + N], truth), where
    assert np.all(C[:, :oc] == -1.0) and np.all(C[:, oc + N:] == -1.0), "wrote outside the C view: " + where


def _dev_ints(torch, gen, shape):
    return torch.randint(-4, 5, shape, generator=gen, device="cuda", dtype=torch.int8).to(torch.float16)


@pytest.mark.parametrize("seed", range(16))
def test_exact_random_large(mm, cuda, seed):
    """Random problems of 200 .. 6000 rows and columns and 1 .. 3000 deep, where the planner picks
    among persistent grids, K-split last rounds, the six tiles and the tile+stream split (the plan
    is printed), on views with random row pitches and one-element base offsets, with the
    wrapper's workspace or none: bit-exact against a device fp64 product, confined to C."""
    torch = cuda
    rng = np.random.default_rng(9000 + seed)
    M, N = (int(x) for x in rng.integers(200, 6001, size=2))
    K = int(rng.integers(1, 3001))
    pa, pb, pc = (int(x) for x in rng.integers(0, 9, size=3))
    oa, ob, oc = (int(x) for x in rng.integers(0, 2, size=3))
    if seed % 4 in (0, 2):  # aligned views (16-byte rows and bases)
        pa, pb, pc = (8 * int(x) for x in rng.integers(0, 2, size=3))
        oa = ob = oc = 0
    if seed % 4 == 0:  # a few rows past whole 256-row tiles: the tile+stream split
        M = 256 * int(rng.integers(12, 24)) + int(rng.integers(1, 65))
        N = 256 * int(rng.integers(12, 24))
        K = 64 * int(rng.integers(16, 48))
    elif seed % 4 == 2:  # whole 256 x 256 tiles over more than one round: the persistent grids
        M, N = (256 * int(x) for x in rng.integers(17, 24, size=2))
        K = 64 * int(rng.integers(4, 48))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    Abig = _dev_ints(torch, gen, (M, K + pa + oa))
    Bbig = _dev_ints(torch, gen, (K, N + pb + ob))
    Ad, Bd = Abig[:, oa:oa + K], Bbig[:, ob:ob + N]
    Cbig = torch.full((M, N + pc + oc), -1.0, dtype=torch.float32, device="cuda")
    Cv = Cbig[:, oc:oc + N]
    ws = None if seed % 2 == 0 else False
    plan = mm.gemm_plan(M, N, K, lda=Ad.stride(0), ldb=Bd.stride(0), ldc=Cv.stride(0), A=Ad, B=Bd, C_out=Cv)
    where = f"{M}x{N}x{K} pitches +{pa},+{pb},+{pc} offsets {oa},{ob},{oc} workspace {ws is None}"
    print(f"[random_large] {where} plan {plan['kernel']} tile {plan['block_m']}x{plan['block_n']} "
          f"splits {plan['tile_splits']} persistent {plan['tile_persistent']} stream rows {plan['stream_rows']}",
          flush=True)
    mm.gemm(Ad, Bd, Cv, workspace=ws)
    torch.cuda.synchronize()
    assert bool((Cbig[:, :oc] == -1.0).all()) and bool((Cbig[:, oc + N:] == -1.0).all()), "wrote outside C: " + where
    _assert_exact_rows(torch, Ad, Bd, Cv, where)
    del Abig, Bbig, Cbig
    torch.cuda.empty_cache()


def _assert_exact_rows(torch, A, B, C, label, chunk=8192):
    """C (a device view) equals the fp64 product A.B exactly, compared on the device in row chunks
    (integer inputs: every value is an integer below 2^24, exact in fp32 and fp64)."""
    Bd = B.double()
    for r0 in range(0, A.shape[0], chunk):
        want = (A[r0:r0 + chunk].double() @ Bd).float()
        same = torch.equal(C[r0:r0 + chunk], want)
        assert same, f"{label}: rows {r0}..{r0 + chunk} differ (max |d| {(C[r0:r0 + chunk] - want).abs().max().item()})"
    del Bd


@pytest.mark.parametrize("case", ["big_c", "big_c_persistent", "big_a", "big_b"])
def test_large_operands_exact(mm, cuda, case):
    """Operands and results past 2^31 elements (byte offsets past 4 GiB): per-tile buffer
    descriptors rebased from 64-bit pointers, 64-bit C addressing, the element-wise K-tail
    gather and the K-split partials, all bit-exact against a device fp64 product and confined to
    C's view.  big_c: C of 66000 x 33008 floats (K = 40); big_c_persistent: C of 65792 x 33032
    floats on the persistent 256 x 256 grid (K = 256); big_a: A of 66000 x 33001 halves (odd
    rows, K tail gathered); big_b: B of 66000 x 33001 halves under M = 16 and M = 300."""
    torch = cuda
    gen = torch.Generator(device="cuda")
    gen.manual_seed(20241202)
    if case == "big_c":
        shapes = [(66000, 33000, 40)]
        A_all = _dev_ints(torch, gen, (66000, 40))
        B = _dev_ints(torch, gen, (40, 33000))
    elif case == "big_c_persistent":
        shapes = [(65792, 33024, 256)]
        assert mm.gemm_plan(*shapes[0])["tile_persistent"] == 1
        A_all = _dev_ints(torch, gen, (65792, 256))
        B = _dev_ints(torch, gen, (256, 33024))
    elif case == "big_a":
        shapes = [(66000, 72, 33001)]
        A_all = _dev_ints(torch, gen, (66000, 33001))
        B = _dev_ints(torch, gen, (33001, 72))
    else:
        shapes = [(16, 33001, 66000), (300, 33001, 66000)]
        A_all = _dev_ints(torch, gen, (300, 66000))
        B = _dev_ints(torch, gen, (66000, 33001))
    try:
        for M, N, K in shapes:
            print(f"large operands {case}: {M}x{N}x{K}", flush=True)
            A = A_all[:M]
            off, pad = 4, 4
            Cbuf = torch.full((M, N + off + pad), -1.0, dtype=torch.float32, device="cuda")
            Cv = Cbuf[:, off:off + N]
            mm.gemm(A, B, Cv)
            torch.cuda.synchronize()
            assert bool((Cbuf[:, :off] == -1.0).all()) and bool((Cbuf[:, off + N:] == -1.0).all()), \
                f"{case} {M}x{N}x{K}: wrote outside the C view"
            _assert_exact_rows(torch, A, B, Cv, f"{case} {M}x{N}x{K}")
            del Cbuf, Cv
        big = max(A_all.numel(), B.numel(), shapes[0][0] * (shapes[0][1] + 8))
        assert big > 2 ** 31, f"{case}: no operand past 2^31 elements ({big})"
    finally:
        del A_all, B
        torch.cuda.empty_cache()


LARGE_CONTRACTIONS = {  # (mt, bt, rt, nt, rt_l)
    "big_out": (128, 270000, 64, 2, 64),         # Out past 2^31 floats; 32-bit buffer loads
    "big_g": (128, 64, 64, 2100, 128),           # G past 2^31 halves: 64-bit direct-to-LDS loads
    "big_g_ragged": (129, 100, 64, 1100, 128),   # the same with partial tiles (M = 8256, N = 100)
    "big_g_lane_k": (128, 64, 64, 2200, 120),    # rt_l = 120: K tiles cross n blocks, per-lane K
    "big_g_regs": (128, 64, 64, 2700, 100),      # rt_l = 100: 8-element chunks cross n blocks,
}                                                # the register-staged fold kernel


@pytest.mark.parametrize("case", sorted(LARGE_CONTRACTIONS))
def test_large_reference_contraction_exact(mm, cuda, case):
    """The reference's tensor program (Out[m][b][r] = sum_{n,l} G[r][n][m][l] In[b][n][l],
    mmmTensor.cpp:246-252) past 2^31 elements, bit-exact on integer inputs against a device fp64
    product.  big_out: the direct-to-LDS fold kernel's scattered epilogue at offsets past 4 GiB;
    big_g / big_g_ragged / big_g_lane_k: a G of more than 1 GiB, read through 64-bit per-lane
    addresses (rows and columns of partial tiles clamped to the last valid one; K tiles crossing
    n blocks); big_g_regs: the register-staged fold kernel on a G past 2^31 halves."""
    torch = cuda
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    mt, bt, rt, nt, rt_l = LARGE_CONTRACTIONS[case]
    print(f"large reference contraction {case}: mt {mt} bt {bt} rt {rt} nt {nt} rt_l {rt_l}", flush=True)
    G = _dev_ints(torch, gen, (rt, nt, mt, rt_l))
    In = _dev_ints(torch, gen, (bt, nt, rt_l))
    assert max(G.numel(), mt * bt * rt) > 2 ** 31 or case == "big_g_ragged"
    assert 16 * nt * rt_l < 2 ** 24  # every partial sum exact in fp32
    try:
        Out = torch.full((mt, bt, rt), -1.0, dtype=torch.float32, device="cuda")
        mm.contract(mm.contract_desc_reference(mt, bt, rt, nt, rt_l), G, In, Out)
        torch.cuda.synchronize()
        Bt = In.reshape(bt, nt * rt_l).double().t()
        step = 8
        for m0 in range(0, mt, step):
            ms = min(step, mt - m0)
            A2 = G[:, :, m0:m0 + ms, :].permute(2, 0, 1, 3).reshape(ms * rt, nt * rt_l).double()
            want = (A2 @ Bt).float().reshape(ms, rt, bt).permute(0, 2, 1)
            assert torch.equal(Out[m0:m0 + ms], want), f"{case}: m {m0}..{m0 + ms} differ"
    finally:
        del G, In
        torch.cuda.empty_cache()


@pytest.mark.parametrize("shape,kernel", [((16, 33001, 8192), "tile"), ((16, 40000, 8192), "tile"),
                                          ((64, 50257, 4096), "tile"), ((16, 49152, 8192), "stream"),
                                          ((32, 81920, 4096), "stream")], ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else v)
@pytest.mark.parametrize("ws", [None, False], ids=["workspace", "no_workspace"])
def test_skinny_many_strips_exact(mm, cuda, shape, kernel, ws):
    """M <= 64 with more 128-column strips than CUs: unaligned B rows and thinly filled rounds on
    the tile kernels (K splits where the planner takes them), fuller rounds streamed over several
    rounds.  Integer inputs, bit-exact against a device fp64 product, confined to C's view."""
    torch = cuda
    M, N, K = shape
    plan = mm.gemm_plan(M, N, K)
    assert plan["kernel"] == kernel, plan
    gen = torch.Generator(device="cuda")
    gen.manual_seed(sum(shape))
    A = _dev_ints(torch, gen, (M, K))
    B = _dev_ints(torch, gen, (K, N))
    Cbuf = torch.full((M, N + 8), -1.0, dtype=torch.float32, device="cuda")
    Cv = Cbuf[:, 4:4 + N]
    mm.gemm(A, B, Cv, workspace=ws)
    torch.cuda.synchronize()
    assert bool((Cbuf[:, :4] == -1.0).all()) and bool((Cbuf[:, 4 + N:] == -1.0).all()), "wrote outside the C view"
    _assert_exact_rows(torch, A, B, Cv, f"{shape} workspace {ws is None}")
