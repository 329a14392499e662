"""GPU tests of the measurement probes and the bound hipBLASLt comparison launcher.

The probes (include/mmm.h, mmm_probe_*) give the bench line a measured clock and measured
ceilings; these tests check that they run and report values in the ranges the hardware allows,
and that the bound hipBLASLt launcher computes the same GEMM as the library (tolerance).
"""
import numpy as np
import pytest

from conftest import to_dev

pytestmark = pytest.mark.gpu


def test_probe_clock_range(mm, cuda):
    """Shader clock from s_memtime / s_memrealtime: between the MI355X's lowest DPM level and
    its 2.4 GHz maximum (with margin), and the spin lasted the requested real-time ticks."""
    out = cuda.zeros(2, dtype=cuda.int64, device="cuda")
    for ticks in (2000, 20000):
        mm.probe_clock(out, ticks)
        cuda.cuda.synchronize()
        h = out.cpu()
        assert int(h[1]) >= ticks
        mhz = mm.clock_mhz(h)
        assert 300.0 <= mhz <= 2600.0, mhz


def test_probe_mfma_ceiling_runs(mm, cuda):
    """The ceiling probe writes every tile of C (store_tiles) with finite values, and one float
    per thread without it; it rejects shapes its grid does not cover."""
    M, N, K = 512, 768, 128
    A = cuda.empty((M, K), dtype=cuda.float16, device="cuda")
    B = cuda.empty((K, N), dtype=cuda.float16, device="cuda")
    mm.fill_uniform(A, 9, 0)
    mm.fill_uniform(B, 9, 1)
    C = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    mm.probe_mfma_ceiling(A, B, C, store_tiles=True)
    cuda.cuda.synchronize()
    assert cuda.isfinite(C).all()
    C.fill_(float("nan"))
    mm.probe_mfma_ceiling(A, B, C, store_tiles=False)
    cuda.cuda.synchronize()
    grid = (M // 256) * (N // 256)
    assert cuda.isfinite(C.view(-1)[: grid * 512]).all()
    assert cuda.isnan(C.view(-1)[grid * 512:]).all()
    with pytest.raises(mm.MMMError):
        mm.probe_mfma_ceiling(A[:, :96], B[:96], C)  # K % 64 != 0


@pytest.mark.parametrize("shape", [(256, 256, 128), (512, 768, 512), (8192, 8192, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_probe_lds_mfma_closed_form(mm, cuda, shape):
    """The operand-path probe streams every K tile of its workgroups' shares through the tile
    kernel's fragment reads and MFMAs: on inputs in {-1, 0, 1} each workgroup's outputs sum
    exactly to (tiles * K / 128) * (1^T A0)(B0 1), A0 / B0 its first tile's rows of A and columns
    of B over K 0 .. 127 (the two staged K tiles), with and without the per-K-tile barrier, and
    the barrier changes no bit of any output."""
    torch = cuda
    M, N, K = shape
    gen = torch.Generator(device="cuda")
    gen.manual_seed(M + N + K)
    A = torch.randint(-1, 2, (M, K), generator=gen, device="cuda", dtype=torch.int8).to(torch.float16)
    B = torch.randint(-1, 2, (K, N), generator=gen, device="cuda", dtype=torch.int8).to(torch.float16)
    tiles_m, tiles_n = M // 256, N // 256
    tiles = tiles_m * tiles_n
    grid = min(tiles, 256)
    print(f"[probe_lds_mfma] {M}x{N}x{K} grid {grid}", flush=True)
    outs = {}
    for barrier in (True, False):
        out = torch.full((grid * 512 + 64,), float("nan"), dtype=torch.float32, device="cuda")
        mm.probe_lds_mfma(A, B, out, barrier=barrier)
        torch.cuda.synchronize()
        assert torch.isnan(out[grid * 512:]).all(), "wrote past its outputs"
        outs[barrier] = out[: grid * 512].cpu().numpy().astype(np.float64).reshape(grid, 512)
    assert np.array_equal(outs[True], outs[False])
    Ah = A.float().cpu().numpy().astype(np.int64)
    Bh = B.float().cpu().numpy().astype(np.int64)
    for g in range(grid):
        tm, tn = mm.tile_of_block(g, tiles_m, tiles_n)
        mine = (tiles - g + grid - 1) // grid
        a_rows = Ah[tm * 256:(tm + 1) * 256, :128].sum(axis=0)
        b_cols = Bh[:128, tn * 256:(tn + 1) * 256].sum(axis=1)
        want = mine * K // 128 * int(a_rows @ b_cols)
        assert outs[True][g].sum() == want, f"workgroup {g} (tile {tm},{tn}): {outs[True][g].sum()} != {want}"


def test_probe_lds_mfma_rejects(mm, cuda):
    """Shapes outside the probe's grid (K not a multiple of 128, M not of 256) and an output
    buffer shorter than one float per thread are refused before any launch."""
    A = cuda.zeros((512, 256), dtype=cuda.float16, device="cuda")
    B = cuda.zeros((256, 512), dtype=cuda.float16, device="cuda")
    with pytest.raises(mm.MMMError):
        mm.probe_lds_mfma(A[:, :192].contiguous(), B[:192].contiguous())  # K % 128 != 0
    with pytest.raises(mm.MMMError):
        mm.probe_lds_mfma(A[:300].contiguous(), B)  # M % 256 != 0
    short = cuda.empty(4 * 512 - 1, dtype=cuda.float32, device="cuda")
    with pytest.raises(mm.MMMError):
        mm.probe_lds_mfma(A, B, short)
    with pytest.raises(ValueError):
        mm.probe_lds_mfma(A[:, :128], B[:128])  # not contiguous


@pytest.mark.parametrize("lds", [False, True])
def test_probe_read_runs(mm, cuda, lds):
    """The streaming-read probe reads every byte: an all-zero buffer XOR-folds to zeros, and a
    single planted word shows up in the plain-load fold."""
    src = cuda.zeros(1 << 24, dtype=cuda.uint8, device="cuda")
    out = cuda.full((8192 * 256,), -1, dtype=cuda.int32, device="cuda")
    mm.probe_read(src, out, direct_to_lds=lds)
    cuda.cuda.synchronize()
    if not lds:
        assert (out == 0).all()
        src.view(cuda.int32)[12345] = 0x5A5A5A5A
        mm.probe_read(src, out)
        cuda.cuda.synchronize()
        folded = int(np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32)))
        assert folded == 0x5A5A5A5A


def test_probe_read_lds_pieces(mm, cuda):
    """The direct-to-LDS read probe loads the pieces it claims: each 1 KB piece p starts with the
    word p + 1, and workgroup b reports the first word of wave 0's ring slot 0, which is the last
    piece that wave put there.  Wave 4b (8192 workgroups x 4 waves) takes pieces 4b + 32768 j and
    ring slot j % 32; with 2^21 - 1 pieces (2 GiB less 1 KB) that is j = 32, piece 4b + 2^20."""
    pieces = (1 << 21) - 1
    src = cuda.zeros(pieces * 1024, dtype=cuda.uint8, device="cuda")
    src.view(cuda.int32)[::256] = cuda.arange(1, pieces + 1, dtype=cuda.int32, device="cuda")
    out = cuda.full((8192,), -1, dtype=cuda.int32, device="cuda")
    mm.probe_read(src, out, direct_to_lds=True)
    cuda.cuda.synchronize()
    waves = 8192 * 4
    expect = []
    for b in range(8192):
        wid = 4 * b
        j_last = max(j for j in range(0, pieces // waves + 1, 32) if wid + j * waves < pieces)
        expect.append(wid + j_last * waves + 1)
    assert np.array_equal(out.cpu().numpy(), np.array(expect, dtype=np.int32))
    del src
    cuda.cuda.empty_cache()


@pytest.mark.parametrize("shape", [(256, 256, 256), (1000, 777, 320), (16, 4096, 4096)])
def test_bound_hipblaslt_matches_library(orc, mm, cuda, shape):
    """The bound hipBLASLt launcher (descriptors and heuristic planned once) computes the same
    FP16 -> FP32 GEMM as the library, within the BASELINE tolerance, on repeated calls."""
    M, N, K = shape
    A = orc.uniform_f16((M, K), 5, 0)
    B = orc.uniform_f16((K, N), 5, 1)
    Ad, Bd = to_dev(cuda, A), to_dev(cuda, B)
    ours = mm.gemm(Ad, Bd).cpu().numpy().astype(np.float64)
    Cw = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    launch = mm.bind_witness_hipblaslt(Ad, Bd, Cw)
    for _ in range(3):
        launch()
    cuda.cuda.synchronize()
    W = Cw.cpu().numpy().astype(np.float64)
    _, S = orc.gemm_f64(A, B)
    assert np.all(np.abs(W - ours) <= 2e-3 * S)


@pytest.mark.parametrize("shape", [(512, 768, 320), (8192, 8192, 512), (4097, 4095, 1000)])
def test_clocked_entry_point(mm, cuda, shape):
    """mmm_gemm_f16f32_clocked computes exactly what mmm_gemm_f16f32_ws computes (same launch)
    and, for the tile kernels, writes workgroup 0's counters: a positive duration at a clock in
    the hardware's range."""
    M, N, K = shape
    A = cuda.empty((M, K), dtype=cuda.float16, device="cuda")
    B = cuda.empty((K, N), dtype=cuda.float16, device="cuda")
    mm.fill_uniform(A, 3, 0)
    mm.fill_uniform(B, 3, 1)
    ref = mm.gemm(A, B)
    Cc = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    clock = cuda.zeros((2, 4), dtype=cuda.int64, device="cuda")
    launch = mm.bind_gemm_clocked(A, B, Cc, clock)
    launch()
    launch()
    cuda.cuda.synchronize()
    assert cuda.equal(Cc, ref)
    h = clock.cpu()
    assert (h[:, 2] > h[:, 0]).all() and (h[:, 3] > h[:, 1]).all()
    for mhz in mm.clocks_mhz(clock):
        assert 300.0 <= mhz <= 2600.0, mhz


def test_clocked_streaming_kernel_leaves_clock(mm, cuda):
    """The M <= 64 streaming kernels record nothing: the counters stay as the caller left them."""
    A = cuda.empty((16, 2048), dtype=cuda.float16, device="cuda")
    B = cuda.empty((2048, 4096), dtype=cuda.float16, device="cuda")
    mm.fill_uniform(A, 4, 0)
    mm.fill_uniform(B, 4, 1)
    Cc = cuda.empty((16, 4096), dtype=cuda.float32, device="cuda")
    clock = cuda.full((1, 4), 7, dtype=cuda.int64, device="cuda")
    mm.bind_gemm_clocked(A, B, Cc, clock)()
    cuda.cuda.synchronize()
    assert (clock.cpu() == 7).all()
    assert cuda.equal(Cc, mm.gemm(A, B))
