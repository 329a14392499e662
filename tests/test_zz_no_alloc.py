"""GPU test of mmm_gemm_f16f32_noalloc, the entry point whose K-split partials live in the
library's own device array: through the C ABI, its output equals mmm_gemm_f16f32_ws's (given a
workspace from torch) bit for bit -- the same kernels with the same split plan -- on calls in a
row that reuse the array, each call smaller than the one before, with and without a K split,
plus the argument checks.  Collected last (test_zz_*) so a failure here hides no other test.
"""
import ctypes as C

import pytest

pytestmark = pytest.mark.gpu


def _call_ws(mm, torch, A, B, Cout, ws):
    M, K = A.shape
    N = B.shape[1]
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = mm.lib().mmm_gemm_f16f32_ws(C.c_void_p(A.data_ptr()), C.c_void_p(B.data_ptr()), C.c_void_p(Cout.data_ptr()),
                                     M, N, K, K, N, N, C.c_void_p(ws.data_ptr()), ws.numel(), st)
    assert rc == 0


def _call_noalloc(mm, torch, A, B, Cout):
    M, K = A.shape
    N = B.shape[1]
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    return mm.lib().mmm_gemm_f16f32_noalloc(C.c_void_p(A.data_ptr()), C.c_void_p(B.data_ptr()),
                                            C.c_void_p(Cout.data_ptr()), M, N, K, K, N, N, st)


# each smaller than the one before; the first three split K (tile split, tile split, streaming split)
SHAPES = [(2304, 2304, 8192), (1024, 1024, 8192), (16, 4096, 4096), (300, 264, 200)]


def test_noalloc_matches_workspace_entry(mm, cuda):
    torch = cuda
    ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    plans = [mm.gemm_plan(*s)["workspace_bytes"] for s in SHAPES]
    assert plans[0] > 0 and plans[1] > 0 and plans[2] > 0 and plans[3] == 0
    for rep in range(2):  # the array keeps the previous call's partials: repeat the sequence
        for (M, N, K) in SHAPES:
            A = torch.empty((M, K), dtype=torch.float16, device="cuda")
            B = torch.empty((K, N), dtype=torch.float16, device="cuda")
            mm.fill_uniform(A, 31 + rep, 0)
            mm.fill_uniform(B, 31 + rep, 1)
            ref = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            _call_ws(mm, torch, A, B, ref, ws)
            out = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            assert _call_noalloc(mm, torch, A, B, out) == 0
            torch.cuda.synchronize()
            assert not torch.isnan(ref).any()
            assert torch.equal(out, ref), f"{M}x{N}x{K} rep {rep}"


@pytest.mark.parametrize("shape", [(2304, 2304, 8192), (16, 4096, 4096), (16, 8192, 8192)],
                         ids=lambda s: "x".join(map(str, s)))
def test_noalloc_graph_capture(mm, cuda, shape):
    """The documented order for callers under graph capture: one eager call (looks the array's
    address up), then a captured call, replayed.  Every shape splits K into the array (a tile
    split with its reduction launch; the streaming kernel's split on 128- and 256-column
    strips).  Every replay, with eager work and synchronisation in between, equals
    mmm_gemm_f16f32_ws's result bit for bit."""
    torch = cuda
    M, N, K = shape
    assert mm.gemm_plan(M, N, K)["workspace_bytes"] > 0
    ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    A = torch.empty((M, K), dtype=torch.float16, device="cuda")
    B = torch.empty((K, N), dtype=torch.float16, device="cuda")
    mm.fill_uniform(A, 41, 0)
    mm.fill_uniform(B, 41, 1)
    ref = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    _call_ws(mm, torch, A, B, ref, ws)
    out = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    assert _call_noalloc(mm, torch, A, B, out) == 0  # eager first
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = _call_noalloc(mm, torch, A, B, out)
    assert rc == 0
    other = torch.empty((300, 264), dtype=torch.float32, device="cuda")
    for i in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
        # eager calls that reuse the array between the replays
        a2 = torch.empty((300, 200), dtype=torch.float16, device="cuda")
        b2 = torch.empty((200, 264), dtype=torch.float16, device="cuda")
        mm.fill_uniform(a2, 42 + i, 0)
        mm.fill_uniform(b2, 42 + i, 1)
        assert _call_noalloc(mm, torch, A, B, other.new_empty((M, N))) == 0
        assert _call_noalloc(mm, torch, a2, b2, other) == 0
        torch.cuda.synchronize()


def test_noalloc_argument_checks(mm, cuda):
    L = mm.lib()
    null = C.c_void_p(0)
    dummy = C.c_void_p(0x1000)
    assert L.mmm_gemm_f16f32_noalloc(null, null, null, 8, 8, 8, 8, 8, 8, null) == mm.HIP_ERROR_INVALID_VALUE
    assert L.mmm_gemm_f16f32_noalloc(dummy, dummy, dummy, 8, 8, 8, 7, 8, 8, null) == mm.HIP_ERROR_INVALID_VALUE
    assert L.mmm_gemm_f16f32_noalloc(null, null, null, 0, 8, 8, 8, 8, 8, null) == 0  # M == 0: no-op
