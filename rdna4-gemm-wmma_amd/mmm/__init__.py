"""Python binding of the MI355X GEMM / contraction library (ctypes over lib/libmmm.so).

The library's C ABI is declared in ``include/mmm.h``; this module mirrors it one to one
for Python callers (tests, bench).  Device buffers are torch tensors (torch is only the
allocator and stream provider here); every call goes through the HIP kernels in
``lib/libmmm.so``.  There is no CPU fallback: if the library is missing, loading fails.

The entry points mirror the reference's kernel entry (thrasos-g/RDNA4-GEMM-WMMA,
``WMMA_Swizzled_Full<WAVE_M,WAVE_N,WAVES_I,WAVES_J>(A, B, C)``, mmm.cpp:1214-1215, and the
tensor variant mmmTensor.cpp:44-45): device pointers, M/N/K, tile parameters.
"""
from __future__ import annotations

import ctypes as C
import threading
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)
REPO_ROOT = os.path.dirname(PKG_ROOT)
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libmmm.so")
HEADER_PATH = os.path.join(REPO_ROOT, "include", "mmm.h")

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1

_lib = None


class MMMError(RuntimeError):
    """A library call returned a hipError_t other than hipSuccess."""

    def __init__(self, func: str, code: int):
        self.code = code
        super().__init__(f"{func} failed: hipError_t {code} ({_error_name(code)})")


def _error_name(code: int) -> str:
    try:
        hip = C.CDLL("libamdhip64.so")
        hip.hipGetErrorName.restype = C.c_char_p
        hip.hipGetErrorName.argtypes = [C.c_int]
        return hip.hipGetErrorName(code).decode()
    except OSError:
        return "unknown"


class GemmPlan(C.Structure):
    """mmm_gemm_plan (include/mmm.h)."""
    _fields_ = [("kernel", C.c_int), ("wave_m", C.c_int), ("wave_n", C.c_int), ("waves_i", C.c_int),
                ("waves_j", C.c_int), ("block_m", C.c_int), ("block_n", C.c_int), ("direct_to_lds", C.c_int),
                ("tile_rows", C.c_int), ("stream_rows", C.c_int), ("tile_workgroups", C.c_int64),
                ("stream_workgroups", C.c_int64), ("stream_splits", C.c_int), ("tile_splits", C.c_int),
                ("tile_split_tiles", C.c_int), ("tile_persistent", C.c_int), ("workspace_bytes", C.c_int64),
                ("stream_columns", C.c_int)]


class ContractDesc(C.Structure):
    """mmm_contract_desc (include/mmm.h)."""

    _fields_ = [(name, C.c_int64 * 2) for name in (
        "m_ext", "n_ext", "k_ext", "a_m_stride", "a_k_stride", "b_k_stride", "b_n_stride", "c_m_stride",
        "c_n_stride")]

    def as_dict(self):
        return {name: tuple(getattr(self, name)) for name, _ in self._fields_}

    @property
    def M(self) -> int:
        return self.m_ext[0] * self.m_ext[1]

    @property
    def N(self) -> int:
        return self.n_ext[0] * self.n_ext[1]

    @property
    def K(self) -> int:
        return self.k_ext[0] * self.k_ext[1]


def declared_symbols(header: str = HEADER_PATH):
    """Names of the functions include/mmm.h declares."""
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mmm_[a-z0-9_]+)\s*\(", text)))


def build() -> None:
    """Compile the gfx950 library in-tree (make -C rdna4-gemm-wmma_amd)."""
    import subprocess

    subprocess.run(["make", "-s", "-j4", "-C", PKG_ROOT], check=True)


def lib() -> C.CDLL:
    """Load lib/libmmm.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C {PKG_ROOT}` (or __graft_entry__.build())")
    # torch wheels carry their own HIP runtime under the same soname (libamdhip64.so.7).
    # Loading torch first makes this library bind to that runtime; loading it first would
    # put a second HIP runtime into the process, and torch's device memory would not be
    # visible to it (hipErrorNoDevice).
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = C.CDLL(LIB_PATH)
    p, i, i64, s, sz = C.c_void_p, C.c_int, C.c_int64, C.c_void_p, C.c_size_t
    L.mmm_gemm_f16f32.argtypes = [p, p, p, i, i, i, i64, i64, i64, s]
    L.mmm_gemm_f16f32_ws.argtypes = [p, p, p, i, i, i, i64, i64, i64, p, sz, s]
    L.mmm_gemm_f16f32_clocked.argtypes = [p, p, p, i, i, i, i64, i64, i64, p, sz, p, s]
    L.mmm_gemm_f16f32_noalloc.argtypes = [p, p, p, i, i, i, i64, i64, i64, s]
    L.mmm_gemm_workspace_f16f32.argtypes = [p, p, p, i, i, i, i64, i64, i64, C.POINTER(sz)]
    L.mmm_gemm_f16f32_tiled.argtypes = [p, p, p, i, i, i, i64, i64, i64, i, i, i, i, p, sz, s]
    L.mmm_contract_desc_baseline.argtypes = [C.POINTER(ContractDesc), i, i, i, i, i]
    L.mmm_contract_desc_reference.argtypes = [C.POINTER(ContractDesc), i, i, i, i, i]
    L.mmm_contract5d_f16f32.argtypes = [C.POINTER(ContractDesc), p, p, p, s]
    L.mmm_contract5d_f16f32_ws.argtypes = [C.POINTER(ContractDesc), p, p, p, p, sz, s]
    L.mmm_contract5d_workspace_f16f32.argtypes = [C.POINTER(ContractDesc), p, p, p, C.POINTER(sz)]
    L.mmm_fill_uniform_f16.argtypes = [p, i64, C.c_uint64, C.c_uint32, s]
    L.mmm_fill_normal_f16.argtypes = [p, i64, C.c_uint64, C.c_uint32, C.c_double, s]
    L.mmm_tile_of_block.argtypes = [i, i, i, C.POINTER(i), C.POINTER(i)]
    L.mmm_gemm_naive_f16f32.argtypes = [p, p, p, i, i, i, i64, i64, i64, s]
    L.mmm_gemm_truth_f64.argtypes = [p, p, p, p, i, i, i, i64, i64, i64, s]
    L.mmm_contract5d_truth_f64.argtypes = [C.POINTER(ContractDesc), p, p, p, p, s]
    L.mmm_gemm_plan_f16f32.argtypes = [p, p, p, i, i, i, i64, i64, i64, C.POINTER(GemmPlan)]
    L.mmm_probe_clock.argtypes = [p, i64, s]
    L.mmm_probe_mfma_ceiling.argtypes = [p, p, p, i, i, i, i, p, s]
    L.mmm_probe_lds_mfma.argtypes = [p, p, p, i64, i, i, i, i, p, s]
    L.mmm_probe_read.argtypes = [p, i64, i, p, i64, s]
    for name in ("mmm_gemm_f16f32", "mmm_gemm_f16f32_ws", "mmm_gemm_f16f32_clocked", "mmm_gemm_f16f32_noalloc", "mmm_gemm_workspace_f16f32", "mmm_gemm_f16f32_tiled",
                 "mmm_contract_desc_baseline", "mmm_contract_desc_reference", "mmm_contract5d_f16f32",
                 "mmm_contract5d_f16f32_ws", "mmm_contract5d_workspace_f16f32", "mmm_fill_uniform_f16",
                 "mmm_fill_normal_f16", "mmm_tile_of_block", "mmm_gemm_naive_f16f32", "mmm_gemm_truth_f64",
                 "mmm_contract5d_truth_f64", "mmm_gemm_plan_f16f32", "mmm_probe_clock", "mmm_probe_mfma_ceiling",
                 "mmm_probe_lds_mfma", "mmm_probe_read"):
        getattr(L, name).restype = C.c_int
    L.mmm_version.restype = C.c_char_p
    L.mmm_version.argtypes = []
    _lib = L
    return L


def _check(func: str, code: int) -> None:
    if code != HIP_SUCCESS:
        raise MMMError(func, code)


def _stream(stream):
    import torch

    if stream is None:
        stream = torch.cuda.current_stream()
    return C.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream))


def _ptr(t) -> C.c_void_p:
    return C.c_void_p(t.data_ptr())


def _check_f16(name: str, t) -> None:
    import torch

    if t.dtype != torch.float16 or not t.is_cuda:
        raise TypeError(f"{name} must be a CUDA float16 tensor")


# Tile parameters (WAVE_M, WAVE_N, WAVES_I, WAVES_J) of the instantiated block tiles.
TILES = {"256x256": (4, 4, 2, 2), "128x256": (2, 4, 2, 2), "256x128": (4, 2, 2, 2), "128x128": (2, 2, 2, 2),
         "64x64": (1, 1, 2, 2), "192x192": (3, 3, 2, 2)}

# The most workspace any K split uses (the library plans its splits within this).
MAX_WORKSPACE_BYTES = 64 << 20

# K-split workspaces the wrappers pass to the library: one per (device, stream), from torch's
# allocator, grown on demand.  Calls on one stream are ordered, so they may share one.
_ws_lock = threading.Lock()
_ws_cache = {}


def _workspace(device, st: C.c_void_p, nbytes: int):
    import torch

    key = (device.index if device.index is not None else torch.cuda.current_device(), st.value or 0)
    with _ws_lock:
        t = _ws_cache.get(key)
        if t is None or t.numel() < nbytes:
            t = torch.empty(nbytes, dtype=torch.uint8, device=device)
            _ws_cache[key] = t
        return t


def _ws_args(workspace, device, st, nbytes: int):
    """(pointer, bytes) for a call needing nbytes: the caller's tensor, none (workspace=False),
    or the per-stream cache."""
    if workspace is False or nbytes == 0:
        return None, 0
    t = workspace if workspace is not None else _workspace(device, st, nbytes)
    return C.c_void_p(t.data_ptr()), t.numel() * t.element_size()


def gemm(A, B, C_out=None, tile=None, stream=None, workspace=None):
    """C = A @ B for fp16 A [M,K] and B [K,N] (row-major, any leading dimension via strides).

    Returns the fp32 C [M,N].  ``tile`` is None (library heuristic), a key of TILES, or a
    (WAVE_M, WAVE_N, WAVES_I, WAVES_J) tuple.  ``workspace``: a CUDA tensor for the K-split
    partials (mmm_gemm_f16f32_ws), None for a per-stream one from torch's allocator, or False
    for none (the unsplit kernels).
    """
    import torch

    _check_f16("A", A)
    _check_f16("B", B)
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[0]:
        raise ValueError("A must be [M,K] and B [K,N]")
    if A.stride(1) != 1 or B.stride(1) != 1:
        raise ValueError("A and B must be row-major (unit stride along the last dimension)")
    M, K = A.shape
    N = B.shape[1]
    if C_out is None:
        C_out = torch.empty((M, N), dtype=torch.float32, device=A.device)
    if C_out.dtype != torch.float32 or C_out.stride(1) != 1 or tuple(C_out.shape) != (M, N):
        raise ValueError("C must be a row-major float32 [M,N] tensor")
    lda = A.stride(0) if M > 1 else max(K, 1)
    ldb = B.stride(0) if K > 1 else max(N, 1)
    ldc = C_out.stride(0) if M > 1 else max(N, 1)
    st = _stream(stream)
    L = lib()
    if tile is None:
        # one library call: the per-stream workspace holds the largest split the library plans
        wp, wb = _ws_args(workspace, A.device, st, MAX_WORKSPACE_BYTES)
        _check("mmm_gemm_f16f32_ws",
               L.mmm_gemm_f16f32_ws(_ptr(A), _ptr(B), _ptr(C_out), M, N, K, lda, ldb, ldc, wp, wb, st))
    else:
        params = TILES[tile] if isinstance(tile, str) else tuple(tile)
        wp, wb = _ws_args(workspace, A.device, st, MAX_WORKSPACE_BYTES)
        _check("mmm_gemm_f16f32_tiled",
               L.mmm_gemm_f16f32_tiled(_ptr(A), _ptr(B), _ptr(C_out), M, N, K, lda, ldb, ldc, *params, wp, wb, st))
    return C_out


def _ws_tensor(workspace, device, st):
    """The workspace tensor a bound launcher keeps alive: the caller's, the per-stream one, or None."""
    if workspace is False:
        return None
    return workspace if workspace is not None else _workspace(device, st, MAX_WORKSPACE_BYTES)


def _bound(fn, name: str, args: tuple, keep: tuple):
    def launch():
        rc = fn(*args)
        if rc != HIP_SUCCESS:
            raise MMMError(name, rc)

    launch.tensors = keep  # the launcher holds its operands (and workspace) alive
    return launch


def bind_gemm(A, B, C_out, stream=None, workspace=None, tile=None):
    """A zero-argument launcher of C = A @ B on fixed tensors and a fixed stream.

    gemm()'s checks run once, here; each call of the result is one mmm_gemm_f16f32_ws call (or
    mmm_gemm_f16f32_tiled with ``tile``) with prebuilt arguments, for loops that launch one
    problem many times (a benchmark, a serving step).  ``workspace`` and ``tile`` as for gemm.
    The tensors must keep their storage while it is used."""
    import torch

    if C_out is None or C_out.dtype != torch.float32:
        raise ValueError("C must be a row-major float32 [M,N] tensor")
    M, N, K, lda, ldb, ldc = _gemm_shapes(A, B, C_out)
    st = _stream(stream)
    ws = _ws_tensor(workspace, A.device, st)
    wp = C.c_void_p(ws.data_ptr()) if ws is not None else None
    wb = ws.numel() * ws.element_size() if ws is not None else 0
    if tile is not None:
        params = TILES[tile] if isinstance(tile, str) else tuple(tile)
        args = (_ptr(A), _ptr(B), _ptr(C_out), M, N, K, lda, ldb, ldc, *params, wp, wb, st)
        return _bound(lib().mmm_gemm_f16f32_tiled, "mmm_gemm_f16f32_tiled", args, (A, B, C_out, ws))
    args = (_ptr(A), _ptr(B), _ptr(C_out), M, N, K, lda, ldb, ldc, wp, wb, st)
    return _bound(lib().mmm_gemm_f16f32_ws, "mmm_gemm_f16f32_ws", args, (A, B, C_out, ws))


def bind_gemm_clocked(A, B, C_out, clock, stream=None, workspace=None):
    """As bind_gemm, through mmm_gemm_f16f32_clocked: launch i (i = 0, 1, ...) writes workgroup 0's
    start and end counters to clock[i] (a CUDA int64 tensor [n, 4]; launches past n wrap)."""
    import torch

    if C_out is None or C_out.dtype != torch.float32:
        raise ValueError("C must be a row-major float32 [M,N] tensor")
    if clock.dtype != torch.int64 or clock.dim() != 2 or clock.shape[1] != 4 or not clock.is_contiguous():
        raise ValueError("clock must be a contiguous CUDA int64 tensor [n, 4]")
    M, N, K, lda, ldb, ldc = _gemm_shapes(A, B, C_out)
    st = _stream(stream)
    ws = _ws_tensor(workspace, A.device, st)
    wp = C.c_void_p(ws.data_ptr()) if ws is not None else None
    wb = ws.numel() * ws.element_size() if ws is not None else 0
    fn = lib().mmm_gemm_f16f32_clocked
    state = {"i": 0}
    base = (_ptr(A), _ptr(B), _ptr(C_out), M, N, K, lda, ldb, ldc, wp, wb)

    def launch():
        slot = C.c_void_p(clock.data_ptr() + 32 * (state["i"] % clock.shape[0]))
        state["i"] += 1
        rc = fn(*base, slot, st)
        if rc != HIP_SUCCESS:
            raise MMMError("mmm_gemm_f16f32_clocked", rc)

    launch.tensors = (A, B, C_out, ws, clock)
    return launch


def clocks_mhz(clock):
    """Shader clock (MHz) of each launch recorded by bind_gemm_clocked (rows of [n, 4] counters)."""
    h = clock.cpu().tolist()
    return [(c1 - c0) / (r1 - r0) * 100.0 if r1 > r0 else float("nan") for c0, r0, c1, r1 in h]


def bind_contract(desc: "ContractDesc", A, B, C_out, stream=None, workspace=None):
    """A zero-argument launcher of contract(desc, A, B, C_out) on fixed tensors and stream: one
    mmm_contract5d_f16f32_ws call per launch (the library validates the descriptor each call)."""
    import torch

    _check_f16("A", A)
    _check_f16("B", B)
    if C_out.dtype != torch.float32 or not C_out.is_cuda:
        raise TypeError("C must be a CUDA float32 tensor")
    st = _stream(stream)
    d = ContractDesc.from_buffer_copy(desc)
    ws = _ws_tensor(workspace, A.device, st)
    wp = C.c_void_p(ws.data_ptr()) if ws is not None else None
    wb = ws.numel() * ws.element_size() if ws is not None else 0
    args = (C.pointer(d), _ptr(A), _ptr(B), _ptr(C_out), wp, wb, st)
    return _bound(lib().mmm_contract5d_f16f32_ws, "mmm_contract5d_f16f32_ws", args, (A, B, C_out, ws, d))


KERNELS = {0: "none", 1: "zero", 2: "tile", 3: "stream", 4: "tile+stream"}


def gemm_plan(M: int, N: int, K: int, lda=None, ldb=None, ldc=None, A=None, B=None, C_out=None) -> dict:
    """The launch mmm_gemm_f16f32 would make (host-only query; pointers only matter for alignment)."""
    pl = GemmPlan()
    addr = lambda t: C.c_void_p(t.data_ptr() if hasattr(t, "data_ptr") else t) if t is not None else None
    _check("mmm_gemm_plan_f16f32",
           lib().mmm_gemm_plan_f16f32(addr(A), addr(B), addr(C_out), M, N, K, K if lda is None else lda,
                                      N if ldb is None else ldb, N if ldc is None else ldc, C.byref(pl)))
    out = {f: getattr(pl, f) for f, _ in GemmPlan._fields_}
    out["kernel"] = KERNELS[pl.kernel]
    return out


def _gemm_shapes(A, B, out):
    _check_f16("A", A)
    _check_f16("B", B)
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[0]:
        raise ValueError("A must be [M,K] and B [K,N]")
    if A.stride(1) != 1 or B.stride(1) != 1:
        raise ValueError("A and B must be row-major (unit stride along the last dimension)")
    M, K = A.shape
    N = B.shape[1]
    lda = A.stride(0) if M > 1 else max(K, 1)
    ldb = B.stride(0) if K > 1 else max(N, 1)
    ldo = out.stride(0) if M > 1 else max(N, 1)
    if out.stride(1) != 1 or tuple(out.shape) != (M, N):
        raise ValueError("outputs must be row-major [M,N] tensors")
    return M, N, K, lda, ldb, ldo


def gemm_naive(A, B, C_out=None, stream=None):
    """The reference's GEMM_Naive on the device: fp32 accumulator, k ascending (cross-check)."""
    import torch

    if C_out is None:
        C_out = torch.empty((A.shape[0], B.shape[1]), dtype=torch.float32, device=A.device)
    if C_out.dtype != torch.float32:
        raise ValueError("C must be float32")
    M, N, K, lda, ldb, ldc = _gemm_shapes(A, B, C_out)
    _check("mmm_gemm_naive_f16f32",
           lib().mmm_gemm_naive_f16f32(_ptr(A), _ptr(B), _ptr(C_out), M, N, K, lda, ldb, ldc, _stream(stream)))
    return C_out


def gemm_truth(A, B, with_scale: bool = True, stream=None):
    """fp64 T = A @ B and S = sum_k |a*b| on the device; returns (T, S) (S is None unless asked)."""
    import torch

    M, N = A.shape[0], B.shape[1]
    T = torch.empty((M, N), dtype=torch.float64, device=A.device)
    S = torch.empty_like(T) if with_scale else None
    M, N, K, lda, ldb, ldt = _gemm_shapes(A, B, T)
    _check("mmm_gemm_truth_f64",
           lib().mmm_gemm_truth_f64(_ptr(A), _ptr(B), _ptr(T), _ptr(S) if S is not None else None, M, N, K,
                                    lda, ldb, ldt, _stream(stream)))
    return T, S


def contract_truth(desc: "ContractDesc", A, B, T_out, S_out=None, stream=None):
    """fp64 truth (and scale) of a contraction, written at C's offsets into T_out / S_out."""
    import torch

    _check_f16("A", A)
    _check_f16("B", B)
    for t in (T_out, S_out):
        if t is not None and (t.dtype != torch.float64 or not t.is_cuda):
            raise TypeError("T and S must be CUDA float64 tensors")
    _check("mmm_contract5d_truth_f64",
           lib().mmm_contract5d_truth_f64(C.byref(desc), _ptr(A), _ptr(B), _ptr(T_out),
                                          _ptr(S_out) if S_out is not None else None, _stream(stream)))
    return T_out, S_out


def contract_desc_baseline(b: int, i: int, k: int, l: int, j: int) -> ContractDesc:
    d = ContractDesc()
    _check("mmm_contract_desc_baseline", lib().mmm_contract_desc_baseline(C.byref(d), b, i, k, l, j))
    return d


def contract_desc_reference(mt: int, bt: int, rt: int, nt: int, rt_l: int) -> ContractDesc:
    d = ContractDesc()
    _check("mmm_contract_desc_reference", lib().mmm_contract_desc_reference(C.byref(d), mt, bt, rt, nt, rt_l))
    return d


def contract(desc: ContractDesc, A, B, C_out, stream=None, workspace=None):
    """Runs the 5-D contraction described by desc (A, B fp16; C fp32; caller-shaped tensors).
    ``workspace`` as for gemm (used when the fold is a plain GEMM that splits K)."""
    import torch

    _check_f16("A", A)
    _check_f16("B", B)
    if C_out.dtype != torch.float32 or not C_out.is_cuda:
        raise TypeError("C must be a CUDA float32 tensor")
    st = _stream(stream)
    L = lib()
    wp, wb = _ws_args(workspace, A.device, st, MAX_WORKSPACE_BYTES)
    _check("mmm_contract5d_f16f32_ws",
           L.mmm_contract5d_f16f32_ws(C.byref(desc), _ptr(A), _ptr(B), _ptr(C_out), wp, wb, st))
    return C_out


def fill_uniform(t, seed: int, tensor_id: int, stream=None):
    """Fill fp16 tensor t with the seeded uniform[-1,1) stream (seed, tensor_id)."""
    _check_f16("t", t)
    _check("mmm_fill_uniform_f16", lib().mmm_fill_uniform_f16(_ptr(t), t.numel(), seed, tensor_id, _stream(stream)))
    return t


def fill_normal(t, seed: int, tensor_id: int, scale: float = 0.1, stream=None):
    """Fill fp16 tensor t with the seeded N(0,1)*scale stream (seed, tensor_id)."""
    _check_f16("t", t)
    _check("mmm_fill_normal_f16",
           lib().mmm_fill_normal_f16(_ptr(t), t.numel(), seed, tensor_id, scale, _stream(stream)))
    return t


def tile_of_block(block: int, tiles_m: int, tiles_n: int):
    tm, tn = C.c_int(), C.c_int()
    _check("mmm_tile_of_block", lib().mmm_tile_of_block(block, tiles_m, tiles_n, C.byref(tm), C.byref(tn)))
    return tm.value, tn.value


def version() -> str:
    return lib().mmm_version().decode()


# ------------------------------------------------------------------------------ measurement probes
def probe_clock(out, ticks: int = 2000, stream=None):
    """Enqueue the shader-clock probe (one wave spinning `ticks` ticks of the 100 MHz real-time
    counter); out is a CUDA int64 tensor of at least 2 elements receiving (shader cycles,
    real-time ticks).  clock_mhz(out) converts after a synchronisation."""
    import torch

    if out.dtype != torch.int64 or not out.is_cuda or out.numel() < 2:
        raise TypeError("out must be a CUDA int64 tensor of at least 2 elements")
    _check("mmm_probe_clock", lib().mmm_probe_clock(_ptr(out), ticks, _stream(stream)))
    return out


def clock_mhz(out) -> float:
    """Shader clock in MHz from a probe_clock result (host copy of the two counters)."""
    cyc, ticks = (int(v) for v in out[:2].tolist())
    return cyc / ticks * 100.0 if ticks > 0 else float("nan")


def probe_mfma_ceiling(A, B, C_out, store_tiles: bool = True, stream=None, clock=None):
    """The persistent 256x256 tile kernel's MFMA stream with register-resident operands (see
    include/mmm.h); 2*M*N*K flops per call, no operand traffic.  ``clock``: None, or a CUDA int64
    tensor of 4 elements receiving workgroup 0's start and end counters."""
    _check_f16("A", A)
    _check_f16("B", B)
    M, K = A.shape
    N = B.shape[1]
    ck = C.c_void_p(clock.data_ptr()) if clock is not None else None
    _check("mmm_probe_mfma_ceiling", lib().mmm_probe_mfma_ceiling(_ptr(A), _ptr(B), _ptr(C_out), M, N, K,
                                                                  1 if store_tiles else 0, ck, _stream(stream)))
    return C_out


def probe_lds_mfma(A, B, out=None, barrier: bool = True, stream=None, clock=None):
    """The persistent 256x256 tile kernel's fragment reads and MFMAs on operands already in LDS
    (see include/mmm.h); 2*M*N*K flops per call, no operand loads or C stores.  Returns the
    per-thread outputs (float32, min(M/256 * N/256, 256) * 512 of them).  ``clock``: None, or a
    CUDA int64 tensor of 4 elements receiving workgroup 0's start and end counters."""
    import torch

    _check_f16("A", A)
    _check_f16("B", B)
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[0] or not (A.is_contiguous() and B.is_contiguous()):
        raise ValueError("A must be a contiguous [M,K] and B a contiguous [K,N] tensor")
    M, K = A.shape
    N = B.shape[1]
    if out is None:
        out = torch.empty(min((M // 256) * (N // 256), 256) * 512, dtype=torch.float32, device=A.device)
    if out.dtype != torch.float32 or not out.is_cuda or not out.is_contiguous():
        raise TypeError("out must be a contiguous CUDA float32 tensor")
    ck = C.c_void_p(clock.data_ptr()) if clock is not None else None
    _check("mmm_probe_lds_mfma", lib().mmm_probe_lds_mfma(_ptr(A), _ptr(B), _ptr(out), out.numel(), M, N, K,
                                                          1 if barrier else 0, ck, _stream(stream)))
    return out


def probe_read(src, out, direct_to_lds: bool = False, stream=None):
    """Stream every byte of the CUDA tensor src once (plain 16-byte loads, or direct to LDS)."""
    nbytes = src.numel() * src.element_size()
    _check("mmm_probe_read", lib().mmm_probe_read(_ptr(src), nbytes, 1 if direct_to_lds else 0, _ptr(out),
                                                  out.numel() * out.element_size() // 4, _stream(stream)))
    return out


# ------------------------------------------------------------------------------ vendor witness
WITNESS_PATH = os.path.join(PKG_ROOT, "lib", "libmmm_witness.so")
_witness = None
_witness_ws = None


def _witness_lib():
    global _witness
    if _witness is None:
        lib()  # torch first, then this library, so both bind to torch's HIP runtime
        W = C.CDLL(WITNESS_PATH)
        p, i, i64, sz = C.c_void_p, C.c_int, C.c_int64, C.c_size_t
        W.mmm_witness_hipblaslt_gemm.restype = i
        W.mmm_witness_hipblaslt_gemm.argtypes = [p, p, p, i, i, i, i64, i64, i64, p, sz, p]
        W.mmm_witness_hipblaslt_create.restype = i
        W.mmm_witness_hipblaslt_create.argtypes = [i, i, i, i64, i64, i64, sz, C.POINTER(p)]
        W.mmm_witness_hipblaslt_run.restype = i
        W.mmm_witness_hipblaslt_run.argtypes = [p, p, p, p, p, sz, p]
        W.mmm_witness_hipblaslt_destroy.restype = None
        W.mmm_witness_hipblaslt_destroy.argtypes = [p]
        fp = C.POINTER(C.c_float)
        W.mmm_witness_hipblaslt_tune.restype = i
        W.mmm_witness_hipblaslt_tune.argtypes = [p, p, p, p, p, sz, p, i, C.POINTER(i), fp, fp]
        W.mmm_witness_hipblaslt_info.restype = i
        W.mmm_witness_hipblaslt_info.argtypes = [p, C.POINTER(i), C.POINTER(i)]
        _witness = W
    return _witness


def _witness_workspace(device):
    import torch

    global _witness_ws
    if _witness_ws is None:
        _witness_ws = torch.empty(64 << 20, dtype=torch.uint8, device=device)
    return _witness_ws


def witness_hipblaslt(A, B, C_out=None, stream=None):
    """hipBLASLt on the same FP16->FP32 row-major problem (comparison point only; plans the
    problem on every call -- use bind_witness_hipblaslt for timing)."""
    import torch

    W = _witness_lib()
    ws = _witness_workspace(A.device)
    M, K = A.shape
    N = B.shape[1]
    if C_out is None:
        C_out = torch.empty((M, N), dtype=torch.float32, device=A.device)
    rc = W.mmm_witness_hipblaslt_gemm(_ptr(A), _ptr(B), _ptr(C_out), M, N, K, A.stride(0), B.stride(0),
                                      C_out.stride(0), _ptr(ws), ws.numel(), _stream(stream))
    if rc != 0:
        raise MMMError("mmm_witness_hipblaslt_gemm", rc)
    return C_out


class _WitnessPlan:
    """A hipBLASLt plan (descriptors, layouts, up to 16 heuristic candidates) built once for one
    shape; its runs use the heuristic's first candidate until tune() binds the fastest."""

    def __init__(self, W, M, N, K, lda, ldb, ldc, ws_bytes):
        self._W = W
        self.ptr = C.c_void_p()
        rc = W.mmm_witness_hipblaslt_create(M, N, K, lda, ldb, ldc, ws_bytes, C.byref(self.ptr))
        if rc != 0:
            raise MMMError("mmm_witness_hipblaslt_create", rc)

    def info(self):
        n, chosen = C.c_int(), C.c_int()
        self._W.mmm_witness_hipblaslt_info(self.ptr, C.byref(n), C.byref(chosen))
        return n.value, chosen.value

    def tune(self, A, B, C_out, ws, stream=None, reps: int = 5):
        """Time every candidate on these operands (median of `reps` matmuls after one untimed)
        and bind the fastest; returns {"algos": n, "best_index": i, "ms": [...per candidate]}."""
        n, _ = self.info()
        each = (C.c_float * max(n, 1))()
        best, best_ms = C.c_int(), C.c_float()
        rc = self._W.mmm_witness_hipblaslt_tune(self.ptr, _ptr(A), _ptr(B), _ptr(C_out), _ptr(ws), ws.numel(),
                                                _stream(stream), reps, C.byref(best), C.byref(best_ms), each)
        if rc != 0:
            raise MMMError("mmm_witness_hipblaslt_tune", rc)
        return {"algos": n, "best_index": best.value, "ms": [round(each[i], 5) for i in range(n)]}

    def __del__(self):
        if getattr(self, "ptr", None) and self.ptr.value:
            self._W.mmm_witness_hipblaslt_destroy(self.ptr)


def bind_witness_hipblaslt(A, B, C_out, stream=None, tune: bool = True):
    """A zero-argument launcher of hipBLASLt's C = A @ B on fixed tensors and stream: the
    descriptors, layouts and up to 16 algorithm candidates are built once here, and each call is
    one hipblasLtMatmul -- the same footing as bind_gemm's launchers.  With tune (the default)
    every candidate is timed on these operands first and the fastest is bound (launch.tuning
    records the candidate count, the winner's index in the heuristic's order and each median);
    without it the heuristic's first candidate runs."""
    W = _witness_lib()
    ws = _witness_workspace(A.device)
    M, K = A.shape
    N = B.shape[1]
    plan = _WitnessPlan(W, M, N, K, A.stride(0), B.stride(0), C_out.stride(0), ws.numel())
    args = (plan.ptr, _ptr(A), _ptr(B), _ptr(C_out), _ptr(ws), ws.numel(), _stream(stream))
    launch = _bound(W.mmm_witness_hipblaslt_run, "mmm_witness_hipblaslt_run", args, (A, B, C_out, ws))
    launch.plan = plan  # keeps the plan alive as long as the launcher
    launch.tuning = plan.tune(A, B, C_out, ws, stream) if tune else {"algos": plan.info()[0], "best_index": 0}

    def with_operands(A2, B2, C2):
        """The same plan and bound candidate on other tensors of the same shapes and strides."""
        if (A2.shape, B2.shape, C2.shape) != (A.shape, B.shape, C_out.shape) or \
                (A2.stride(0), B2.stride(0), C2.stride(0)) != (A.stride(0), B.stride(0), C_out.stride(0)):
            raise ValueError("with_operands: shapes and row strides must match the bound plan")
        args2 = (plan.ptr, _ptr(A2), _ptr(B2), _ptr(C2), _ptr(ws), ws.numel(), _stream(stream))
        other = _bound(W.mmm_witness_hipblaslt_run, "mmm_witness_hipblaslt_run", args2, (A2, B2, C2, ws))
        other.plan, other.tuning = plan, launch.tuning
        return other

    launch.with_operands = with_operands
    return launch
