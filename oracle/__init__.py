"""CPU oracle for the FP16->FP32 GEMM / 5-D contraction path (ctypes over oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg may import this package, and only as the checker (or the timed CPU
baseline).  The product (``rdna4-gemm-wmma_amd/``) never imports it.

Every routine restates a part of thrasos-g/RDNA4-GEMM-WMMA; the citations are in
``oracle.c``.  fp16 tensors are numpy ``float16`` arrays (IEEE binary16 bits).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

_i64 = C.c_int64
_p = C.c_void_p


def build() -> None:
    """Compile oracle.c (gcc + OpenMP) into _build/liboracle.so."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f64_to_f16.restype = C.c_uint16
        L.orc_f64_to_f16.argtypes = [C.c_double]
        for name in ("orc_f32_to_f16_array", "orc_f64_to_f16_array", "orc_f16_to_f32_array"):
            getattr(L, name).argtypes = [_p, _p, _i64]
            getattr(L, name).restype = None
        L.orc_splitmix64.restype = C.c_uint64
        L.orc_splitmix64.argtypes = [C.c_uint64]
        L.orc_fill_uniform_f16.argtypes = [_p, _i64, C.c_uint64, C.c_uint32]
        L.orc_fill_uniform_f16.restype = None
        L.orc_fill_normal_f16.argtypes = [_p, _i64, C.c_uint64, C.c_uint32, C.c_double]
        L.orc_fill_normal_f16.restype = None
        L.orc_gemm_f64_sub.argtypes = [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _p]
        L.orc_gemm_f64_sub.restype = None
        L.orc_gemm_naive_f32_sub.argtypes = [_p, _i64, _p, _i64, _i64, _p, _i64, _p, _i64, _p]
        L.orc_gemm_naive_f32_sub.restype = None
        L.orc_gemm_refkernel_f32_sub.argtypes = [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _p, _i64, _p]
        L.orc_gemm_refkernel_f32_sub.restype = None
        L.orc_contract_baseline_f64.argtypes = [_p, _p, _i64, _i64, _i64, _i64, _p, _i64, _p, _p]
        L.orc_contract_baseline_f64.restype = None
        L.orc_contract_reference_f64.argtypes = [_p, _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p, _p]
        L.orc_contract_reference_f64.restype = None
        L.orc_pack_reference_G.argtypes = [_p, _p, _i64, _i64, _i64, _i64]
        L.orc_pack_reference_G.restype = None
        L.orc_ref_block_remap.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]
        L.orc_ref_block_remap.restype = None
        L.orc_check_tol.argtypes = [_p, _i64, _p, _p, _i64, _i64, C.c_double, C.POINTER(C.c_double)]
        L.orc_check_tol.restype = _i64
        L.orc_cpu_gemm_f16f32.argtypes = [_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, C.c_int]
        L.orc_cpu_gemm_f16f32.restype = None
        L.orc_max_threads.restype = C.c_int
        L.orc_max_threads.argtypes = []
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _idx(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.int64))


# ---------------------------------------------------------------- conversions / PRNG
def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out.view(np.float16)


def f64_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f64_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out.view(np.float16)


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h).view(np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


def splitmix64(z: int) -> int:
    return int(lib().orc_splitmix64(C.c_uint64(z & 0xFFFFFFFFFFFFFFFF)))


def uniform_f16(shape, seed: int, tensor_id: int) -> np.ndarray:
    """fp16 tensor, values uniform in [-1, 1) from the counter-based stream (seed, tensor_id)."""
    out = np.empty(shape, dtype=np.float16)
    lib().orc_fill_uniform_f16(_ptr(out), out.size, seed, tensor_id)
    return out


def normal_f16(shape, seed: int, tensor_id: int, scale: float = 0.1) -> np.ndarray:
    """fp16 tensor, values N(0,1)*scale (Box-Muller) from the stream (seed, tensor_id)."""
    out = np.empty(shape, dtype=np.float16)
    lib().orc_fill_normal_f16(_ptr(out), out.size, seed, tensor_id, scale)
    return out


# ---------------------------------------------------------------- GEMM truth / restatements
def gemm_f64(A: np.ndarray, B: np.ndarray, rows=None, cols=None, b_layout: str = "kn"):
    """fp64 truth C = A @ B and S = sum_k |a*b| on the sub-grid rows x cols.

    A is [M][K] (row-major).  B is [K][N] for b_layout "kn" (mmm.cpp) or [N][K] for "nk"
    (the TN read of mmmTensor.cpp:168).
    """
    A = np.ascontiguousarray(A, dtype=np.float16)
    B = np.ascontiguousarray(B, dtype=np.float16)
    M, K = A.shape
    if b_layout == "kn":
        Kb, N = B.shape
        bks, bns = N, 1
    else:
        N, Kb = B.shape
        bks, bns = 1, Kb
    assert Kb == K
    rows = _idx(np.arange(M) if rows is None else rows)
    cols = _idx(np.arange(N) if cols is None else cols)
    Cm = np.empty((rows.size, cols.size), dtype=np.float64)
    S = np.empty_like(Cm)
    lib().orc_gemm_f64_sub(_ptr(A), K, 1, _ptr(B), bks, bns, K, _ptr(rows), rows.size, _ptr(cols), cols.size,
                           _ptr(Cm), _ptr(S))
    return Cm, S


def gemm_naive_f32(A: np.ndarray, B: np.ndarray, rows=None, cols=None) -> np.ndarray:
    """GEMM_Naive (mmm.cpp:52-62): fp32 accumulator, k ascending."""
    A = np.ascontiguousarray(A, dtype=np.float16)
    B = np.ascontiguousarray(B, dtype=np.float16)
    M, K = A.shape
    N = B.shape[1]
    rows = _idx(np.arange(M) if rows is None else rows)
    cols = _idx(np.arange(N) if cols is None else cols)
    out = np.empty((rows.size, cols.size), dtype=np.float32)
    lib().orc_gemm_naive_f32_sub(_ptr(A), K, _ptr(B), N, K, _ptr(rows), rows.size, _ptr(cols), cols.size, _ptr(out))
    return out


def gemm_refkernel_f32(A: np.ndarray, B: np.ndarray, rows=None, cols=None, b_layout: str = "kn") -> np.ndarray:
    """WMMA_Swizzled_Full's arithmetic (mmm.cpp:1309-1356): 32-deep LDS tiles, 16-deep steps."""
    A = np.ascontiguousarray(A, dtype=np.float16)
    B = np.ascontiguousarray(B, dtype=np.float16)
    M, K = A.shape
    if b_layout == "kn":
        N = B.shape[1]
        bks, bns = N, 1
    else:
        N = B.shape[0]
        bks, bns = 1, K
    rows = _idx(np.arange(M) if rows is None else rows)
    cols = _idx(np.arange(N) if cols is None else cols)
    out = np.empty((rows.size, cols.size), dtype=np.float32)
    lib().orc_gemm_refkernel_f32_sub(_ptr(A), K, 1, _ptr(B), bks, bns, K, _ptr(rows), rows.size, _ptr(cols),
                                     cols.size, _ptr(out))
    return out


# ---------------------------------------------------------------- contractions
def contract_baseline_f64(A: np.ndarray, B: np.ndarray, bi=None):
    """C[b,i,j] = sum_{k,l} A[b,i,k,l] B[k,l,j] as a loop nest; returns (C, S) [len(bi)][nj]."""
    A = np.ascontiguousarray(A, dtype=np.float16)
    B = np.ascontiguousarray(B, dtype=np.float16)
    nb, ni, nk, nl = A.shape
    nk2, nl2, nj = B.shape
    assert (nk2, nl2) == (nk, nl)
    bi = _idx(np.arange(nb * ni) if bi is None else bi)
    Cm = np.empty((bi.size, nj), dtype=np.float64)
    S = np.empty_like(Cm)
    lib().orc_contract_baseline_f64(_ptr(A), _ptr(B), ni, nk, nl, nj, _ptr(bi), bi.size, _ptr(Cm), _ptr(S))
    return Cm, S


def contract_reference_f64(G: np.ndarray, In: np.ndarray, mr=None):
    """Out[m][b][r] = sum_{n,l} G[r][n][m][l] In[b][n][l] (mmmTensor.cpp); returns (C, S) [len(mr)][bt]."""
    G = np.ascontiguousarray(G, dtype=np.float16)
    In = np.ascontiguousarray(In, dtype=np.float16)
    rt, nt, mt, rt_l = G.shape
    bt, nt2, rl2 = In.shape
    assert (nt2, rl2) == (nt, rt_l)
    mr = _idx(np.arange(mt * rt) if mr is None else mr)
    Cm = np.empty((mr.size, bt), dtype=np.float64)
    S = np.empty_like(Cm)
    lib().orc_contract_reference_f64(_ptr(G), _ptr(In), mt, bt, rt, nt, rt_l, _ptr(mr), mr.size, _ptr(Cm), _ptr(S))
    return Cm, S


def pack_reference_G(G: np.ndarray) -> np.ndarray:
    """The reference's host pack (mmmTensor.cpp:329-340): A[(m*rt+r)][(n*rt_l+l)] = G[r][n][m][l]."""
    G = np.ascontiguousarray(G, dtype=np.float16)
    rt, nt, mt, rt_l = G.shape
    out = np.empty((mt * rt, nt * rt_l), dtype=np.float16)
    lib().orc_pack_reference_G(_ptr(G), _ptr(out), mt, rt, nt, rt_l)
    return out


def ref_block_remap(bx: int, by: int, gx: int, gy: int):
    """The reference's block remap (mmm.cpp:1219-1236)."""
    sx, sy = C.c_int(), C.c_int()
    lib().orc_ref_block_remap(bx, by, gx, gy, C.byref(sx), C.byref(sy))
    return sx.value, sy.value


# ---------------------------------------------------------------- tolerance / CPU baseline
TOL_REL = 1e-3  # |C - C_ref| <= 1e-3 * sum_k |a_ik * b_kj|


def check_tol(Cv: np.ndarray, T: np.ndarray, S: np.ndarray, rel: float = TOL_REL):
    """Count elements violating |C - T| <= rel * S; returns (violations, worst |C-T|/S)."""
    Cv = np.ascontiguousarray(Cv, dtype=np.float32)
    T = np.ascontiguousarray(T, dtype=np.float64)
    S = np.ascontiguousarray(S, dtype=np.float64)
    assert Cv.shape == T.shape == S.shape
    nr, nc = T.shape
    worst = C.c_double()
    bad = lib().orc_check_tol(_ptr(Cv), nc, _ptr(T), _ptr(S), nr, nc, rel, C.byref(worst))
    return int(bad), float(worst.value)


def cpu_gemm_f16f32(A: np.ndarray, B: np.ndarray, threads: int = 0) -> np.ndarray:
    """Multithreaded CPU FP16->FP32 GEMM (F16C convert + AVX2/FMA 6x16 micro-kernel)."""
    A = np.ascontiguousarray(A, dtype=np.float16)
    B = np.ascontiguousarray(B, dtype=np.float16)
    M, K = A.shape
    N = B.shape[1]
    out = np.empty((M, N), dtype=np.float32)
    lib().orc_cpu_gemm_f16f32(_ptr(A), K, _ptr(B), N, _ptr(out), N, M, N, K, threads)
    return out


def max_threads() -> int:
    return int(lib().orc_max_threads())
