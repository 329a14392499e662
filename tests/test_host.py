"""Host-side tests (no GPU): the C ABI library loads and exports what include/mmm.h declares,
the descriptor presets encode the reference's layouts, the tile scheduler is a bijection,
and argument validation fails before any device work."""
import ctypes as C
import json
import os
import subprocess
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol(mm):
    declared = mm.declared_symbols()
    assert len(declared) >= 9
    L = mm.lib()
    for name in declared:
        assert hasattr(L, name), f"{name} declared in include/mmm.h but not exported"
    out = subprocess.run(["nm", "-D", "--defined-only", mm.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(declared) <= exported
    assert mm.version().startswith("mmm-gfx950")


def test_library_is_built_for_gfx950(mm):
    """The library (built here from this repository's sources) embeds a gfx950 code object."""
    data = open(mm.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


def test_contract_desc_baseline(mm):
    d = mm.contract_desc_baseline(8, 1024, 32, 64, 2048)
    assert (d.M, d.N, d.K) == (8192, 2048, 2048)
    A = np.zeros((8, 1024, 32, 64))
    B = np.zeros((32, 64, 2048))
    Cz = np.zeros((8, 1024, 2048))
    # strides (elements) of A[b,i,k,l], B[k,l,j], C[b,i,j]
    sa = [s // 8 for s in A.strides]
    sb = [s // 8 for s in B.strides]
    sc = [s // 8 for s in Cz.strides]
    assert tuple(d.a_m_stride) == (sa[0], sa[1]) and tuple(d.a_k_stride) == (sa[2], sa[3])
    assert tuple(d.b_k_stride) == (sb[0], sb[1]) and d.b_n_stride[1] == sb[2]
    assert tuple(d.c_m_stride) == (sc[0], sc[1]) and d.c_n_stride[1] == sc[2]


def test_contract_desc_reference(mm):
    """mmmTensor.cpp:20-28: G[r][n][m][l], Input[b][n][l], Out[m][b][r]; m' = m*rt + r, k' = n*rt_l + l."""
    mt, bt, rt, nt, rt_l = 128, 8192, 64, 64, 128
    d = mm.contract_desc_reference(mt, bt, rt, nt, rt_l)
    assert (d.M, d.N, d.K) == (mt * rt, bt, nt * rt_l)
    assert tuple(d.m_ext) == (mt, rt) and tuple(d.k_ext) == (nt, rt_l) and d.n_ext[1] == bt
    # pack index (mmmTensor.cpp:336): g_idx = r*nt*mt*rt_l + n*mt*rt_l + m*rt_l + l
    for (m, r, n, l) in [(3, 5, 7, 11), (127, 63, 63, 127)]:
        a_off = m * d.a_m_stride[0] + r * d.a_m_stride[1] + n * d.a_k_stride[0] + l * d.a_k_stride[1]
        assert a_off == r * nt * mt * rt_l + n * mt * rt_l + m * rt_l + l
    # TN read (mmmTensor.cpp:168): Input[b*DIM_K + k]
    for (b, n, l) in [(5, 2, 9), (8191, 63, 127)]:
        assert b * d.b_n_stride[1] + n * d.b_k_stride[0] + l * d.b_k_stride[1] == b * (nt * rt_l) + n * rt_l + l
    # output remap (mmmTensor.cpp:251): Out[m*bt*rt + b*rt + r]
    for (m, r, b) in [(2, 3, 4), (127, 63, 8191)]:
        assert m * d.c_m_stride[0] + r * d.c_m_stride[1] + b * d.c_n_stride[1] == m * bt * rt + b * rt + r


@pytest.mark.parametrize("tm,tn", [(t1, t2) for t1 in range(1, 41, 3) for t2 in range(1, 41, 5)] +
                         [(32, 32), (17, 16), (17, 32), (33, 16), (32, 8), (1, 64), (64, 1), (129, 3)])
def test_tile_map_bijection(mm, tm, tn):
    seen = np.zeros((tm, tn), dtype=np.int32)
    for b in range(tm * tn):
        i, j = mm.tile_of_block(b, tm, tn)
        assert 0 <= i < tm and 0 <= j < tn
        seen[i, j] += 1
    assert np.all(seen == 1)


def test_tile_map_xcd_locality(mm):
    """At 8192^3 (32 x 32 tiles of 256), the 32 workgroups one XCD runs first (ids x, x+8, ...)
    form a 4 x 8 tile patch: they share 4 A panels and 8 B panels in that XCD's L2."""
    for x in range(8):
        tiles = [mm.tile_of_block(x + 8 * s, 32, 32) for s in range(32)]
        rows = {t[0] for t in tiles}
        cols = {t[1] for t in tiles}
        assert len(rows) == 4 and len(cols) == 8


def test_argument_validation_without_gpu(mm):
    L = mm.lib()
    null = C.c_void_p(0)
    HIP_INVALID = mm.HIP_ERROR_INVALID_VALUE
    assert L.mmm_gemm_f16f32(null, null, null, 8, 8, 8, 8, 8, 8, null) == HIP_INVALID
    assert L.mmm_gemm_f16f32(null, null, null, -1, 8, 8, 8, 8, 8, null) == HIP_INVALID
    assert L.mmm_gemm_f16f32(null, null, null, 0, 8, 8, 8, 8, 8, null) == 0  # M == 0: no-op
    assert L.mmm_gemm_f16f32(null, null, null, 8, 0, 8, 8, 8, 8, null) == 0
    dummy = C.c_void_p(0x1000)
    assert L.mmm_gemm_f16f32(dummy, dummy, dummy, 8, 8, 8, 7, 8, 8, null) == HIP_INVALID  # lda < K
    assert L.mmm_gemm_f16f32(dummy, dummy, dummy, 8, 8, 8, 8, 7, 8, null) == HIP_INVALID  # ldb < N
    assert L.mmm_gemm_f16f32(dummy, dummy, dummy, 8, 8, 8, 8, 8, 7, null) == HIP_INVALID  # ldc < N
    assert L.mmm_gemm_f16f32_tiled(dummy, dummy, dummy, 8, 8, 8, 8, 8, 8, 2, 2, 4, 4, null, 0, null) == HIP_INVALID
    assert L.mmm_gemm_f16f32_tiled(dummy, dummy, dummy, 8, 8, 8, 8, 8, 8, 3, 4, 2, 2, null, 0, null) == HIP_INVALID
    # a workspace must be 16-byte aligned (checked before any launch)
    odd = C.c_void_p(0x1008)
    assert L.mmm_gemm_f16f32_ws(dummy, dummy, dummy, 8, 8, 8, 8, 8, 8, odd, 1 << 20, null) == HIP_INVALID
    assert L.mmm_gemm_f16f32_tiled(dummy, dummy, dummy, 8, 8, 8, 8, 8, 8, 2, 2, 2, 2, odd, 1 << 20, null) == HIP_INVALID
    assert L.mmm_gemm_f16f32_ws(null, null, null, 8, 8, 8, 8, 8, 8, null, 0, null) == HIP_INVALID
    assert L.mmm_gemm_workspace_f16f32(null, null, null, 8, 8, 8, 8, 8, 8, None) == HIP_INVALID
    d = mm.contract_desc_baseline(2, 3, 4, 5, 6)
    assert L.mmm_contract5d_f16f32(C.byref(d), null, null, null, null) == HIP_INVALID
    assert L.mmm_contract5d_f16f32(None, dummy, dummy, dummy, null) == HIP_INVALID
    assert L.mmm_contract5d_f16f32_ws(C.byref(d), dummy, dummy, dummy, odd, 1 << 20, null) == HIP_INVALID
    assert L.mmm_contract5d_workspace_f16f32(C.byref(d), null, null, null, None) == HIP_INVALID
    assert L.mmm_fill_uniform_f16(null, 10, 0, 0, null) == HIP_INVALID
    assert L.mmm_fill_uniform_f16(null, 0, 0, 0, null) == 0
    assert L.mmm_contract_desc_baseline(None, 1, 1, 1, 1, 1) == HIP_INVALID
    tm, tn = C.c_int(), C.c_int()
    assert L.mmm_tile_of_block(4, 2, 2, C.byref(tm), C.byref(tn)) == HIP_INVALID
    assert L.mmm_tile_of_block(0, 0, 2, C.byref(tm), C.byref(tn)) == HIP_INVALID
    # measurement probes validate before launching
    assert L.mmm_probe_clock(null, 2000, null) == HIP_INVALID
    assert L.mmm_probe_clock(dummy, 0, null) == HIP_INVALID
    assert L.mmm_probe_clock(dummy, 10 ** 8, null) == HIP_INVALID  # more than 100 ms of spinning
    assert L.mmm_probe_mfma_ceiling(dummy, dummy, dummy, 300, 256, 64, 1, null, null) == HIP_INVALID  # M % 256
    assert L.mmm_probe_mfma_ceiling(dummy, dummy, dummy, 256, 256, 96, 1, null, null) == HIP_INVALID  # K % 64
    assert L.mmm_probe_mfma_ceiling(null, dummy, dummy, 256, 256, 64, 1, null, null) == HIP_INVALID
    assert L.mmm_probe_mfma_ceiling(dummy, dummy, dummy, 256, 256, 64, 1, C.c_void_p(0x1004), null) == HIP_INVALID
    assert L.mmm_gemm_f16f32_clocked(dummy, dummy, dummy, 8, 8, 8, 8, 8, 8, null, 0, C.c_void_p(0x1004),
                                     null) == HIP_INVALID  # clock not 8-byte aligned
    assert L.mmm_gemm_f16f32_clocked(dummy, dummy, dummy, 8, 8, 8, 7, 8, 8, null, 0, null, null) == HIP_INVALID
    assert L.mmm_probe_read(dummy, 1000, 0, dummy, 1 << 20, null) == HIP_INVALID  # not a multiple of 1024
    assert L.mmm_probe_read(dummy, 1 << 20, 0, dummy, 100, null) == HIP_INVALID  # out too small
    assert L.mmm_probe_read(dummy, 1 << 31, 1, dummy, 1 << 20, null) == HIP_INVALID  # LDS path: < 2^31 bytes


def test_unaligned_rows_use_direct_to_lds(mm):
    """Rows that are only 2-byte aligned (odd lda / ldb) stay on the direct-to-LDS path: its
    16-byte buffer loads then run at 2-byte-aligned addresses, which MI355X serves in ROCm's
    unaligned memory mode (exact results: the full-size ragged GPU tests).  Odd byte addresses
    take the register-staged path."""
    for (M, N, K) in [(4097, 4095, 4111), (4096, 4096, 4111), (1000, 777, 333)]:
        p = mm.gemm_plan(M, N, K)
        assert p["direct_to_lds"] == 1, (M, N, K)
    assert mm.gemm_plan(4096, 4096, 4112, lda=4113)["direct_to_lds"] == 1
    assert mm.gemm_plan(300, 264, 200, A=3)["direct_to_lds"] == 0


def test_contract_descriptor_overflow_rejected(mm):
    """Extents whose product would overflow int64 (2^33 * 2^31) are rejected before they are
    multiplied, by every entry point that reads a descriptor (no GPU needed)."""
    L = mm.lib()
    HIP_INVALID = mm.HIP_ERROR_INVALID_VALUE
    dummy = C.c_void_p(0x1000)
    for field, ext in (("m_ext", (1 << 33, 1 << 31)), ("n_ext", (1 << 31, 1 << 33)), ("k_ext", (1 << 32, 1 << 32)),
                       ("m_ext", (1 << 31, 1))):
        d = mm.contract_desc_baseline(2, 3, 4, 5, 6)
        getattr(d, field)[0], getattr(d, field)[1] = ext
        need = C.c_size_t(7)
        assert L.mmm_contract5d_workspace_f16f32(C.byref(d), None, None, None, C.byref(need)) == HIP_INVALID, field
        assert L.mmm_contract5d_f16f32(C.byref(d), dummy, dummy, dummy, None) == HIP_INVALID, field
        assert L.mmm_contract5d_truth_f64(C.byref(d), dummy, dummy, dummy, None, None) == HIP_INVALID, field


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]


def test_header_is_plain_c():
    """include/mmm.h compiles as C (no torch or C++ types at the boundary)."""
    src = "#include \"mmm.h\"\nint main(void) { mmm_contract_desc d; (void)d; return 0; }\n"
    r = subprocess.run(["gcc", "-std=c99", "-x", "c", "-fsyntax-only", "-I", os.path.join(REPO, "include"),
                        "-I", "/opt/rocm/include", "-D__HIP_PLATFORM_AMD__", "-"], input=src, capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stderr


def test_cpp_header_drop_in(mm, tmp_path):
    """include/mmm.hpp (the reference's template spelling: WMMA_Swizzled_Full and the lineage's
    other names, GEMM_Naive) compiles and links against the library; with null pointers every
    entry point reports hipErrorInvalidValue (no GPU needed)."""
    src = tmp_path / "use_mmm.cpp"
    src.write_text("""
#include <cstdio>
#include "mmm.hpp"
int main() {
  int bad = 0;
  bad += mmm::WMMA_Swizzled_Full<2, 2, 4, 4>(nullptr, nullptr, nullptr, 64, 64, 64) != hipErrorInvalidValue;
  bad += mmm::WMMA_Swizzled_Full<4, 4, 4, 4>(nullptr, nullptr, nullptr, 64, 64, 64) != hipErrorInvalidValue;
  bad += mmm::WMMA_Templated_Base<2, 2, 4, 4>(nullptr, nullptr, nullptr, 64, 64, 64) != hipErrorInvalidValue;
  bad += mmm::WMMA_LDS_Padded<2, 2, 4, 4>(nullptr, nullptr, nullptr, 64, 64, 64) != hipErrorInvalidValue;
  bad += mmm::WMMA_LDS_Swizzled<2, 2, 4, 4>(nullptr, nullptr, nullptr, 64, 64, 64) != hipErrorInvalidValue;
  bad += mmm::GEMM_Naive(nullptr, nullptr, nullptr, 64, 64, 64) != hipErrorInvalidValue;
  bad += mmm::WMMA_Auto(nullptr, nullptr, nullptr, 8, 8, 8, 8, 8, 8) != hipErrorInvalidValue;
  bad += mmm::WMMA_Tensor(nullptr, nullptr, nullptr, 2, 3, 4, 5, 6) != hipErrorInvalidValue;
  std::printf("%d\\n", bad);
  return bad;
}
""")
    exe = tmp_path / "use_mmm"
    libdir = os.path.dirname(mm.LIB_PATH)
    r = subprocess.run(["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(REPO, "include"),
                        "-I", "/opt/rocm/include", str(src), "-o", str(exe), f"-L{libdir}", "-lmmm",
                        f"-Wl,-rpath,{libdir}"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "0", r.stdout + r.stderr


def test_cpp_header_float16_call_sites(mm, tmp_path):
    """With a compiler that has _Float16 (clang, as hipcc uses), include/mmm.hpp takes the
    reference's own operand types at its call sites -- _Float16* (mmm.cpp:1446-1447, 1496) and
    const _Float16* (mmmTensor.cpp:44-45) -- while a literal nullptr still resolves to the
    mmm_half forms; null pointers report hipErrorInvalidValue (no GPU needed)."""
    src = tmp_path / "use_f16.cpp"
    src.write_text("""
#include <cstdio>
#include "mmm.hpp"
int main() {
  _Float16* dA = nullptr;
  const _Float16* cG = nullptr;
  float* dC = nullptr;
  int bad = 0;
  bad += mmm::WMMA_Swizzled_Full<2, 2, 4, 4>(dA, dA, dC, 64, 64, 64) != hipErrorInvalidValue;
  bad += mmm::WMMA_Swizzled_Full<2, 2, 4, 4>(nullptr, nullptr, nullptr, 64, 64, 64) != hipErrorInvalidValue;
  bad += mmm::WMMA_Templated_Base<2, 2, 4, 4>(dA, dA, dC, 64, 64, 64) != hipErrorInvalidValue;
  bad += mmm::WMMA_LDS_Padded<2, 2, 4, 4>(dA, dA, dC, 64, 64, 64) != hipErrorInvalidValue;
  bad += mmm::WMMA_LDS_Swizzled<2, 2, 4, 4>(dA, dA, dC, 64, 64, 64) != hipErrorInvalidValue;
  bad += mmm::GEMM_Naive(cG, cG, dC, 64, 64, 64) != hipErrorInvalidValue;
  bad += mmm::WMMA_Auto(dA, cG, dC, 8, 8, 8, 8, 8, 8) != hipErrorInvalidValue;
  bad += mmm::WMMA_Tensor(cG, cG, dC, 2, 3, 4, 5, 6) != hipErrorInvalidValue;
  std::printf("%d\\n", bad);
  return bad;
}
""")
    exe = tmp_path / "use_f16"
    libdir = os.path.dirname(mm.LIB_PATH)
    r = subprocess.run(["/opt/rocm/llvm/bin/clang++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I",
                        os.path.join(REPO, "include"), "-I", "/opt/rocm/include", str(src), "-o", str(exe),
                        f"-L{libdir}", "-lmmm", f"-Wl,-rpath,{libdir}", "-L/opt/rocm/lib", "-lamdhip64"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "0", r.stdout + r.stderr


def test_isa_report(tmp_path):
    """Every gfx950 kernel: wave64, no VGPR spill or scratch, LDS within one CU's 160 KiB; the
    main tiles issue matrix-core ops and direct-to-LDS loads; the committed report lists them."""
    from mmm import isa

    rows = isa.collect(str(tmp_path))
    names = [r["kernel"] for r in rows]
    assert any(n.startswith("gemm_nn_kernel") for n in names)
    assert "gemm_skinny_kernel" in names
    assert any(n.startswith("check_fold_kernel") for n in names)
    for r in rows:
        assert r["wavefront"] == 64, r["kernel"]
        assert r["scratch"] == 0 and r["vgpr_spill"] == 0, r["kernel"]
        assert r["lds"] <= isa.LDS_PER_CU, r["kernel"]
        assert r["vgpr_total"] <= isa.VGPRS_PER_SIMD, r["kernel"]
        assert r["wg_per_cu"] >= 1, r["kernel"]
    main = [r for r in rows if r["kernel"].startswith("gemm_nn_kernel<Tile<256, 256, 2, 4")]
    assert main and main[0]["mfma"] > 0 and main[0]["dma_lds"] > 0
    committed = open(os.path.join(REPO, "profiles", "isa_resources.md")).read()
    missing = [n for n in names if f"`{n}`" not in committed]
    assert not missing, f"profiles/isa_resources.md is stale; regenerate it (missing {missing})"


def test_gemm_plan(mm):
    """The launch the library chooses, queried without a GPU (mmm_gemm_plan_f16f32)."""
    p = mm.gemm_plan(8192, 8192, 8192)
    assert p["kernel"] == "tile" and (p["block_m"], p["block_n"]) == (256, 256)
    assert p["tile_persistent"] == 1  # 1024 whole tiles: 256 workgroups loop over 4 each
    assert p["workspace_bytes"] == 0  # no K split
    assert mm.gemm_plan(4096, 4096, 4096)["tile_persistent"] == 0  # one round
    assert p["direct_to_lds"] == 1 and p["tile_workgroups"] == 32 * 32 and p["stream_rows"] == 0
    p = mm.gemm_plan(4097, 4095, 4111)  # one row past 16 tile rows: that row streams
    assert p["kernel"] == "tile+stream" and p["tile_rows"] == 4096 and p["stream_rows"] == 1
    # B rows 2-byte aligned: 128 strips of 32 columns, K reduced inside each workgroup
    assert p["stream_workgroups"] == 128 and p["stream_splits"] == 0 and p["stream_columns"] == 32
    p = mm.gemm_plan(4097, 4096, 4112)  # aligned rows: 32 strips of 128 columns, K split 8 ways
    assert p["stream_workgroups"] == 32 * 8 and p["stream_splits"] == 8 and p["stream_columns"] == 128
    # the in-workgroup kernel's bounds for M <= 16: B rows not 16-byte aligned, at least 128
    # strips of 32 columns (N >= 4065), B at most 64 MiB; otherwise the split kernel
    for (M, N, K, ldb), splits in [((16, 4065, 4111, None), 0), ((16, 4063, 4111, None), 8),
                                   ((16, 4095, 8193, None), 0), ((16, 4095, 8200, None), 8),
                                   ((16, 4095, 4111, 4096), 8), ((17, 4095, 4111, None), 8)]:
        assert mm.gemm_plan(M, N, K, ldb=ldb)["stream_splits"] == splits, (M, N, K, ldb)
    p = mm.gemm_plan(16, 8192, 8192)
    assert p["kernel"] == "stream" and p["stream_rows"] == 16 and p["tile_workgroups"] == 0
    # long K streams: 32 strips of 256 columns (512-byte row pieces), K split 8 ways
    assert p["stream_splits"] == 8 and p["stream_workgroups"] == 32 * 8 and p["stream_columns"] == 256
    assert p["workspace_bytes"] == 32 * 8 * 16 * 256 * 4  # [strip][split][16][256] fp32 partials
    need = C.c_size_t(0)
    assert mm.lib().mmm_gemm_workspace_f16f32(None, None, None, 16, 8192, 8192, 8192, 8192, 8192,
                                              C.byref(need)) == 0 and need.value == p["workspace_bytes"]
    # too little K to split: 32-column strips, K split among each workgroup's waves
    p = mm.gemm_plan(16, 8192, 128)
    assert p["stream_splits"] == 0 and p["stream_workgroups"] == 8192 // 32 and p["stream_columns"] == 32
    # 256-column strips only where each wave streams >= 256 K rows (512 for more than 16 rows),
    # K >= 8192 and the 128-column grid is split; otherwise 128 columns
    for (M, N, K), cols in [((16, 16384, 8192), 256), ((1, 8192, 28672), 256), ((13, 8200, 8192), 256),
                            ((16, 4096, 8192), 128), ((16, 4096, 14336), 128), ((16, 14336, 4096), 128),
                            ((16, 28672, 8192), 128), ((17, 8192, 8192), 128), ((32, 8192, 16384), 256),
                            ((20, 16384, 8192), 256), ((32, 8192, 12288), 128), ((33, 16384, 16384), 256),
                            ((64, 8192, 16384), 256), ((48, 8192, 12288), 128), ((64, 8192, 8192), 128)]:
        assert mm.gemm_plan(M, N, K)["stream_columns"] == cols, (M, N, K)
    assert mm.gemm_plan(16, 8192, 8192, ldb=8196)["stream_columns"] == 128  # B rows not 16-byte aligned
    assert mm.gemm_plan(8192, 8192, 8192)["stream_columns"] == 0
    # the split grid stays within one round of 256 workgroups: 112 strips x 2, not x 3
    p = mm.gemm_plan(24, 14336, 4096)
    assert p["kernel"] == "stream" and p["stream_splits"] == 2 and p["stream_workgroups"] == 224
    p = mm.gemm_plan(32, 28672, 8192)  # 224 strips fill the chip unsplit
    assert p["stream_splits"] == 1 and p["stream_workgroups"] == 224
    # 33-64 rows: from an unsplit 128-column grid to 256 columns on long K; short K over many
    # strips (2-3 splits, K <= 4096) on 64 x 64 tiles
    p = mm.gemm_plan(64, 28672, 8192)
    assert p["stream_columns"] == 256 and p["stream_splits"] == 2 and p["stream_workgroups"] == 224
    for (M, N, K), kernel in [((64, 14336, 4096), "tile"), ((40, 11008, 4096), "tile"), ((64, 16384, 4096), "tile"),
                              ((64, 10240, 8192), "stream"), ((64, 6144, 4096), "stream"), ((32, 14336, 4096), "stream")]:
        p = mm.gemm_plan(M, N, K)
        assert p["kernel"] == kernel, (M, N, K, p["kernel"])
        if kernel == "tile":
            assert (p["block_m"], p["block_n"]) == (64, 64) and p["stream_rows"] == 0
    assert mm.gemm_plan(65, 8192, 8192)["kernel"] == "tile"
    # more 128-column strips than CUs: B rows that are not 16-byte aligned, or rounds less than 2/3
    # filled on average, run on the tile kernels; fuller rounds stream unsplit
    for (M, N, K), kernel in [((16, 33001, 8192), "tile"), ((64, 50257, 4096), "tile"), ((16, 33000, 8192), "tile"),
                              ((16, 40000, 8192), "tile"), ((16, 49152, 8192), "stream"), ((32, 81920, 4096), "stream"),
                              ((16, 151936, 4096), "stream"), ((16, 65536, 4096), "stream")]:
        p = mm.gemm_plan(M, N, K)
        assert p["kernel"] == kernel, (M, N, K, p["kernel"])
        if kernel == "stream":
            assert p["stream_splits"] == 1 and p["stream_workgroups"] == (N + 127) // 128
    # grids too small for 128x128 tiles to fill the chip take 64x64 tiles (1024^3: 256 of them)
    p = mm.gemm_plan(1024, 1024, 1024)
    assert (p["block_m"], p["block_n"], p["wave_m"], p["wave_n"], p["tile_workgroups"]) == (64, 64, 1, 1, 256)
    assert mm.gemm_plan(2048, 2048, 2048)["block_m"] == 128  # a full round of 128x128 tiles
    # under-filled last round: 576 tiles = 2 rounds + 64; those 64 run as 4 K ranges each
    p = mm.gemm_plan(6144, 6144, 6144)
    assert (p["block_m"], p["tile_splits"], p["tile_split_tiles"], p["tile_workgroups"]) == (256, 4, 64, 576)
    assert p["workspace_bytes"] == 64 * 4 * 256 * 256 * 4  # [split tile][split][256][256] fp32
    p = mm.gemm_plan(6150, 6144, 1030)  # short K: the reduction would cost more than it saves
    assert (p["tile_splits"], p["tile_split_tiles"]) == (1, 0)
    p = mm.gemm_plan(16 * 256 + 40, 4096, 264)  # 40 rows past 16 tile rows stream
    assert p["kernel"] == "tile+stream" and p["tile_rows"] == 4096 and p["stream_rows"] == 40
    assert mm.gemm_plan(5, 5, 0)["kernel"] == "zero"
    assert mm.gemm_plan(0, 5, 5)["kernel"] == "none"
    # odd addresses cannot use the direct-to-LDS loads or the streaming kernel
    p = mm.gemm_plan(300, 264, 200, A=3)
    assert p["kernel"] == "tile" and p["direct_to_lds"] == 0
    assert mm.gemm_plan(8, 64, 64, A=3)["kernel"] == "tile"
    for shape in [(256, 256, 256), (1000, 3000, 70), (8192, 2048, 2048), (65, 4096, 4096), (6000, 200, 50)]:
        p = mm.gemm_plan(*shape)
        assert (p["wave_m"], p["wave_n"], p["waves_i"], p["waves_j"]) in mm.TILES.values()
        assert p["block_m"] == p["waves_i"] * p["wave_m"] * 32 and p["block_n"] == p["waves_j"] * p["wave_n"] * 32
    with pytest.raises(mm.MMMError):
        mm.gemm_plan(64, 64, 64, lda=32)
    with pytest.raises(mm.MMMError):
        mm.gemm_plan(-1, 64, 64)


@pytest.mark.parametrize("fm,fn", [(8, 4), (4, 4), (2, 2), (6, 3)])
def test_line_store_lane_map(fm, fn):
    """The whole-line C epilogue (store_wave_tile_lines in mmm_gemm.hip), restated lane by lane:
    a 16x16x32 accumulator block gives lane l row l % 16 and columns 4*(l//16) .. +3; lanes l and
    l ^ 8 trade their block-(nb+1) values, lanes with (l & 8) == 0 store rows 0-7 of the pair
    from block nb and rows 8-15 from the traded values, the others the reverse.  Every element of
    the wave tile is written exactly once with its own value, and each paired store instruction
    covers 8 rows x 32 consecutive floats (whole 128-byte lines); an odd last block (fn = 3, the
    192x192 tile) is stored as before, 16 rows x 16 floats."""
    ldc = 1000  # any row pitch
    lanes = np.arange(64)
    # acc[mb][nb][e] of lane l holds the value C[16 mb + l % 16][16 nb + 4 (l // 16) + e]
    def value(r, c):
        return r * 100000 + c
    acc = np.zeros((fm, fn, 64, 4), dtype=np.int64)
    for mb in range(fm):
        for nb in range(fn):
            for e in range(4):
                acc[mb, nb, :, e] = value(16 * mb + lanes % 16, 16 * nb + 4 * (lanes // 16) + e)
    written = {}
    lo = (lanes & 8) == 0
    r0 = (lanes & 7) * ldc + 4 * (lanes >> 4) + np.where(lo, 0, 16)
    r1 = ((lanes & 7) + 8) * ldc + 4 * (lanes >> 4) + np.where(lo, 16, 0)
    for mb in range(fm):
        for nb in range(0, fn - 1, 2):
            traded = acc[mb, nb + 1][lanes ^ 8]
            rows_lo = np.where(lo[:, None], acc[mb, nb], traded)
            rows_hi = np.where(lo[:, None], traded, acc[mb, nb])
            for base, data in ((r0, rows_lo), (r1, rows_hi)):
                addr = base + 16 * mb * ldc + 16 * nb
                cols = set()
                for l in range(64):
                    for e in range(4):
                        a = int(addr[l]) + e
                        assert a not in written
                        written[a] = int(data[l, e])
                        cols.add(a)
                rows = {a // ldc for a in cols}
                assert len(rows) == 8  # 8 rows ...
                for rr in rows:  # ... of 32 consecutive floats each
                    rc = sorted(a % ldc for a in cols if a // ldc == rr)
                    assert rc == list(range(rc[0], rc[0] + 32))
        if fn % 2:
            nb = fn - 1
            for l in range(64):
                for e in range(4):
                    a = (16 * mb + l % 16) * ldc + 16 * nb + 4 * (l // 16) + e
                    assert a not in written
                    written[a] = int(acc[mb, nb, l, e])
    assert len(written) == fm * 16 * fn * 16
    for a, v in written.items():
        assert v == value(a // ldc, a % ldc)


def test_bench_shape_sets():
    """bench.py's sweep shape sets and its rotating launcher (no GPU)."""
    sys.path.insert(0, REPO)
    import bench

    assert bench.parse_shapes("llm") == bench.SWEEP_SHAPES_LLM
    decode = bench.parse_shapes("decode")
    assert len(decode) == 32 and all(1 <= m <= 64 for m, _, _ in decode)
    small = bench.parse_shapes("small_m")
    assert len(small) == 40 and all(128 < m <= 256 for m, _, _ in small)
    assert bench.parse_shapes("16x8192x8192, 1x2x3") == [(16, 8192, 8192), (1, 2, 3)]
    with pytest.raises(ValueError):
        bench.parse_shapes("1x2")
    calls = []
    launch = bench._cycle([lambda: calls.append(0), lambda: calls.append(1), lambda: calls.append(2)])
    for _ in range(7):
        launch()
    assert calls == [0, 1, 2, 0, 1, 2, 0]
    single = lambda: None
    assert bench._cycle([single]) is single
