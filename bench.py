#!/usr/bin/env python3
"""Benchmark of the MI355X FP16->FP32 GEMM / 5-D contraction (one GPU).

Driver contract: ``python bench.py --gpus N --steps K --warmup W`` prints ONE JSON line.
A step is one launch of the hot path over one batch of synthetic input already resident
in HBM.  The default workload is BASELINE configs[1]: the 8192^3 row-major GEMM with
inputs uniform in [-1, 1) from seed 1 (generated on the device by the library's seeded
generator).  ``value`` is TFLOP/s (2*M*N*K per step over the timed region).

Extra objects on the line:
  roofline     -- the dominant kernel's achieved rate (algorithmic flops, or bytes for the
                  HBM-bound skinny shape, per launch over the average launch duration measured
                  with HIP events on the launch stream) against MI355X's published peak
                  (dense FP16 MFMA 2516.6 TFLOP/s = 256 CU x 4096 flop/clk x 2.4 GHz; HBM3E
                  8 TB/s); `traffic` is the HBM bytes per launch from rocprofv3 FETCH_SIZE +
                  WRITE_SIZE (read from profiles/, null when not measured for the workload).
  cpu_baseline -- the oracle's multithreaded CPU FP16->FP32 GEMM on a bounded sample of the
                  same workload, on this host's cores (reported only).
  hipblaslt    -- hipBLASLt on the same inputs and problem (FP16 in, FP32 out): the fastest of
                  its heuristic's (up to 16) candidates, each timed on these inputs first.
  validation   -- one step's output checked in full on the device against the fp64 truth:
                  |C - T| <= 1e-3 * sum_k |a*b| for every element (violations must be 0).

Order of a run: the validation and hipBLASLt's candidate search come first (`before_timing_s`
is how long they kept the GPU busy), then the W untimed and K timed steps, then hipBLASLt's W
and K, the MFMA-ceiling probe and the CPU baseline.

Other workloads (parity configs, reported with --workload or --report, never the default):
gemm256, ragged, contraction, skinny (and skinny_nows, the same problem without a workspace),
contraction_ref (and contraction_ref_rtl120 / contraction_ref_big, its fold variants with K tiles
crossing n blocks and with a G of 2 GiB).  One GPU only: --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import itertools
import json
import os
import re
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "rdna4-gemm-wmma_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "FP16→FP32 GEMM TFLOP/s at 8192³; % of MI355X dense FP16 MFMA peak"
PEAK_TFLOPS = 2516.6  # 256 CU x 4096 flop/clk x 2.4 GHz, dense FP16 MFMA
PEAK_GBS = 8000.0     # HBM3E

WORKLOADS = {
    # name: (M, N, K, kind, seed, dist)
    "gemm256": (256, 256, 256, "gemm", 0, "uniform"),
    "gemm8192": (8192, 8192, 8192, "gemm", 1, "uniform"),
    "ragged": (4097, 4095, 4111, "gemm", 2, "uniform"),
    "contraction": (8192, 2048, 2048, "contraction", 3, "normal"),
    "skinny": (16, 8192, 8192, "gemm", 4, "uniform"),
    # the same problem through the entry point without a workspace (K reduced inside each workgroup)
    "skinny_nows": (16, 8192, 8192, "gemm", 4, "uniform"),
    # the reference's own contraction (mmmTensor.cpp:20-28): G[r][n][m][l] x Input[b][n][l]
    "contraction_ref": (8192, 8192, 8192, "contraction_ref", 5, "uniform"),
    # the same program with rt_l = 120 (K tiles cross n blocks) and with a G of 2 GiB (past the
    # buffer loads' 32-bit offsets)
    "contraction_ref_rtl120": (8192, 8192, 7680, "contraction_ref", 5, "uniform"),
    "contraction_ref_big": (8192, 16384, 131072, "contraction_ref", 5, "uniform"),
    # known-size reference for the HBM byte counters: a 256 MiB fp32 device-to-device copy
    "copy": (8192, 8192, 1, "copy", 0, "uniform"),
    # measured ceilings (library probes): the 8192^3 tile kernel's MFMA stream with register-
    # resident operands, and streaming reads of 1 GiB (plain loads / direct to LDS)
    "mfma_ceiling": (8192, 8192, 8192, "mfma_ceiling", 1, "uniform"),
    # the same kernel's fragment reads and MFMAs on operands already in LDS (no operand loads or C
    # stores), with and without its one workgroup barrier per K tile
    "lds_mfma": (8192, 8192, 8192, "lds_mfma", 1, "uniform"),
    "lds_mfma_nobarrier": (8192, 8192, 8192, "lds_mfma_nobarrier", 1, "uniform"),
    "read_ceiling": (1 << 30, 1, 1, "read", 0, "uniform"),
    "read_ceiling_lds": (1 << 30, 1, 1, "read_lds", 0, "uniform"),
}
DESCRIPTIONS = {
    "gemm256": "gemm_nn 256x256x256 fp16 row-major, U[-1,1) seed 0",
    "gemm8192": "gemm_nn 8192x8192x8192 fp16 row-major, U[-1,1) seed 1",
    "ragged": "gemm_nn 4097x4095x4111 fp16 row-major, U[-1,1) seed 2",
    "contraction": "contract5d C[b,i,j]=sum_kl A[b,i,k,l] B[k,l,j], b=8 i=1024 k=32 l=64 j=2048, N(0,1)*0.1 seed 3",
    "skinny": "gemm_nn 16x8192x8192 fp16 row-major, U[-1,1) seed 4, 3 rotating B buffers",
    "skinny_nows": "gemm_nn 16x8192x8192 fp16 row-major without a workspace, U[-1,1) seed 4, 3 rotating B buffers",
    "contraction_ref": "contract5d Out[m][b][r]=sum_nl G[r][n][m][l] In[b][n][l], mt=128 bt=8192 rt=64 nt=64 rt_l=128, "
                       "U[-1,1) seed 5",
    "contraction_ref_rtl120": "contract5d Out[m][b][r]=sum_nl G[r][n][m][l] In[b][n][l], mt=128 bt=8192 rt=64 nt=64 "
                              "rt_l=120, U[-1,1) seed 5",
    "contraction_ref_big": "contract5d Out[m][b][r]=sum_nl G[r][n][m][l] In[b][n][l], mt=128 bt=16384 rt=64 nt=1024 "
                           "rt_l=128 (G 2 GiB), U[-1,1) seed 5",
    "copy": "copy 256 MiB fp32 device-to-device (counter scaling reference), zeros",
    "mfma_ceiling": "MFMA ceiling probe: the 8192x8192x8192 persistent tile kernel's MFMA stream and C stores with "
                    "register-resident operands (no loads, LDS or barriers), U[-1,1) seed 1",
    "lds_mfma": "operand-path probe: the 8192x8192x8192 persistent tile kernel's fragment reads and MFMAs on "
                "operands staged in LDS once, with its per-K-tile barrier (no operand loads, no C stores), "
                "U[-1,1) seed 1",
    "lds_mfma_nobarrier": "operand-path probe: the 8192x8192x8192 persistent tile kernel's fragment reads and MFMAs "
                          "on operands staged in LDS once, no barrier (no operand loads, no C stores), U[-1,1) seed 1",
    "read_ceiling": "HBM read ceiling probe: one pass over 1 GiB with non-temporal 16-byte loads into registers "
                    "(8192 workgroups, 4 in flight per lane), zeros",
    "read_ceiling_lds": "HBM read ceiling probe: one pass over 1 GiB with direct-to-LDS 16-byte loads (8192 "
                        "workgroups, 32-slot rings), zeros",
}


# (mt, bt, rt, nt, rt_l) of the reference-layout contraction workloads (mmmTensor.cpp:20-24)
REFERENCE_DIMS = {
    "contraction_ref": (128, 8192, 64, 64, 128),
    "contraction_ref_rtl120": (128, 8192, 64, 64, 120),
    "contraction_ref_big": (128, 16384, 64, 1024, 128),
}


def data_description(name: str) -> str:
    """The distribution and seed part of a workload's description ("U[-1,1) seed 1", "zeros")."""
    m = re.search(r"(U\[-1,1\) seed \d+|N\(0,1\)\*0\.1 seed \d+|zeros)", DESCRIPTIONS[name])
    return DESCRIPTIONS[name][m.start():] if m else DESCRIPTIONS[name]


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# the GEMM given by --shape (and --tile): U[-1,1) inputs from seed 7, as in the tile sweep
SHAPE_SEED = 7


def make_workload(name, torch, mmm, tile=None):
    """Device inputs and a launch closure for one step of the named workload (`tile`: a block tile
    forced on a GEMM workload instead of the library's pick)."""
    M, N, K, kind, seed, dist = WORKLOADS[name]
    dev = "cuda"
    fill = mmm.fill_uniform if dist == "uniform" else (lambda t, s, i: mmm.fill_normal(t, s, i, 0.1))
    if kind == "copy":
        src = torch.zeros((M, N), dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        return {"launch": lambda: dst.copy_(src), "witness": None, "host_inputs": None, "M": M, "N": N, "K": K,
                "bytes": 2.0 * src.numel() * 4}
    if kind in ("read", "read_lds"):
        src = torch.zeros(M, dtype=torch.uint8, device=dev)
        out = torch.empty(8192 * 256, dtype=torch.int32, device=dev)
        lds = kind == "read_lds"
        return {"launch": lambda: mmm.probe_read(src, out, direct_to_lds=lds), "witness": None, "host_inputs": None,
                "M": M, "N": N, "K": K, "bytes": float(M)}
    if kind == "mfma_ceiling":
        A = torch.empty((M, K), dtype=torch.float16, device=dev)
        B = torch.empty((K, N), dtype=torch.float16, device=dev)
        fill(A, seed, 0)
        fill(B, seed, 1)
        Cd = torch.empty((M, N), dtype=torch.float32, device=dev)
        def clocked(clock):
            st = {"i": 0}

            def run():
                mmm.probe_mfma_ceiling(A, B, Cd, clock=clock[st["i"] % clock.shape[0]])
                st["i"] += 1

            return run

        return {"launch": lambda: mmm.probe_mfma_ceiling(A, B, Cd), "witness": None, "host_inputs": None,
                "clocked": clocked, "M": M, "N": N, "K": K}
    if kind in ("lds_mfma", "lds_mfma_nobarrier"):
        A = torch.empty((M, K), dtype=torch.float16, device=dev)
        B = torch.empty((K, N), dtype=torch.float16, device=dev)
        fill(A, seed, 0)
        fill(B, seed, 1)
        out = torch.empty(256 * 512, dtype=torch.float32, device=dev)
        barrier = kind == "lds_mfma"

        def clocked(clock):
            st = {"i": 0}

            def run():
                mmm.probe_lds_mfma(A, B, out, barrier=barrier, clock=clock[st["i"] % clock.shape[0]])
                st["i"] += 1

            return run

        return {"launch": lambda: mmm.probe_lds_mfma(A, B, out, barrier=barrier), "witness": None,
                "host_inputs": None, "clocked": clocked, "M": M, "N": N, "K": K}
    if kind == "contraction_ref":
        mt, bt, rt, nt, rt_l = REFERENCE_DIMS[name]
        assert (mt * rt, bt, nt * rt_l) == (M, N, K)
        G = torch.empty((rt, nt, mt, rt_l), dtype=torch.float16, device=dev)
        In = torch.empty((bt, nt, rt_l), dtype=torch.float16, device=dev)
        fill(G, seed, 0)
        fill(In, seed, 1)
        Out = torch.empty((mt, bt, rt), dtype=torch.float32, device=dev)
        desc = mmm.contract_desc_reference(mt, bt, rt, nt, rt_l)
        launch = mmm.bind_contract(desc, G, In, Out)

        def truth():
            T = torch.empty(Out.shape, dtype=torch.float64, device=dev)
            S = torch.empty_like(T)
            mmm.contract_truth(desc, G, In, T, S)
            return T, S

        return {"launch": launch, "witness": None, "host_inputs": None, "M": M, "N": N, "K": K,
                "validate": lambda: validate_step(torch, launch, Out, truth)}
    if kind == "contraction":
        b, i, k, l, j = 8, 1024, 32, 64, 2048
        A = torch.empty((b, i, k, l), dtype=torch.float16, device=dev)
        B = torch.empty((k, l, j), dtype=torch.float16, device=dev)
        fill(A, seed, 0)
        fill(B, seed, 1)
        Cd = torch.empty((b, i, j), dtype=torch.float32, device=dev)
        desc = mmm.contract_desc_baseline(b, i, k, l, j)
        A2, B2, C2 = A.view(M, K), B.view(K, N), Cd.view(M, N)
        launch = mmm.bind_contract(desc, A, B, Cd)
        return {
            "launch": launch,
            "validate": lambda: validate_step(torch, launch, C2, lambda: mmm.gemm_truth(A2, B2)),
            "witness": lambda: mmm.bind_witness_hipblaslt(A2, B2, C2),
            "clocked": lambda clock: mmm.bind_gemm_clocked(A2, B2, C2, clock),
            "host_inputs": lambda: (A2.cpu().numpy(), B2.cpu().numpy()),
            "M": M, "N": N, "K": K,
        }
    A = torch.empty((M, K), dtype=torch.float16, device=dev)
    fill(A, seed, 0)
    nb = 3 if name.startswith("skinny") else 1  # rotate B past the 256 MB Infinity Cache
    ws = False if name == "skinny_nows" else None
    Bs = []
    for r in range(nb):
        Bt = torch.empty((K, N), dtype=torch.float16, device=dev)
        fill(Bt, seed, 1 + r)
        Bs.append(Bt)
    Cd = torch.empty((M, N), dtype=torch.float32, device=dev)
    state = {"i": 0}
    # launchers bound once (checks and argument marshalling outside the timed loop)
    bound = [mmm.bind_gemm(A, Bt, Cd, workspace=ws, tile=tile) for Bt in Bs]

    def launch():
        bound[state["i"] % nb]()
        state["i"] += 1

    def witness():
        # hipBLASLt planned once per B buffer (descriptors, layouts, heuristic), one matmul per launch
        wb = [mmm.bind_witness_hipblaslt(A, Bt, Cd) for Bt in Bs]
        wstate = {"i": 0}

        def run():
            wb[wstate["i"] % nb]()
            wstate["i"] += 1

        run.tuning = wb[0].tuning
        return run

    # the tile kernels record their clock (the M <= 64 streaming kernels do not)
    clocked = (lambda clock: mmm.bind_gemm_clocked(A, Bs[0], Cd, clock, workspace=ws)) if M > 64 and not tile else None
    return {"launch": launch, "witness": witness, "clocked": clocked,
            "validate": lambda: validate_step(torch, bound[0], Cd, lambda: mmm.gemm_truth(A, Bs[0])),
            "host_inputs": lambda: (A.cpu().numpy(), Bs[0].cpu().numpy()),
            "M": M, "N": N, "K": K}


def validate_step(torch, launch, C_out, truth, tol: float = 1e-3):
    """One step, then every output checked on the device against the fp64 truth T and scale
    S = sum_k |a*b| of the on-device cross-check kernel: |C - T| <= tol * S (NaN fails)."""
    C_out.fill_(float("nan"))
    launch()
    T, S = truth()
    torch.cuda.synchronize()
    d = (C_out.double() - T).abs()
    ok = d <= tol * S
    worst = (d / S.clamp_min(1e-300)).nan_to_num(nan=float("inf")).max().item()
    out = {"outputs": int(C_out.numel()), "violations": int((~ok).sum().item()), "worst_err_over_S": worst,
           "tolerance": f"|C - T| <= {tol:g} * sum_k |a*b|, T and S the fp64 truth on the device"}
    del T, S, d, ok
    torch.cuda.empty_cache()
    return out


def time_launches(torch, fn, steps: int, warmup: int):
    """W untimed launches, then exactly `steps` launches between synchronizations.

    Returns (ms per step over the whole timed region, list of per-launch ms from HIP events
    recorded on the launch stream, wall seconds)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t_begin = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_begin.record(stream)
    for s in range(steps):
        starts[s].record(stream)
        fn()
        ends[s].record(stream)
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = t_begin.elapsed_time(t_end)
    per = [starts[s].elapsed_time(ends[s]) for s in range(steps)]
    return total_ms / steps, per, wall


def clocked_pass(torch, mmm, W, steps: int):
    """`steps` more launches right after the timed region, through the entry point that records
    the shader clock inside the kernel (workgroup 0's s_memtime / s_memrealtime at its start and
    end): the clock those launches ran at, and their own throughput."""
    clock = torch.zeros((steps, 4), dtype=torch.int64, device="cuda")
    ms, per, _ = time_launches(torch, W["clocked"](clock), steps, 0)
    mhz = [c for c in mmm.clocks_mhz(clock) if c == c]
    if not mhz:
        return None
    return {"sclk_mhz": round(statistics.fmean(mhz), 1), "min": round(min(mhz), 1), "max": round(max(mhz), 1),
            "launches": steps, "ms_per_launch": round(statistics.fmean(per), 5)}


def smi_snapshot():
    """The SMU's own readings (amdsmi gpu_metrics: current gfx clock per XCD, socket power);
    refreshed about once a second, so they describe the last second, not one launch."""
    try:
        import amdsmi

        amdsmi.amdsmi_init()
        try:
            h = amdsmi.amdsmi_get_processor_handles()[0]
            m = amdsmi.amdsmi_get_gpu_metrics_info(h)
            return {"gfxclk_mhz": m.get("current_gfxclk"), "gfxclk_mhz_per_xcd": m.get("current_gfxclks"),
                    "socket_power_w": m.get("current_socket_power"),
                    "power_limit_w": amdsmi.amdsmi_get_power_info(h).get("power_limit", 0) / 1e6}
        finally:
            amdsmi.amdsmi_shut_down()
    except Exception as e:  # informational only
        return {"error": repr(e)[:200]}


def read_traffic(workload: str):
    """HBM bytes per launch for the workload, from the committed rocprofv3 PMC summary."""
    path = os.path.join(REPO, "profiles", f"traffic_{workload}.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


def cpu_baseline(W, budget_s: float = 12.0):
    """Oracle CPU GEMM on a bounded sample of the workload's inputs (about budget_s of work).

    If one pass over the whole workload fits the budget, whole passes are repeated until the
    budget is spent (the best pass is reported); otherwise a leading row block of A is used."""
    import numpy as np
    import oracle

    A, B = W["host_inputs"]()
    M, N, K = W["M"], W["N"], W["K"]
    threads = oracle.max_threads()
    probe_rows = min(M, 192)
    t0 = time.perf_counter()
    oracle.cpu_gemm_f16f32(np.ascontiguousarray(A[:probe_rows]), B, threads)  # warm-up
    t_probe = time.perf_counter() - t0
    rate = 2.0 * probe_rows * N * K / max(t_probe, 1e-6)
    rows = int(min(M, max(probe_rows, budget_s * rate / (2.0 * N * K))))
    rows = max(6, rows - rows % 6) if rows < M else M
    As = np.ascontiguousarray(A[:rows])
    times = []
    t_all = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        oracle.cpu_gemm_f16f32(As, B, threads)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_all >= budget_s or len(times) >= 50:
            break
    best = min(times)
    return {
        "value": round(2.0 * rows * N * K / best / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{rows}x{N}x{K} (rows 0..{rows - 1} of the {M}x{N}x{K} workload, same seeded inputs), "
                  f"best of {len(times)} passes in {sum(times):.1f} s after a {probe_rows}-row warm-up",
        "cpu": _cpu_model(),
        "host_cpus": os.cpu_count(),
    }


def _cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the CPU baseline's record."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def run_workload(name, torch, mmm, steps, warmup, with_cpu, with_witness, with_ceiling=False, with_validate=True,
                 tile=None):
    """One workload's measurements.  Order: the step's output is validated in full (fp64 truth on
    the device) and the hipBLASLt comparison is planned and tuned (every heuristic candidate timed,
    the fastest bound) before anything is timed; then the library's W + K launches, its clocked
    launches, hipBLASLt's W + K launches, the MFMA-ceiling probe and the CPU baseline."""
    W = make_workload(name, torch, mmm, tile=tile)
    M, N, K = W["M"], W["N"], W["K"]
    flops = 2.0 * M * N * K
    algo_bytes = W.get("bytes", 2.0 * M * K + 2.0 * K * N + 4.0 * M * N)
    t_pre = time.perf_counter()
    validation = W["validate"]() if with_validate and W.get("validate") else None
    with_witness = with_witness and W.get("witness") is not None
    witness, witness_err = None, None
    if with_witness:
        try:
            witness = W["witness"]()
        except Exception as e:  # the comparison point must not hide the measurement
            witness_err = str(e)
    torch.cuda.synchronize()
    pre_s = time.perf_counter() - t_pre
    ms, per, wall = time_launches(torch, W["launch"], steps, warmup)
    clk = clocked_pass(torch, mmm, W, steps) if W.get("clocked") else None
    avg_launch = statistics.fmean(per)
    hbm = name in ("skinny", "skinny_nows", "copy", "read_ceiling", "read_ceiling_lds")
    with_cpu = with_cpu and W["host_inputs"] is not None
    res = {
        "workload": name,
        "ms_per_step": ms,
        "tflops": flops / (ms * 1e-3) / 1e12,
        "gbs": algo_bytes / (ms * 1e-3) / 1e9,
        "launch_ms": {"avg": avg_launch, "min": min(per), "median": statistics.median(per),
                      "first": per[0], "last": per[-1]},
        "wall_s": wall,
        "before_timing_s": pre_s,
    }
    if hbm:
        achieved = algo_bytes / (avg_launch * 1e-3) / 1e9
        res["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                           "frac": round(achieved / PEAK_GBS, 4), "traffic": read_traffic(name)}
    else:
        achieved = flops / (avg_launch * 1e-3) / 1e12
        res["roofline"] = {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                           "frac": round(achieved / PEAK_TFLOPS, 4), "traffic": read_traffic(name)}
    if clk is not None:
        # dense FP16 peak at the measured clock: 256 CU x 4096 flop per clock
        tf = flops / (clk["ms_per_launch"] * 1e-3) / 1e12
        clk["tflops"] = round(tf, 1)
        clk["pct_peak_at_clock"] = round(100.0 * tf / (256 * 4096 * clk["sclk_mhz"] * 1e6 / 1e12), 2)
        entry = {"mfma_ceiling": "mmm_probe_mfma_ceiling", "lds_mfma": "mmm_probe_lds_mfma",
                 "lds_mfma_nobarrier": "mmm_probe_lds_mfma"}.get(name, "mmm_gemm_f16f32_clocked")
        clk["method"] = (f"in-kernel: workgroup 0's s_memtime / s_memrealtime at its start and end ({entry}), "
                         "over `launches` launches right after the timed region; "
                         "tflops and pct_peak_at_clock are those launches' own")
        res["clock"] = clk
    res["smi"] = smi_snapshot()
    if validation is not None:
        res["validation"] = validation
    if with_witness:
        try:
            if witness is None:
                raise RuntimeError(witness_err)
            wms, wper, _ = time_launches(torch, witness, steps, warmup)
            res["hipblaslt"] = {"ms_per_step": wms, "tflops": flops / (wms * 1e-3) / 1e12,
                                "gbs": algo_bytes / (wms * 1e-3) / 1e9,
                                "launch_ms_median": statistics.median(wper),
                                "algos": witness.tuning["algos"], "best_index": witness.tuning["best_index"],
                                "algo_choice": "fastest of the heuristic's candidates, each timed on these "
                                               "inputs (median of 5 after 1)"}
        except Exception as e:  # the comparison point must not hide the measurement
            res["hipblaslt"] = {"error": str(e)}
    if with_ceiling:
        # the same step count on the library's MFMA-ceiling probe (this workload's MFMA stream
        # with register-resident operands), measured live in this process
        Cw = make_workload("mfma_ceiling", torch, mmm)
        cms, cper, _ = time_launches(torch, Cw["launch"], steps, warmup)
        cclk = clocked_pass(torch, mmm, Cw, steps)
        ctf = flops / (cms * 1e-3) / 1e12
        res["ceiling"] = {"mfma_tflops": round(ctf, 1), "frac": round(res["tflops"] / ctf, 4),
                          "sclk_mhz": cclk["sclk_mhz"] if cclk else None,
                          "what": "mmm_probe_mfma_ceiling: the same grid's MFMA stream and C stores without "
                                  "operand loads, LDS or barriers, same warm-up and steps; frac = value / mfma_tflops"}
        del Cw
    if with_cpu:
        res["cpu_baseline"] = cpu_baseline(W)
    return res


def steady_state(name, torch, mmm, seconds: float):
    """The workload launched back to back for `seconds` (the first 60% untimed, so the power
    controller settles), then: throughput over the rest (HIP events around it), the SMU's
    gfx clock and socket power read right after (amdsmi, refreshed about once a second), and
    the in-kernel clock of 20 clock-recording launches that follow."""
    W = make_workload(name, torch, mmm)
    M, N, K = W["M"], W["N"], W["K"]
    work = W.get("bytes", 2.0 * M * N * K)
    fn = W["launch"]
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.6 * seconds:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = 0
    e0.record()
    t1 = time.perf_counter()
    while time.perf_counter() - t1 < 0.4 * seconds:
        for _ in range(20):
            fn()
        n += 20
        torch.cuda.synchronize()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / n
    out = {"seconds": seconds, "launches_timed": n, "ms_per_launch": round(ms, 5), "smi": smi_snapshot()}
    if "bytes" in W:
        out["gbs"] = round(work / (ms * 1e-3) / 1e9, 1)
    else:
        out["tflops"] = round(work / (ms * 1e-3) / 1e12, 1)
    if W.get("clocked"):
        out["clock"] = clocked_pass(torch, mmm, W, 20)
    return out


# the 8192^3 kernel and the probes that take its parts away, in the order of the table
DECOMPOSE = [
    ("gemm8192", "the library's kernel (mmm_gemm_f16f32)", "operand loads (HBM/L2 -> LDS), barrier, LDS fragment "
     "reads, MFMAs, C stores"),
    ("lds_mfma", "mmm_probe_lds_mfma, barrier = 1", "barrier, LDS fragment reads, MFMAs"),
    ("lds_mfma_nobarrier", "mmm_probe_lds_mfma, barrier = 0", "LDS fragment reads, MFMAs"),
    ("mfma_ceiling", "mmm_probe_mfma_ceiling", "MFMAs on register operands, C stores"),
]


def run_decompose(path, torch, mmm, seconds: float, rounds: int = 2):
    """Steady-state throughput, clock and power of the 8192^3 kernel and of the probes that leave
    out its operand loads, its barrier and its LDS reads in turn (DECOMPOSE), `rounds` rounds in
    rotated order, each variant run back to back for `seconds` (steady_state); writes a markdown
    table to `path`."""
    rows = {name: [] for name, _, _ in DECOMPOSE}
    for r in range(rounds):
        order = DECOMPOSE[r % len(DECOMPOSE):] + DECOMPOSE[:r % len(DECOMPOSE)]
        for name, _, _ in order:
            res = steady_state(name, torch, mmm, seconds)
            _log(f"[decompose] round {r} {name}: {res['tflops']} TFLOP/s, clock {res.get('clock')}, smi {res['smi']}")
            rows[name].append(res)
            torch.cuda.empty_cache()
    flop_per_clk = 256 * 4096  # dense FP16 MFMA: 256 CU x 4096 flop per clock

    def span(vals, fmt):
        vals = [v for v in vals if isinstance(v, (int, float))]
        if not vals:
            return "-"
        lo, hi = min(vals), max(vals)
        return fmt.format(lo) if fmt.format(lo) == fmt.format(hi) else fmt.format(lo) + "-" + fmt.format(hi)

    lines = [
        "| variant | runs | what is left of the kernel | TFLOP/s | in-kernel clock (MHz) | SMU gfxclk (MHz) | "
        "socket power (W) | MFMA busy at the in-kernel clock |",
        "|---|---|---|---|---|---|---|---|",
    ]
    for name, runs, left in DECOMPOSE:
        rs = rows[name]
        tf = [x["tflops"] for x in rs]
        clk = [x["clock"]["sclk_mhz"] for x in rs if x.get("clock")]
        smi_clk = [x["smi"].get("gfxclk_mhz") for x in rs]
        pw = [x["smi"].get("socket_power_w") for x in rs]
        busy = [x["tflops"] * 1e12 / (flop_per_clk * x["clock"]["sclk_mhz"] * 1e6) for x in rs if x.get("clock")]
        lines.append(f"| `{name}` | {runs} | {left} | {span(tf, '{:.0f}')} | {span(clk, '{:.0f}')} | "
                     f"{span(smi_clk, '{:.0f}')} | {span(pw, '{:.0f}')} | {span(busy, '{:.3f}')} |")
    head = [
        "# Where the 8192^3 kernel's time goes: the kernel against probes that leave out its parts",
        "",
        "Command (repository root on the GPU box):",
        "",
        "```",
        "python3 bench.py " + " ".join(sys.argv[1:]),
        "```",
        "",
        f"Device: {torch.cuda.get_device_name(0)}.  Each variant runs M = N = K = 8192 (2.2e12 flop per launch) "
        f"back to back for {seconds:g} s per round, {rounds} rounds in rotated order: throughput over the last 40% "
        "of each run (HIP events), then the SMU's gfx clock and socket power (amdsmi, about one reading a "
        "second), then the in-kernel shader clock of 20 clock-recording launches (workgroup 0's s_memtime / "
        "s_memrealtime).  Cells give the range over the rounds.  MFMA busy = TFLOP/s / (256 CU x 4096 flop "
        "per clock x in-kernel clock).  The probes (include/mmm.h) run the kernel's own code for what they "
        "keep: `mmm_probe_lds_mfma` its per-K-tile fragment reads and MFMAs at its LDS addresses on two "
        "K tiles staged once, `mmm_probe_mfma_ceiling` its MFMA stream on register operands.",
        "",
    ]
    text = "\n".join(head + lines) + "\n"
    with open(path, "w") as f:
        f.write(text)
    print(text, file=sys.stderr, flush=True)
    return rows


# shapes of the tile sweep (--sweep): squares, the configs, and tall / wide / deep / shallow cases
# rounds of the sweep: every column is timed once per round, in a rotated order
SWEEP_ROUNDS = 3
SWEEP_SHAPES = [(256, 256, 256), (512, 512, 512), (1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096),
                (6144, 6144, 6144), (8192, 8192, 8192), (8192, 2048, 2048), (2048, 8192, 2048), (4097, 4095, 4111),
                (16384, 1024, 4096), (1024, 16384, 4096), (8192, 8192, 1024), (1024, 1024, 8192), (3000, 5000, 1000),
                (64, 4096, 4096), (1536, 1536, 12288),
                # partly filled last rounds (K split of the last round) and short-K few-round grids
                (4608, 4608, 8192), (7168, 7168, 7168), (10240, 10240, 4096), (2304, 2304, 8192), (3072, 3072, 3072),
                (6144, 6144, 2048)]


# transformer-layer GEMMs (tokens x out-features x in-features): attention and MLP projections of
# 4k-14k-wide layers at 128-16384 tokens (--sweep PATH --shapes llm)
SWEEP_SHAPES_LLM = [(2048, 4096, 4096), (4096, 11008, 4096), (4096, 4096, 11008), (4096, 14336, 4096),
                    (4096, 4096, 14336), (8192, 6144, 4096), (4096, 28672, 8192), (4096, 8192, 28672),
                    (16384, 4096, 4096), (2048, 14336, 4096), (1024, 8192, 8192), (512, 8192, 8192),
                    (256, 4096, 4096), (128, 14336, 4096), (8192, 8192, 4096), (8192, 1024, 8192)]


# 136-256 tokens x out-features x in-features (prefill chunks, large decode batches): the shapes the
# tile prices were refitted on (--sweep PATH --shapes small_m, with and without --rotate)
SWEEP_SHAPES_SMALL_M = [(m, n, k) for m in (136, 160, 192, 224, 256)
                        for (n, k) in ((4096, 4096), (14336, 4096), (4096, 14336), (8192, 8192), (28672, 8192),
                                       (8192, 28672), (11008, 4096), (4096, 11008))]
# decode-step GEMMs (1-64 tokens x out-features x in-features) of 8B- and 70B-class layers: the
# M <= 64 streaming kernel's range (--sweep PATH --shapes decode; B rotates through HBM)
SWEEP_SHAPES_DECODE = [(m, n, k) for m in (1, 16, 32, 64)
                       for (n, k) in ((4096, 4096), (6144, 4096), (14336, 4096), (4096, 14336), (8192, 8192),
                                      (10240, 8192), (28672, 8192), (8192, 28672))]
# --shapes decode: each column cycles through B buffers totalling at least this much (more than the
# 256 MB Infinity Cache), so B comes from HBM as a model's weights would
SWEEP_ROTATE_BYTES = 512 << 20


def parse_shapes(text: str):
    """"MxNxK,MxNxK,..." -> [(M, N, K), ...]; "llm", "small_m", "decode" -> those sets"""
    if text.strip().lower() == "llm":
        return list(SWEEP_SHAPES_LLM)
    if text.strip().lower() == "small_m":
        return list(SWEEP_SHAPES_SMALL_M)
    if text.strip().lower() == "decode":
        return list(SWEEP_SHAPES_DECODE)
    shapes = []
    for item in text.split(","):
        dims = tuple(int(x) for x in item.lower().split("x"))
        if len(dims) != 3 or min(dims) < 1:
            raise ValueError(f"bad shape {item!r}: want MxNxK with positive sizes")
        shapes.append(dims)
    return shapes


def _cycle(fns):
    """One launcher that runs fns in turn (the first alone when there is one)."""
    if len(fns) == 1:
        return fns[0]
    it = itertools.cycle(fns)

    def launch():
        next(it)()

    launch.tuning = getattr(fns[0], "tuning", None)
    return launch


def run_sweep(path: str, torch, mmm, steps: int, warmup: int, with_witness: bool, shapes=None,
              rotate_bytes: int = 0) -> None:
    """Every instantiated tile and the library's own choice on each problem of `shapes`
    (SWEEP_SHAPES by default); median per-launch TFLOP/s, written as a markdown table to path.
    With rotate_bytes, every column cycles through ceil(rotate_bytes / bytes of B) copies of B
    (at most 16), so that B is read from HBM rather than from the Infinity Cache."""
    tiles = list(mmm.TILES)
    lines = ["| M x N x K | library pick | pick TFLOP/s | " + " | ".join(tiles) + " | best | pick / best | hipBLASLt | hipBLASLt candidate |",
             "|" + "---|" * (len(tiles) + 7)]
    for (M, N, K) in (shapes or SWEEP_SHAPES):
        A = torch.empty((M, K), dtype=torch.float16, device="cuda")
        nb = min(16, max(1, -(-rotate_bytes // (2 * K * N)))) if rotate_bytes else 1
        Bs = [torch.empty((K, N), dtype=torch.float16, device="cuda") for _ in range(nb)]
        B = Bs[0]
        mmm.fill_uniform(A, 7, 0)
        for i, Bi in enumerate(Bs):
            mmm.fill_uniform(Bi, 7, 1 + i)
        Cm = torch.empty((M, N), dtype=torch.float32, device="cuda")
        flops = 2.0 * M * N * K

        def tf(fn):
            _, per, _ = time_launches(torch, fn, steps, warmup)
            return flops / (statistics.median(per) * 1e-3) / 1e12

        plan = mmm.gemm_plan(M, N, K, A=A, B=B, C_out=Cm)
        pick = plan["kernel"] if plan["kernel"] != "tile" else f"{plan['block_m']}x{plan['block_n']}"
        if plan["kernel"] == "tile+stream":
            pick = f"{plan['block_m']}x{plan['block_n']} + stream {plan['stream_rows']}"
        # every launcher bound once (checks, marshalling and hipBLASLt's planning outside the timing)
        launchers = {"pick": _cycle([mmm.bind_gemm(A, Bi, Cm) for Bi in Bs])}
        launchers.update({t: _cycle([mmm.bind_gemm(A, Bi, Cm, tile=t) for Bi in Bs]) for t in tiles})
        if with_witness:
            try:
                w0 = mmm.bind_witness_hipblaslt(A, B, Cm)  # candidates timed on the first B
                launchers["hipblaslt"] = _cycle([w0] + [w0.with_operands(A, Bi, Cm) for Bi in Bs[1:]])
            except Exception as e:  # witness library absent or hipBLASLt refused the shape
                _log(f"[sweep] hipBLASLt unavailable for {M}x{N}x{K}: {e}")
        # The chip's power controller takes tens of milliseconds to settle after the load changes,
        # so each shape first runs its pick for at least 100 ms untimed.  Then SWEEP_ROUNDS rounds
        # time every column once, each round in a rotated order, and a column's figure is its
        # median over the rounds: no column always runs right after the warm-up or a slow neighbour.
        t_end = time.perf_counter() + 0.1
        while time.perf_counter() < t_end:
            for _ in range(10):
                launchers["pick"]()
            torch.cuda.synchronize()
        names = list(launchers)
        got = {n: [] for n in names}
        for r in range(SWEEP_ROUNDS):
            for n in names[r % len(names):] + names[:r % len(names)]:
                got[n].append(tf(launchers[n]))
        med = {n: statistics.median(v) for n, v in got.items()}
        auto = med["pick"]
        per_tile = {t: med[t] for t in tiles}
        best = max(per_tile, key=per_tile.get)
        wit = med.get("hipblaslt", float("nan"))
        wpick = launchers["hipblaslt"].tuning if "hipblaslt" in launchers else None
        row = (f"| {M} x {N} x {K} | {pick} | {auto:.1f} | " + " | ".join(f"{per_tile[t]:.1f}" for t in tiles) +
               f" | {best} | {auto / per_tile[best]:.2f} | {wit:.1f} | "
               + (f"#{wpick['best_index']} of {wpick['algos']}" if wpick else "") + " |")
        lines.append(row)
        _log("[sweep] " + row)
        del A, B, Bs, Cm, launchers
        torch.cuda.empty_cache()
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=100,
                    help="untimed launches first (the clock ramps up over the first ~50 ms of load)")
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="gemm8192")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-witness", action="store_true", help="skip the hipBLASLt comparison")
    ap.add_argument("--no-ceiling", action="store_true", help="skip the live MFMA-ceiling probe (gemm8192 only)")
    ap.add_argument("--no-validate", action="store_true",
                    help="skip the full-output fp64 validation of the step that precedes the timing")
    ap.add_argument("--steady", type=float, metavar="SECONDS", default=0.0,
                    help="also run the workload back to back for SECONDS and add its steady-state throughput, "
                         "SMU clock/power and in-kernel clock to the line (object `steady`)")
    ap.add_argument("--report", metavar="PATH", help="measure every workload and write a JSON report to PATH")
    ap.add_argument("--sweep", metavar="PATH", help="time every tile against the library's pick over a shape "
                                                     "grid and write a markdown table to PATH")
    ap.add_argument("--decompose", metavar="PATH", help="run the 8192^3 kernel and the probes that leave out its "
                                                         "operand loads, barrier and LDS reads in the steady state "
                                                         "and write a markdown table to PATH")
    ap.add_argument("--decompose-seconds", type=float, default=4.0, metavar="SECONDS",
                    help="with --decompose: seconds each variant runs back to back per round (two rounds)")
    ap.add_argument("--shape", metavar="MxNxK", help="measure this GEMM (U[-1,1) inputs, seed 7) instead of --workload")
    ap.add_argument("--tile", metavar="BMxBN", help="with --shape: force this block tile (one of the library's six; "
                                                    "default: the library's own pick)")
    ap.add_argument("--shapes", metavar="MxNxK,...", help="the problems --sweep runs: a list, `llm` for the "
                                                          "transformer-layer set, `small_m` for 136-256-token "
                                                          "layer GEMMs, or `decode` for 1-64-token layer GEMMs "
                                                          "with B rotating through HBM (default: the built-in "
                                                          "list)")
    ap.add_argument("--rotate", action="store_true",
                    help="with --sweep: cycle every column through copies of B totalling 512 MiB (read from "
                         "HBM, not the Infinity Cache); always on for --shapes decode")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(the GEMM shards by N or M with no exchange; no multi-GPU launch is built)"}))
        return 2
    if args.steps < 1 or args.warmup < 0:
        ap.error("--steps must be >= 1 and --warmup >= 0")

    import torch
    import mmm

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    mmm.lib()

    if args.sweep:
        decode = bool(args.shapes) and args.shapes.strip().lower() == "decode"
        run_sweep(args.sweep, torch, mmm, args.steps, args.warmup, with_witness=not args.no_witness,
                  shapes=parse_shapes(args.shapes) if args.shapes else None,
                  rotate_bytes=SWEEP_ROTATE_BYTES if decode or args.rotate else 0)

    if args.decompose:
        run_decompose(args.decompose, torch, mmm, args.decompose_seconds)

    if args.report:
        report = []
        for name in ["gemm8192", "contraction", "ragged", "skinny", "skinny_nows", "gemm256", "contraction_ref"]:
            _log(f"[bench] {name}")
            r = run_workload(name, torch, mmm, args.steps, args.warmup, with_cpu=False,
                             with_witness=not args.no_witness, with_validate=not args.no_validate)
            _log(f"[bench] {name}: {r['tflops']:.1f} TFLOP/s ({r['gbs']:.0f} GB/s); "
                 f"hipBLASLt {r.get('hipblaslt', {}).get('tflops', float('nan')):.1f} TFLOP/s")
            report.append(r)
            torch.cuda.empty_cache()
        with open(args.report, "w") as f:
            json.dump({"device": torch.cuda.get_device_name(0), "results": report}, f, indent=1)

    name = args.workload
    if args.shape:
        (sM, sN, sK), = parse_shapes(args.shape)
        name = "shape"
        WORKLOADS[name] = (sM, sN, sK, "gemm", SHAPE_SEED, "uniform")
        DESCRIPTIONS[name] = (f"gemm_nn {sM}x{sN}x{sK} fp16 row-major, " + (f"tile {args.tile} forced, " if args.tile else "")
                              + f"U[-1,1) seed {SHAPE_SEED}")
    if args.tile and (not args.shape or args.tile not in mmm.TILES):
        ap.error(f"--tile needs --shape and one of {', '.join(mmm.TILES)}")
    r = run_workload(name, torch, mmm, args.steps, args.warmup, with_cpu=not args.no_cpu,
                     with_witness=not args.no_witness, with_ceiling=name == "gemm8192" and not args.no_ceiling,
                     with_validate=not args.no_validate, tile=args.tile)
    M, N, K = WORKLOADS[name][:3]
    skinny = name in ("skinny", "skinny_nows", "copy", "read_ceiling", "read_ceiling_lds")
    line = {
        "metric": METRIC if name == "gemm8192" else f"{name} {'GB/s' if skinny else 'TFLOP/s'}",
        "value": round(r["gbs"] if skinny else r["tflops"], 2),
        "unit": "GB/s" if skinny else "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 (f32 accumulate)",
        "data": f"synthetic: seeded on-device generator, {data_description(name)}",
        "config": {"workload": DESCRIPTIONS[name], "M": M, "N": N, "K": K},
        "pct_peak": round(100.0 * r["tflops"] / PEAK_TFLOPS, 2),
        "launch_ms": {k: round(v, 5) for k, v in r["launch_ms"].items()},
        "roofline": r["roofline"],
        "before_timing_s": round(r["before_timing_s"], 3),
    }
    if "validation" in r:
        line["validation"] = r["validation"]
    if "clock" in r:
        line["clock"] = r["clock"]
    if "ceiling" in r:
        line["ceiling"] = r["ceiling"]
    line["smi"] = r["smi"]
    if args.steady > 0:
        line["steady"] = steady_state(name, torch, mmm, args.steady)
    if "cpu_baseline" in r:
        line["cpu_baseline"] = r["cpu_baseline"]
    if "hipblaslt" in r:
        line["hipblaslt"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r["hipblaslt"].items()}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
