"""Register / LDS / occupancy report of every gfx950 kernel in the library.

The reference keeps a device-assembly dump for inspection (compile.bat:16, ``hipcc
--offload-device-only -S``).  This does the same for every source of lib/libmmm.so and turns
the code-object metadata into a table: registers (arch VGPR, AGPR, SGPR), spills, static LDS,
scratch, the occupancy those allow on a CDNA4 compute unit, and static instruction counts of
the kernel body (matrix-core ops, direct-to-LDS loads, LDS reads, barriers).

    python rdna4-gemm-wmma_amd/mmm/isa.py [--out profiles/isa_resources.md]
"""
import argparse
import concurrent.futures
import os
import re
import subprocess
import sys

import yaml

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPO_ROOT = os.path.dirname(PKG_ROOT)
SOURCES = ["csrc/mmm_gemm.hip", "csrc/mmm_skinny.hip", "csrc/mmm_check.hip", "csrc/mmm_capi.hip", "csrc/mmm_probe.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I../include", "-Icsrc", "-S", "--offload-device-only"]

# CDNA4 compute unit: 4 SIMDs, 512 unified (arch + accumulation) VGPRs per lane per SIMD,
# allocated in granules of 8, at most 8 waves per SIMD; 160 KiB of LDS per CU.
SIMDS_PER_CU = 4
VGPRS_PER_SIMD = 512
VGPR_GRANULE = 8
MAX_WAVES_PER_SIMD = 8
LDS_PER_CU = 160 * 1024

# static instruction classes counted in each kernel body
CLASSES = [
    ("mfma", re.compile(r"^\s*v_mfma_")),
    ("dma_lds", re.compile(r"^\s*(buffer|global)_load_(lds_\w+|\w+.*\blds\b)")),
    ("ds_read", re.compile(r"^\s*ds_read")),
    ("vmem_load", re.compile(r"^\s*(buffer|global)_load_(?!lds_)(?!.*\blds\b)")),
    ("vmem_store", re.compile(r"^\s*(buffer|global)_store_")),
    ("barrier", re.compile(r"^\s*s_barrier\b")),
    ("waitcnt", re.compile(r"^\s*s_waitcnt\b")),
]


def compile_asm(src: str, out_dir: str) -> str:
    out = os.path.join(out_dir, os.path.basename(src).replace(".hip", ".s"))
    subprocess.run([HIPCC, *FLAGS, "-o", out, src], cwd=PKG_ROOT, check=True, stdout=subprocess.DEVNULL,
                   stderr=subprocess.DEVNULL)
    return out


def demangle(names):
    try:
        r = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True, check=True)
        return r.stdout.strip().split("\n")
    except (OSError, subprocess.CalledProcessError):
        return list(names)


def short_name(demangled: str) -> str:
    s = demangled.replace("(anonymous namespace)::", "").replace("mmm::", "")
    s = re.sub(r"^void ", "", s)
    depth = 0
    for i, ch in enumerate(s):  # drop the parameter list
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return s[:i]
    return s


def parse_asm(path: str):
    text = open(path).read()
    meta = re.search(r"\.amdgpu_metadata\n(---\n.*?\n\.\.\.)\n", text, re.S)
    kernels = yaml.safe_load(meta.group(1))["amdhsa.kernels"] if meta else []
    lines = text.split("\n")
    bodies = {}
    for k in kernels:
        sym = k[".symbol"][:-3] if k[".symbol"].endswith(".kd") else k[".name"]
        start = next((i for i, ln in enumerate(lines) if ln.split(";")[0].strip() == sym + ":"), None)
        if start is None:
            continue
        counts = {c: 0 for c, _ in CLASSES}
        total = 0
        for ln in lines[start + 1:]:
            if ln.startswith(".Lfunc_end") or ln.strip().startswith(".size\t" + sym):
                break
            t = ln.split(";")[0]
            if not t.strip() or t.strip().startswith((".", "//")) or t.rstrip().endswith(":"):
                continue
            total += 1
            for c, rx in CLASSES:
                if rx.match(t):
                    counts[c] += 1
        counts["instructions"] = total
        bodies[sym] = counts
    accum = {m.group(1): int(m.group(2)) for m in
             re.finditer(r"\.amdhsa_kernel (\S+)\n(?:.*\n)*?\s*\.amdhsa_accum_offset (\d+)", text)}
    return kernels, bodies, accum


def occupancy(total_vgpr: int, lds: int, threads: int):
    waves_per_wg = max(1, (threads + 63) // 64)
    alloc = max(VGPR_GRANULE, (total_vgpr + VGPR_GRANULE - 1) // VGPR_GRANULE * VGPR_GRANULE)
    waves_vgpr = min(MAX_WAVES_PER_SIMD, VGPRS_PER_SIMD // alloc)
    wg_vgpr = (waves_vgpr * SIMDS_PER_CU) // waves_per_wg
    wg_lds = LDS_PER_CU // lds if lds > 0 else 10 ** 6
    wg_waves = (MAX_WAVES_PER_SIMD * SIMDS_PER_CU) // waves_per_wg
    wg = min(wg_vgpr, wg_lds, wg_waves)
    limiter = "vgpr" if wg == wg_vgpr else ("lds" if wg == wg_lds else "waves")
    return wg, wg * waves_per_wg / SIMDS_PER_CU, limiter


def collect(out_dir: str):
    os.makedirs(out_dir, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=4) as ex:
        paths = list(ex.map(lambda s: compile_asm(s, out_dir), SOURCES))
    rows = []
    for src, path in zip(SOURCES, paths):
        kernels, bodies, accum = parse_asm(path)
        names = demangle([k[".name"] for k in kernels])
        for k, dn in zip(kernels, names):
            sym = k[".symbol"][:-3] if k[".symbol"].endswith(".kd") else k[".name"]
            total = int(k[".vgpr_count"])
            agpr = int(k.get(".agpr_count", 0))
            arch = accum.get(sym, total) if agpr else total
            lds = int(k[".group_segment_fixed_size"])
            threads = int(k[".max_flat_workgroup_size"])
            wg, waves, limiter = occupancy(total, lds, threads)
            rows.append({
                "source": os.path.basename(src), "kernel": short_name(dn), "threads": threads,
                "vgpr": arch, "agpr": agpr, "vgpr_total": total, "sgpr": int(k[".sgpr_count"]),
                "vgpr_spill": int(k.get(".vgpr_spill_count", 0)), "sgpr_spill": int(k.get(".sgpr_spill_count", 0)),
                "lds": lds, "scratch": int(k[".private_segment_fixed_size"]),
                "wavefront": int(k[".wavefront_size"]), "wg_per_cu": wg, "waves_per_simd": waves,
                "limiter": limiter, **bodies.get(sym, {}),
            })
    return rows


def to_markdown(rows) -> str:
    cols = ["kernel", "threads", "vgpr", "agpr", "sgpr", "vgpr_spill", "sgpr_spill", "lds", "scratch", "wg_per_cu",
            "waves_per_simd", "limiter", "mfma", "dma_lds", "ds_read", "vmem_load", "vmem_store", "barrier",
            "waitcnt", "instructions"]
    out = ["| " + " | ".join(cols) + " |", "|" + "---|" * len(cols)]
    for r in rows:
        out.append("| " + " | ".join(f"`{r[c]}`" if c == "kernel" else str(r.get(c, "")) for c in cols) + " |")
    return "\n".join(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out", default=None, help="write the markdown report here (default: stdout)")
    ap.add_argument("--asm-dir", default=os.path.join(PKG_ROOT, "_build", "isa"))
    a = ap.parse_args(argv)
    rows = collect(a.asm_dir)
    cmd = "python rdna4-gemm-wmma_amd/mmm/isa.py" + (f" --out {os.path.relpath(a.out, REPO_ROOT)}" if a.out else "")
    text = ("# gfx950 kernel resources (static, from the device assembly)\n\n"
            f"Command: `{cmd}` (hipcc {' '.join(FLAGS)}).\n\n"
            "vgpr = architectural VGPRs, agpr = accumulation VGPRs (together out of 512 per lane per SIMD); "
            "sgpr_spill = SGPRs spilled into VGPR lanes (no memory traffic); "
            "lds and scratch in bytes per workgroup; wg_per_cu / waves_per_simd = occupancy those "
            "resources allow (limiter = the binding one); instruction columns are static counts in "
            "the kernel body, not executed counts.\n\n" + to_markdown(rows) + "\n")
    if a.out:
        with open(a.out, "w") as f:
            f.write(text)
    else:
        sys.stdout.write(text)
    # SGPR spills land in VGPR lanes; VGPR spills and scratch go to memory and count as failures
    bad = [r["kernel"] for r in rows if r["scratch"] or r["vgpr_spill"]]
    if bad:
        print("kernels spilling to scratch: " + ", ".join(bad), file=sys.stderr)
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main())
