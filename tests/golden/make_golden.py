"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

The reference (thrasos-g/RDNA4-GEMM-WMMA) ships no golden vectors, fixtures or known-answer
tests (its only check is a run-time comparison against rocBLAS on unseeded inputs,
mmm.cpp:1387-1407).  These fixtures freeze this build's seeded input stream and small
fp64 results so that later changes to the oracle or the device generator are caught:

  prng_kat.json   first 16 fp16 bit patterns of every (seed, tensor) stream the five
                  benchmark configurations use
  gemm_small.npz  A [24,40], B [40,16] (seed 9) with the fp64 product and S = sum|a*b|
  contract_ref_small.npz
                  the reference-layout contraction (mmmTensor.cpp) at mt=2 bt=6 rt=4 nt=3
                  rt_l=8 (seed 10): G, In and Out[m][b][r] in fp64
  contract_baseline_small.npz
                  the benchmark contraction C[b,i,j] = sum_kl A[b,i,k,l] B[k,l,j] at b=2 i=3
                  k=4 l=5 j=6 (N(0,1)*0.1, seed 11): A, B, C [b*i][j] and S in fp64
  c1_256.json     configuration C1 (256^3, U[-1,1), seed 0): sha256 of A's and B's fp16 bit
                  patterns and of the fp64 C and S, with a few of their values

Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402

STREAMS = [  # (name, seed, tensor_id, dist)
    ("c1_A", 0, 0, "uniform"), ("c1_B", 0, 1, "uniform"),
    ("c2_A", 1, 0, "uniform"), ("c2_B", 1, 1, "uniform"),
    ("c3_A", 2, 0, "uniform"), ("c3_B", 2, 1, "uniform"),
    ("c4_A", 3, 0, "normal"), ("c4_B", 3, 1, "normal"),
    ("c5_A", 4, 0, "uniform"), ("c5_B", 4, 1, "uniform"),
]


def main():
    kat = {}
    for name, seed, tid, dist in STREAMS:
        v = oracle.uniform_f16((16,), seed, tid) if dist == "uniform" else oracle.normal_f16((16,), seed, tid, 0.1)
        kat[name] = {"seed": seed, "tensor_id": tid, "dist": dist,
                     "bits": [int(x) for x in v.view(np.uint16)]}
    with open(os.path.join(HERE, "prng_kat.json"), "w") as f:
        json.dump(kat, f, indent=1)

    A = oracle.uniform_f16((24, 40), 9, 0)
    B = oracle.uniform_f16((40, 16), 9, 1)
    C, S = oracle.gemm_f64(A, B)
    np.savez(os.path.join(HERE, "gemm_small.npz"), A=A, B=B, C=C, S=S)

    G = oracle.normal_f16((4, 3, 2, 8), 10, 0, 0.1)   # [rt][nt][mt][rt_l]
    In = oracle.normal_f16((6, 3, 8), 10, 1, 0.1)     # [bt][nt][rt_l]
    Cr, Sr = oracle.contract_reference_f64(G, In)     # [(m*rt + r)][b]
    Out = Cr.reshape(2, 4, 6).transpose(0, 2, 1)      # [m][b][r]
    np.savez(os.path.join(HERE, "contract_ref_small.npz"), G=G, In=In, Out=np.ascontiguousarray(Out))

    Ab = oracle.normal_f16((2, 3, 4, 5), 11, 0, 0.1)  # [b][i][k][l]
    Bb = oracle.normal_f16((4, 5, 6), 11, 1, 0.1)     # [k][l][j]
    Cb, Sb = oracle.contract_baseline_f64(Ab, Bb)     # [(b*i)][j]
    np.savez(os.path.join(HERE, "contract_baseline_small.npz"), A=Ab, B=Bb, C=Cb, S=Sb)

    with open(os.path.join(HERE, "c1_256.json"), "w") as f:
        json.dump(c1_record(), f, indent=1)


def c1_record():
    """sha256 and sample values of configuration C1's inputs and fp64 result."""
    A = oracle.uniform_f16((256, 256), 0, 0)
    B = oracle.uniform_f16((256, 256), 0, 1)
    C, S = oracle.gemm_f64(A, B)
    h = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    return {"shape": [256, 256, 256], "seed": 0,
            "sha256": {"A_f16_bits": h(A.view(np.uint16)), "B_f16_bits": h(B.view(np.uint16)), "C_f64": h(C),
                       "S_f64": h(S)},
            "samples": {"C[0][0]": float(C[0, 0]), "C[255][255]": float(C[255, 255]), "C[17][200]": float(C[17, 200]),
                        "sum_C": float(C.sum()), "sum_S": float(S.sum())}}


if __name__ == "__main__":
    main()
