"""Writes tests/golden/kats.json: known-answer vectors for the GEMM and the
attention, computed with exact rational arithmetic (Python ints / Fractions),
independent of numpy, torch and the oracle.

The reference ships no golden vectors (its tests draw inputs from MLX's RNG at
run time and compare bits of its own outputs), so these are constructed from
closed forms whose answers are exact in every element type:
  gemm  -- small-integer operands (|a|, |b| <= 3, K <= 24): every partial sum is
           an integer far below 2^8, so acc and the rounded output are exact in
           bf16, f16 and fp32, whatever the summation order; with integer bias
           and alpha, beta in {1, 2, -1, 0.5}.
  sdpa  -- (i) one key: out = v_0; (ii) all keys equal: out = mean of v (v in
           quarters, N a power of two); (iii) every key masked: out = 0;
           (iv) causal, end-aligned, N = 2 keys, qL = 3 rows: row 0 sees no key
           (out = 0), rows 1 and 2 see 1 and 2 keys (out = v_0, (v_0 + v_1) / 2).
           Outputs are exact rationals; a test rounds them once to the element
           type, as the kernel does.

    python tests/golden/make_kats.py
"""

import json
import os
import random
from fractions import Fraction

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kats.json")


def gemm_case(rng, M, K, N, trans_b, bias, alpha, beta):
    a = [[rng.randint(-3, 3) for _ in range(K)] for _ in range(M)]
    b_kn = [[rng.randint(-3, 3) for _ in range(N)] for _ in range(K)]
    c = [rng.randint(-4, 4) for _ in range(N)] if bias else None
    out = []
    for m in range(M):
        row = []
        for n in range(N):
            acc = sum(a[m][k] * b_kn[k][n] for k in range(K))
            v = Fraction(alpha) * acc + Fraction(beta) * c[n] if bias else Fraction(acc)
            row.append(float(v))
        out.append(row)
    b = [list(col) for col in zip(*b_kn)] if trans_b else b_kn
    return {"M": M, "K": K, "N": N, "trans_b": trans_b, "a": a, "b": b, "bias": c,
            "alpha": alpha, "beta": beta, "out": out}


def sdpa_case(name, rng, B, H, Hkv, qL, N, D, kind):
    q = [[[[rng.randint(-2, 2) for _ in range(D)] for _ in range(qL)] for _ in range(H)]
         for _ in range(B)]
    key = [[rng.randint(-2, 2) for _ in range(D)] for _ in range(Hkv)]
    k = [[[list(key[h]) for _ in range(N)] for h in range(Hkv)] for _ in range(B)]
    v = [[[[Fraction(rng.randint(-8, 8), 4) for _ in range(D)] for _ in range(N)]
          for _ in range(Hkv)] for _ in range(B)]
    mask = None
    causal = kind == "causal"
    if kind == "one_key":
        pass  # N == 1
    if kind == "all_masked":
        mask = [[[[False] * N]]]
    g = H // Hkv
    out = []
    for b in range(B):
        ob = []
        for h in range(H):
            oh = []
            for s in range(qL):
                if kind == "all_masked":
                    vis = 0
                elif causal:
                    vis = N - qL + s + 1
                else:
                    vis = N
                if vis <= 0:
                    oh.append([0.0] * D)
                    continue
                vv = v[b][h // g][:vis]
                oh.append([float(sum(row[d] for row in vv) / vis) for d in range(D)])
            ob.append(oh)
        out.append(ob)
    return {"name": name, "B": B, "H": H, "Hkv": Hkv, "qL": qL, "N": N, "D": D,
            "q": q, "k": k, "v": [[[[float(x) for x in r] for r in hh] for hh in bb] for bb in v],
            "mask": mask, "causal": causal, "out": out}


def main():
    rng = random.Random(20261201)
    gemm = []
    for M, K, N, tb, bias, al, be in [(1, 1, 5, False, False, 1, 1), (3, 7, 9, True, False, 1, 1),
                                      (17, 24, 20, False, True, 1, 1), (5, 16, 33, True, True, 2, -1),
                                      (2, 9, 16, False, True, 0.5, 2), (16, 24, 16, True, True, -1, 0.5)]:
        gemm.append(gemm_case(rng, M, K, N, tb, bias, al, be))
    sdpa = [sdpa_case("one_key", rng, 1, 4, 2, 3, 1, 64, "one_key"),
            sdpa_case("equal_keys", rng, 2, 4, 2, 2, 64, 64, "equal"),
            sdpa_case("all_masked", rng, 1, 2, 1, 2, 40, 64, "all_masked"),
            sdpa_case("causal_end_aligned", rng, 1, 4, 1, 3, 2, 64, "causal")]
    with open(OUT, "w") as f:
        json.dump({"gemm": gemm, "sdpa": sdpa}, f, separators=(",", ":"))
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
