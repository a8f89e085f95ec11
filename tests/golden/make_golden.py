"""Write tests/golden/reference_vectors.json.

Inputs are the literal vectors of the reference's own tests for this path
(cited per case).  Expected outputs are computed here independently of the C
oracle: exact rational arithmetic for matmul, Python float64 (math.exp) for
softmax, closed forms for attention, exact u64 integer arithmetic for the
generators.  Run from the repo root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import math
from fractions import Fraction
from pathlib import Path

OUT = Path(__file__).resolve().parent / "reference_vectors.json"
M64 = (1 << 64) - 1
MUL = 6364136223846793005
INC_MMIX = 1442695040888963407


def lcg_states(seed: int, inc: int, n: int) -> list[int]:
    s, out = seed, []
    for _ in range(n):
        s = (s * MUL + inc) & M64
        out.append(s)
    return out


def u53(s: int) -> float:
    return (s >> 11) / float(1 << 53)


def f32(x: float) -> float:
    import struct
    return struct.unpack("f", struct.pack("f", x))[0]


def matmul_exact(a, ash, b, bsh):
    m, k = ash
    k2, n = bsh
    assert k == k2
    A = [Fraction(f32(x)) for x in a]  # the tensors hold f32 values
    B = [Fraction(f32(x)) for x in b]
    return [float(sum(A[i * k + p] * B[p * n + j] for p in range(k))) for i in range(m) for j in range(n)]


def softmax64(x):
    mx = max(x)
    e = [math.exp(v - mx) for v in x]
    s = sum(e)
    return [v / s for v in e]


def main() -> None:
    g: dict = {"_doc": __doc__.strip().splitlines()[0]}

    # ---- generators: rng.rs:20-70 (increment 1), lattice/constants.rs:11-49 (MMIX) ----
    gen = {}
    for seed in (0, 1, 2, 3, 4, 42, 12345):
        st = lcg_states(seed, 1, 8)
        gen[str(seed)] = {
            "states_inc1": [str(s) for s in st],
            "uniform_f64": [u53(s) for s in st],
            "uniform_pm1_f32": [f32(2.0 * u53(s) - 1.0) for s in st],
            "states_mmix": [str(s) for s in lcg_states(seed, INC_MMIX, 8)],
        }
        ms = lcg_states(seed, INC_MMIX, 16)
        normals = []
        for i in range(8):
            u1, u2 = u53(ms[2 * i]), u53(ms[2 * i + 1])
            normals.append(math.sqrt(-2.0 * math.log(max(u1, 1e-30))) * math.cos(2.0 * math.pi * u2))
        gen[str(seed)]["normal_f64"] = normals
    g["lcg"] = gen

    # ---- matmul: literal vectors of the reference tests ----
    mm = []

    def add_mm(name, a, ash, b, bsh, tol, src, ramps=None):
        d = {"name": name, "a_shape": ash, "b_shape": bsh,
             "expected": matmul_exact(a, ash, b, bsh), "tol": tol, "source": src}
        if ramps:  # inputs are f32(i * f32(scale) + offset), i = 0, 1, ... (kept as a formula)
            d["a_ramp"], d["b_ramp"] = ramps
        else:
            d["a"], d["b"] = a, b
        mm.append(d)

    add_mm("inline_2x2", [1, 2, 3, 4], [2, 2], [5, 6, 7, 8], [2, 2], 0.0,
           "crates/barracuda-core/src/ipc/methods_coverage_tests/sprint56b_tests.rs:618-645")
    add_mm("dot_1x3_3x1", [1, 0, 2], [1, 3], [1, 0, 3], [3, 1], 0.0,
           "crates/barracuda-core/src/ipc/methods_coverage_tests/sprint56b_tests.rs:649-669")
    add_mm("basic_2x3_3x2", [1, 2, 3, 4, 5, 6], [2, 3], [1, 2, 3, 4, 5, 6], [3, 2], 1e-5,
           "crates/barracuda/src/ops/matmul.rs:270-290")
    add_mm("identity_2x2", [1, 0, 0, 1], [2, 2], [5, 6, 7, 8], [2, 2], 1e-5,
           "crates/barracuda/src/ops/matmul.rs:299-318")
    add_mm("zeros_2x2", [0, 0, 0, 0], [2, 2], [1, 2, 3, 4], [2, 2], 1e-6,
           "crates/barracuda/src/ops/matmul.rs:319-335")
    add_mm("one_by_one", [5], [1, 1], [3], [1, 1], 1e-5,
           "crates/barracuda/src/ops/matmul.rs:343-356")
    add_mm("selector_4x2_2x3", [1, 2, 3, 4, 5, 6, 7, 8], [4, 2], [1, 0, 0, 0, 1, 0], [2, 3], 1e-5,
           "crates/barracuda/src/ops/matmul.rs:358-377")
    add_mm("precision_2x3_3x2", [1.234, 2.345, 3.456, 4.567, 5.678, 6.789], [2, 3],
           [0.111, 0.222, 0.333, 0.444, 0.555, 0.666], [3, 2], 1e-5,
           "crates/barracuda/src/ops/matmul.rs:413-443")
    c01 = f32(0.01)  # (i as f32) * 0.01 in f32; i * c01 is exact in f64, one rounding to f32
    a = [f32(i * c01) for i in range(64 * 32)]
    b = [f32(i * c01) for i in range(32 * 64)]
    add_mm("ramp_64x32_32x64", a, [64, 32], b, [32, 64], 1e-3,
           "crates/barracuda/src/ops/matmul.rs:381-409", ([0.01, 0.0], [0.01, 0.0]))
    a = [f32(i * c01) for i in range(64 * 64)]
    b = [f32(i * c01 + 0.5) for i in range(64 * 64)]  # (i as f32).mul_add(0.01, 0.5)
    add_mm("ramp_64x64_cross_vendor", a, [64, 64], b, [64, 64], 0.05,
           "crates/barracuda/tests/hardware_verification.rs:272-330", ([0.01, 0.0], [0.01, 0.5]))
    g["matmul"] = mm

    # ---- batched matmul: ops/batch_matmul.rs:172-199 ----
    A = [1, 2, 3, 4, 5, 6, 1, 1, 1, 2, 2, 2]
    B = [1, 0, 0, 1, 1, 1, 2, 0, 0, 2, 1, 1]
    exp = matmul_exact(A[:6], [2, 3], B[:6], [3, 2]) + matmul_exact(A[6:], [2, 3], B[6:], [3, 2])
    g["batch_matmul"] = [{"name": "basic_2x2x3_2x3x2", "a": A, "a_shape": [2, 2, 3], "b": B,
                          "b_shape": [2, 3, 2], "expected": exp, "tol": 0.0,
                          "source": "crates/barracuda/src/ops/batch_matmul.rs:172-199"}]

    # ---- softmax: literal vectors ----
    sm = []

    def add_sm(name, x, shape, src, extra=None):
        cols = shape[-1]
        exp = []
        for r in range(len(x) // cols):
            exp += softmax64([f32(v) for v in x[r * cols:(r + 1) * cols]])
        d = {"name": name, "x": x, "shape": shape, "expected": exp, "source": src}
        if extra:
            d.update(extra)
        sm.append(d)

    add_sm("inc_1_2_3", [1.0, 2.0, 3.0], [3], "crates/barracuda/src/ops/softmax.rs:151-166",
           {"sum_tol": 1e-5, "monotone": True})
    add_sm("tiny_1e-6", [1e-6, 2e-6, 3e-6], [3], "crates/barracuda/src/ops/softmax.rs:168-178",
           {"sum_tol": 1e-5})
    add_sm("large_100_200_300", [100.0, 200.0, 300.0], [3], "crates/barracuda/src/ops/softmax.rs:180-191",
           {"sum_tol": 1e-5, "last_gt": 0.99})
    add_sm("ramp_1000", [f32(i / 10.0) for i in range(1000)], [1000],
           "crates/barracuda/src/ops/softmax.rs:193-206", {"sum_tol": 1e-4})
    add_sm("one_to_five", [1.0, 2.0, 3.0, 4.0, 5.0], [5], "crates/barracuda/src/ops/softmax.rs:208-233",
           {"tol": 1e-5})
    add_sm("cross_hw_1_to_5", [1.0, 2.0, 3.0, 4.0, 5.0], [5],
           "crates/barracuda/tests/cross_hardware_parity.rs:192-230", {"tol": 1e-4})
    add_sm("cross_vendor_1_to_8", [float(i) for i in range(1, 9)], [8],
           "crates/barracuda/tests/hardware_verification.rs:384-420", {"tol": 1e-3})
    add_sm("single_100", [100.0], [1],
           "crates/barracuda-core/src/ipc/methods_coverage_tests/wave79_cpu_edge_tests.rs:321-335",
           {"tol": 0.0})
    add_sm("rows_2x3", [1, 2, 3, 4, 5, 6], [2, 3], "crates/barracuda/src/ops/tensor_axis_ops.rs:158-180",
           {"sum_tol": 1e-5})
    add_sm("single_col_3x1", [1.0, 2.0, 3.0], [3, 1], "crates/barracuda/src/ops/tensor_axis_ops.rs:189-195",
           {"tol": 0.0})
    # softmax_dim(0) of [3,2] [[1,4],[2,5],[3,6]]: each column sums to 1 (tensor_axis_ops.rs:175-184)
    x = [1.0, 4.0, 2.0, 5.0, 3.0, 6.0]
    c0, c1 = softmax64(x[0::2]), softmax64(x[1::2])
    sm.append({"name": "columns_3x2_axis0", "x": x, "shape": [3, 2], "axis": 0,
               "expected": [c0[0], c1[0], c0[1], c1[1], c0[2], c1[2]], "sum_tol": 1e-5,
               "source": "crates/barracuda/src/ops/tensor_axis_ops.rs:175-184"})
    g["softmax"] = sm

    # ---- attention closed forms ----
    att = []
    # uniform Q and K -> every score equal -> output = mean of V rows
    B, H, S, D = 1, 2, 4, 8
    v = [float((i * 7) % 11) for i in range(B * H * S * D)]
    exp = []
    for h in range(B * H):
        for i in range(S):
            for d in range(D):
                exp.append(sum(v[(h * S + j) * D + d] for j in range(S)) / S)
    att.append({"name": "uniform_qk_mean_v", "shape": [B, H, S, D], "q": [0.5] * (B * H * S * D),
                "k": [0.25] * (B * H * S * D), "v": v, "causal": False, "expected": exp, "tol": 1e-5,
                "source": "crates/barracuda/src/ops/attention/tests.rs:8-29"})
    # V == 2 everywhere -> output 2 (flash_attention.rs:152-185 uses the same identity)
    att.append({"name": "constant_v_two", "shape": [1, 1, 16, 4], "q": [float(i % 5) for i in range(64)],
                "k": [float(i % 3) for i in range(64)], "v": [2.0] * 64, "causal": False,
                "expected": [2.0] * 64, "tol": 1e-6,
                "source": "crates/barracuda/src/ops/flash_attention.rs:152-185"})
    # single key -> that V row (ml_tests.rs:147-165: V = [42, 7])
    att.append({"name": "single_key", "shape_q": [1, 1, 1, 2], "shape_kv": [1, 1, 1, 2], "q": [1.0, 0.0],
                "k": [0.3, 0.9], "v": [42.0, 7.0], "causal": False, "expected": [42.0, 7.0], "tol": 1e-6,
                "source": "crates/barracuda-core/src/ipc/methods/ml_tests.rs:147-165"})
    # one-hot Q/K, V = [[10,20],[30,40]] (ml_tests.rs:128-145): row i = softmax([q_i.k_j]/sqrt(2)) V
    q = [1.0, 0.0, 0.0, 1.0]
    k = [1.0, 0.0, 0.0, 1.0]
    vv = [10.0, 20.0, 30.0, 40.0]
    exp = []
    for i in range(2):
        s = [sum(q[i * 2 + d] * k[j * 2 + d] for d in range(2)) / math.sqrt(2.0) for j in range(2)]
        p = softmax64(s)
        exp += [sum(p[j] * vv[j * 2 + d] for j in range(2)) for d in range(2)]
    att.append({"name": "one_hot_2x2", "shape": [1, 1, 2, 2], "q": q, "k": k, "v": vv, "causal": False,
                "expected": exp, "tol": 1e-5,
                "source": "crates/barracuda-core/src/ipc/methods/ml_tests.rs:128-145"})
    # causal with equal scores: row i = mean(V[0..=i]); row 0 = V[0] exactly
    S, D = 5, 3
    v = [float(3 * i + d) for i in range(S) for d in range(D)]
    exp = []
    for i in range(S):
        for d in range(D):
            exp.append(sum(v[j * D + d] for j in range(i + 1)) / (i + 1))
    att.append({"name": "causal_equal_scores_prefix_mean", "shape": [1, 1, S, D], "q": [0.0] * (S * D),
                "k": [1.0] * (S * D), "v": v, "causal": True, "expected": exp, "tol": 1e-6,
                "source": "crates/barracuda/src/ops/causal_attention.rs:85-122 (mask j <= i)"})
    g["attention"] = att

    # ---- inline-data f64 handlers (tensor.matmul_inline, ml.attention): f64 throughout ----
    inl = []
    for name, lhs, rhs, src in (
            ("matmul_inline_2x2", [[1.0, 2.0], [3.0, 4.0]], [[5.0, 6.0], [7.0, 8.0]],
             "crates/barracuda-core/src/ipc/methods_coverage_tests/sprint56b_tests.rs:618-645"),
            ("matmul_inline_non_square", [[1.0, 0.0, 2.0]], [[1.0], [0.0], [3.0]],
             "crates/barracuda-core/src/ipc/methods_coverage_tests/sprint56b_tests.rs:647-669")):
        m, k, n = len(lhs), len(rhs), len(rhs[0])
        exp = [[float(sum(Fraction(lhs[i][p]) * Fraction(rhs[p][j]) for p in range(k))) for j in range(n)]
               for i in range(m)]
        inl.append({"name": name, "method": "tensor.matmul_inline", "params": {"lhs": lhs, "rhs": rhs},
                    "expected": exp, "shape": [m, n], "tol": 0.0, "source": src})
    # one key: its weight is exp(0) / exp(0) = 1 exactly, so the output is that V row exactly
    inl.append({"name": "ml_attention_single_token", "method": "ml.attention",
                "params": {"q": [[1.0, 0.0]], "k": [[1.0, 0.0]], "v": [[42.0, 7.0]]},
                "expected": [[42.0, 7.0]], "tol": 0.0,
                "source": "crates/barracuda-core/src/ipc/methods_coverage_tests/ml_tests.rs:147-165"})
    # one-hot q and k: scores [[a, 0], [0, a]] with a = 1/sqrt(2); row i = softmax(scores_i) V
    a = 1.0 / math.sqrt(2.0)
    vv = [[10.0, 20.0], [30.0, 40.0]]
    exp = []
    for i in range(2):
        p = softmax64([a if j == i else 0.0 for j in range(2)])
        exp.append([p[0] * vv[0][d] + p[1] * vv[1][d] for d in range(2)])
    inl.append({"name": "ml_attention_one_hot", "method": "ml.attention",
                "params": {"q": [[1.0, 0.0], [0.0, 1.0]], "k": [[1.0, 0.0], [0.0, 1.0]], "v": vv},
                "expected": exp, "tol": 1e-14,
                "source": "crates/barracuda-core/src/ipc/methods_coverage_tests/ml_tests.rs:128-145"})
    g["inline_f64"] = inl

    OUT.write_text(json.dumps(g, indent=1))
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
