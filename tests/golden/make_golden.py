"""Write tests/golden/kat_w8a8.json: known-answer vectors for the W8A8 hot path.

The reference (akivet/Mica) ships no golden vectors for this path, so these are derived from the
mathematics alone, in pure Python, independently of oracle/ and of numpy:

  * fp32 steps are evaluated in double and rounded once with struct.pack('f') (round to nearest
    even).  For + - * of two fp32 values the double result is exact (products of two 24-bit
    significands fit in 53 bits; int32 x fp32 products used here fit too), so rounding it once
    is the IEEE fp32 result.  For / and sqrt, double rounding through binary64 is innocuous since
    53 >= 2 * 24 + 2 (Figueroa, "When is double rounding innocuous?", 1995).
  * bf16 conversion rounds the fp32 bit pattern to nearest even on integers.
  * inputs are chosen so most answers are also checkable by hand (scales that are powers of two,
    exact .5 ties, constant rows, all-zero rows, the largest int8 products).

Run:  python tests/golden/make_golden.py   (deterministic; rewrites the JSON)
"""
from __future__ import annotations

import json
import math
import random
import struct
from pathlib import Path

OUT = Path(__file__).resolve().parent / "kat_w8a8.json"


def r32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def bits_f32(u: int) -> float:
    return struct.unpack("<f", struct.pack("<I", u))[0]


def bf16_bits(x: float) -> int:
    u = f32_bits(r32(x))
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF


def bf16_val(b: int) -> float:
    return bits_f32(b << 16)


def rint_even(v: float) -> float:
    f = math.floor(v)
    d = v - f
    if d > 0.5:
        return f + 1.0
    if d < 0.5:
        return f
    return f if f % 2 == 0 else f + 1.0


def quant_row(xs, inv=None, rounding="even"):
    xf = [r32(x * i) for x, i in zip(xs, inv)] if inv is not None else [r32(x) for x in xs]
    amax = max(abs(v) for v in xf)
    s = r32(max(amax, r32(1e-8)) / 127.0)
    q = []
    for v in xf:
        t = r32(v / s)
        if rounding == "even":
            r = rint_even(t)
        else:
            r = float(math.trunc(r32(t + 0.5) if t >= 0 else r32(t - 0.5)))
        q.append(int(max(-127.0, min(127.0, r))))
    return q, s


def quant_cases():
    cases = []
    # s = 1 exactly: the ties 0.5, 1.5, 2.5, 126.5 and their negatives
    cases.append([127.0, 0.5, -0.5, 1.5, 2.5, -2.5, 126.5, -127.0, 3.0, -1.5, 0.0, 64.5, -64.5, 100.25, 7.5, -7.5])
    # s = 2 exactly (amax 254): x / s = 127, .5 ties, 1.5, 2.5
    cases.append([254.0, 1.0, 3.0, 5.0, -1.0, -3.0, -5.0, 2.0, 9.0, -9.0, 0.0, 250.0, -250.0, 127.0, -253.0, 17.0])
    # s = 1/4 (amax 31.75 = 127/4)
    cases.append([31.75, 0.125, -0.125, 0.375, 0.625, -0.375, 10.0, -31.75, 0.0, 1.0, 2.0, 3.125, -3.125, 5.5, 6.5, -7.0])
    # all-zero row: s = 1e-8 / 127, q = 0
    cases.append([0.0] * 16)
    # one non-zero element
    cases.append([0.0] * 7 + [-3.0] + [0.0] * 8)
    # tiny values below the 1e-8 floor of the absmax
    cases.append([bf16_val(bf16_bits(v)) for v in (1e-9, -5e-10, 2e-9, 0.0, 7e-10, -1e-9, 3e-10, 0.0,
                                                     1e-10, -2e-9, 4e-10, 0.0, 6e-10, -8e-10, 9e-10, 1.5e-9)])
    # generic bf16 row with an outlier
    rnd = random.Random(20261201)
    row = [bf16_val(bf16_bits(rnd.gauss(0.0, 1.0))) for _ in range(32)]
    row[5] = bf16_val(bf16_bits(row[5] * 20.0))
    cases.append(row)
    out = []
    for xs in cases:
        xs = [bf16_val(bf16_bits(x)) for x in xs]
        qe, s = quant_row(xs, None, "even")
        qa, _ = quant_row(xs, None, "away")
        out.append({"x_bf16": [bf16_bits(x) for x in xs], "s": s, "s_bits": f32_bits(s), "q_even": qe,
                    "q_away": qa})
    # smoothing: xf = x * inv
    xs = [1.0, 2.0, -0.5, 4.0, 0.25, 8.0, -1.0, 3.0]
    inv = [127.0, 0.5, 3.0, 0.25, 2.0, 0.125, 1.0, 0.5]
    qe, s = quant_row(xs, inv, "even")
    qa, _ = quant_row(xs, inv, "away")
    out.append({"x_bf16": [bf16_bits(x) for x in xs], "inv": inv, "s": s, "s_bits": f32_bits(s), "q_even": qe,
                "q_away": qa})
    return out


def weight_cases():
    """quant_weight known answers (int8_quant.py:54-61): a weight matrix [N, K] quantized per output row,
    i.e. quant_row applied to every row with half-even rounding.  The matrices are fp32 (offline weights
    are fp32 after smoothing): exact .5 ties at s = 1 and s = 1/2, an all-zero row (s = 1e-8 / 127), a
    single-element row, rows below the 1e-8 floor, a row of one repeated value (q = +-127 everywhere)."""
    mats = [
        [[127.0, 0.5, -0.5, 1.5, 2.5, -2.5, 126.5, -126.5],
         [63.5, 0.25, -0.25, 0.75, 1.25, -1.25, 62.75, -0.0],
         [0.0] * 8,
         [1e-9, -3e-9, 5e-9, 0.0, 2e-10, -7e-9, 4e-9, 1e-9],
         [-2.0] * 8],
        [[5.0], [-0.0], [1e-12]],
    ]
    rnd = random.Random(20261202)
    mats.append([[r32(rnd.gauss(0.0, 0.05)) for _ in range(24)] for _ in range(6)])
    out = []
    for w in mats:
        w = [[r32(v) for v in row] for row in w]
        qs = [quant_row(row, None, "even") for row in w]
        out.append({"w_f32_bits": [[f32_bits(v) for v in row] for row in w], "q": [q for q, _ in qs],
                    "s_bits": [f32_bits(s) for _, s in qs]})
    return out


def gemm_cases():
    rnd = random.Random(7)
    out = []
    # hand case, K = 32: A rows (1, 2, 0...), (-3, 4, ...), B rows
    M, N, K = 3, 4, 32
    A = [[0] * K for _ in range(M)]
    B = [[0] * K for _ in range(N)]
    A[0][0], A[0][1] = 1, 2
    A[1][0], A[1][31] = -3, 4
    A[2] = [-127] * K
    B[0][0] = 5
    B[1][1], B[1][31] = -7, 1
    B[2] = [-127] * K
    B[3] = [127 if k % 2 else -127 for k in range(K)]
    sa = [1.0, 0.5, r32(1.0 / 3.0)]
    sb = [1.0, 2.0, r32(0.1), r32(1e-3)]
    out.append((A, B, sa, sb, None))
    # random case with scales ~U(1e-3, 1e-2) and extremes, K = 64
    M, N, K = 5, 6, 64
    A = [[rnd.randint(-127, 127) for _ in range(K)] for _ in range(M)]
    B = [[rnd.randint(-127, 127) for _ in range(K)] for _ in range(N)]
    A[4] = [127] * K
    B[5] = [-127] * K
    sa = [r32(rnd.uniform(1e-3, 1e-2)) for _ in range(M)]
    sb = [r32(rnd.uniform(1e-3, 1e-2)) for _ in range(N)]
    bias = [r32(rnd.uniform(-1, 1)) for _ in range(N)]
    out.append((A, B, sa, sb, bias))
    # the largest accumulator of a 2560-long row: 2560 * 127 * 127 = 41,290,240
    M, N, K = 2, 2, 2560
    A = [[-127] * K, [127 if k % 3 else -127 for k in range(K)]]
    B = [[-127] * K, [127] * K]
    out.append((A, B, [1.0, r32(1.0 / 127)], [1.0, r32(0.01)], None))
    # a case where the epilogue's multiply order shows in the bf16 result: (acc * sa) * sb differs
    # from acc * (sa * sb) after rounding (found by a deterministic search)
    srch = random.Random(3)
    while True:
        a, b = srch.randint(-127, 127), srch.randint(-127, 127)
        s1, s2 = r32(srch.uniform(1e-3, 1e-2)), r32(srch.uniform(1e-3, 1e-2))
        acc = float(a * b)
        if bf16_bits(r32(r32(acc * s1) * s2)) != bf16_bits(r32(acc * r32(s1 * s2))):
            break
    A = [[a] + [0] * 15]
    B = [[b] + [0] * 15]
    out.append((A, B, [s1], [s2], None))
    res = []
    for A, B, sa, sb, bias in out:
        acc = [[sum(a * b for a, b in zip(ar, br)) for br in B] for ar in A]
        y = []
        for m in range(len(A)):
            row = []
            for n in range(len(B)):
                v = r32(r32(r32(float(acc[m][n])) * sa[m]) * sb[n])
                if bias is not None:
                    v = r32(v + bias[n])
                row.append(bf16_bits(v))
            y.append(row)
        res.append({"A": A, "B": B, "sa": sa, "sb": sb, "bias": bias, "acc": acc, "y_bf16": y})
    return res


def norm_cases():
    out = []
    K = 64
    # constant rows with eps = 0: rstd = 1 / |c| exactly, so y = sign(c) * (offset + w)
    w = [bf16_val(bf16_bits(0.5 + 0.03125 * (k % 16) - 0.25)) for k in range(K)]
    for c, offset in ((2.0, 1.0), (-0.5, 1.0), (4.0, 0.0), (0.25, 0.0)):
        x = [c] * K
        y = norm_row(x, w, 0.0, offset)
        out.append({"x_bf16": [bf16_bits(v) for v in x], "w": w, "eps": 0.0, "offset": offset, "y_bf16": y})
    # a generic row, eps = 1e-6; the exact sum of squares is formed on integers
    rnd = random.Random(11)
    x = [bf16_val(bf16_bits(rnd.gauss(0.0, 1.0))) for _ in range(K)]
    x[3] = bf16_val(bf16_bits(x[3] * 20.0))
    w2 = [bf16_val(bf16_bits(rnd.gauss(1.0, 0.1))) for _ in range(K)]
    out.append({"x_bf16": [bf16_bits(v) for v in x], "w": w2, "eps": 1e-6, "offset": 0.0,
                "y_bf16": norm_row(x, w2, 1e-6, 0.0)})
    # a row where the multiply order (x * rstd) * w1 vs x * (rstd * w1) shows in bf16 (searched)
    srch = random.Random(5)
    while True:
        x = [bf16_val(bf16_bits(srch.gauss(0.0, 1.0))) for _ in range(K)]
        w3 = [bf16_val(bf16_bits(srch.gauss(0.0, 0.1))) for _ in range(K)]
        y = norm_row(x, w3, 1e-6, 1.0)
        rstd = norm_rstd(x, 1e-6)
        alt = [bf16_bits(r32(v * r32(rstd * r32(1.0 + wv)))) for v, wv in zip(x, w3)]
        if alt != y:
            break
    out.append({"x_bf16": [bf16_bits(v) for v in x], "w": w3, "eps": 1e-6, "offset": 1.0, "y_bf16": y})
    return out


def norm_rstd(x, eps):
    from fractions import Fraction
    ss32 = r32(float(sum(Fraction(v) * Fraction(v) for v in x)))
    return r32(1.0 / r32(math.sqrt(r32(r32(ss32 / len(x)) + r32(eps)))))


def norm_row(x, w, eps, offset):
    # sum of squares exactly (fractions), rounded once to fp32; mean = RN32(ss / K)
    from fractions import Fraction
    ss = sum(Fraction(v) * Fraction(v) for v in x)
    ss32 = r32(float(ss))
    mean = r32(ss32 / len(x))
    rstd = r32(1.0 / r32(math.sqrt(r32(mean + r32(eps)))))
    return [bf16_bits(r32(r32(v * rstd) * r32(offset + wv))) for v, wv in zip(x, w)]


def silu_cases():
    # closed forms: silu(0) = 0; silu(g) = g for g >= 96 (exp(-g) < 2^-138, 1 + exp(-g) == 1 in fp32);
    # silu(g) = -0 for g <= -128 (the quotient underflows below the bf16 range's resolution)
    g = [0.0, 96.0, 128.0, 1024.0, -128.0, -1024.0, 200.0, -200.0]
    u = [3.0, 0.5, -2.0, 1.0, 5.0, 7.0, -0.25, 1.0]
    h = []
    for gv, uv in zip(g, u):
        act = 0.0 if gv == 0.0 else (gv if gv > 0 else -0.0)
        h.append(bf16_bits(r32(bf16_val(bf16_bits(act)) * uv)))
    return {"g_bf16": [bf16_bits(v) for v in g], "u_bf16": [bf16_bits(v) for v in u], "h_bf16": h}


def softmax_cases():
    return [
        {"z": [0.0, math.log(3.0)], "p": [0.25, 0.75]},
        {"z": [5.0, 5.0, 5.0, 5.0], "p": [0.25, 0.25, 0.25, 0.25]},
        {"z": [0.0, math.log(2.0), math.log(5.0)], "p": [0.125, 0.25, 0.625]},
    ]


def main():
    data = {
        "note": "known answers for the W8A8 hot path; generated by tests/golden/make_golden.py",
        "quant": quant_cases(),
        "quant_weight": weight_cases(),
        "gemm": gemm_cases(),
        "rms_norm": norm_cases(),
        "silu_mul": silu_cases(),
        "softmax": softmax_cases(),
    }
    OUT.write_text(json.dumps(data, separators=(",", ":")) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
