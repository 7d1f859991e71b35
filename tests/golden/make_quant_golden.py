"""Writes tests/golden/quant_golden.json: hand-derivable known answers for the
ggml block quantizers and fp16 rounding.

Inputs are chosen so that every expected value follows from exact integer /
power-of-two arithmetic (no rounding ambiguity except the ones each case is
built to probe), and the expected outputs are computed here from the
published ggml rules written as integer formulas — not by the oracle:

  Q4_0 (quantize_row_q4_0_ref): d = max/−8 where max is the signed value of
        largest magnitude, q = min(15, trunc(x/d + 8.5)).
  Q4_1 (quantize_row_q4_1_ref): d = (max−min)/15, q = min(15, trunc((x−min)/d + 0.5)).
  Q8_0 weights (quantize_row_q8_0_ref): d = amax/127, q = round-half-away(x/d).
  Q8_0 activations (x86 quantize_row_q8_0): q = round-half-even(x·127/amax).
  fp16: IEEE binary16 round-to-nearest-even.

Run: python3 tests/golden/make_quant_golden.py
"""
import json
import os
from fractions import Fraction

HERE = os.path.dirname(os.path.abspath(__file__))


def round_half_even(fr: Fraction) -> int:
    f = fr.numerator // fr.denominator
    rem = fr - f
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and f % 2 == 1):
        return f + 1
    return f


def round_half_away(fr: Fraction) -> int:
    s = -1 if fr < 0 else 1
    a = abs(fr)
    f = a.numerator // a.denominator
    return s * (f + 1 if a - f >= Fraction(1, 2) else f)


def trunc(fr: Fraction) -> int:
    a = abs(fr)
    v = a.numerator // a.denominator
    return v if fr >= 0 else -v


def main():
    cases = {}
    # Q4_0: x_j = j/4 − 4 (j = 0..31): max magnitude −4 → d = 0.5, 1/d = 2 exactly,
    # x/d + 8.5 = j/2 + 0.5 → q_j = min(15, floor(j/2 + 0.5)); the last value
    # (x = 3.75 → 16) exercises the clamp to 15.
    x = [Fraction(j, 4) - 4 for j in range(32)]
    d = Fraction(-4) / -8
    q = [min(15, trunc(xi / d + Fraction(17, 2))) for xi in x]
    cases["q4_0"] = {"x": [float(v) for v in x], "d": float(d), "q": q}
    # Q4_1: x_j = j/8 − 1 (j = 0..31): min −1, max 2.875, d = 3.875/15; chosen
    # because d is not a power of two, the rule is evaluated in float32 by ggml
    # (id = 1/d), so only the endpoint codes are hand-fixed: min → 0, max → 15.
    x = [Fraction(j, 8) - 1 for j in range(32)]
    cases["q4_1_ends"] = {"x": [float(v) for v in x], "q_first": 0, "q_last": 15,
                          "m": -1.0, "d": float((x[-1] - x[0]) / 15)}
    # Q8_0 weights vs activations on ties: amax = 127 → d = 1 and id = 1, so
    # x/d = x·127/amax = x exactly; x = k + 0.5 separates the two roundings.
    ties = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, -3.5, 100.5, -100.5, 126.5, -126.5]
    ties += [0.25 * i for i in range(32 - len(ties))]
    xt = [Fraction(v) for v in ties]
    cases["q8_ties"] = {
        "x": ties,
        "d": 1.0,
        "q_weights_round_half_away": [round_half_away(v) for v in xt],
        "q_activations_round_half_even": [round_half_even(v) for v in xt],
    }
    # fp16 ties: 1 + k·2^-11 lies exactly between two binary16 neighbours for
    # odd k; RNE picks the even mantissa.
    f16 = []
    for k in range(1, 40, 2):
        v = 1 + Fraction(k, 2048)
        lo = (k - 1) // 2  # mantissa of the lower neighbour (ulp 2^-10)
        m = lo if lo % 2 == 0 else lo + 1
        f16.append({"x": float(v), "bits": 0x3C00 + m})
    # overflow boundary: 65504 is the largest finite; 65520 (the midpoint to 2^16) rounds to inf
    f16.append({"x": 65504.0, "bits": 0x7BFF})
    f16.append({"x": 65519.0, "bits": 0x7BFF})
    f16.append({"x": 65520.0, "bits": 0x7C00})
    # smallest subnormal 2^-24 and the midpoint 2^-25 (ties to even → 0)
    f16.append({"x": 2.0 ** -24, "bits": 0x0001})
    f16.append({"x": 2.0 ** -25, "bits": 0x0000})
    f16.append({"x": 3 * 2.0 ** -25, "bits": 0x0002})
    cases["fp16"] = f16
    with open(os.path.join(HERE, "quant_golden.json"), "w") as f:
        json.dump(cases, f, indent=1)


if __name__ == "__main__":
    main()
