"""Writes q8_0_known_answers.json: Q8_0 blocks whose quantisation is fixed by
construction (GGML block_q8_0 / candle BlockQ8_0::from_float: d = amax/127,
q = round-half-away(x / d), d stored as f16).

Each case picks amax so that d = amax/127 is an exact power of two (or zero),
so x * (1/d) is exact and q follows from integer arithmetic; the expected
values below are written from that construction, not computed by any
quantiser.  Run: python make_q8_0_known_answers.py
"""
import json
from pathlib import Path


def f16_bits_pow2(e):
    """f16 bits of 2**e (normal or subnormal)."""
    if e >= -14:
        return (e + 15) << 10
    return 1 << (e + 24)


def rh_away(v):
    """Round half away from zero for exact rationals given as (num, den)."""
    num, den = v
    s = -1 if num < 0 else 1
    n = abs(num)
    q, r = divmod(n, den)
    if 2 * r >= den:
        q += 1
    return s * q


cases = []


def add(name, xs_num, den_pow, e_d, note):
    """x_j = xs_num[j] * 2**den_pow; d = 2**e_d; q_j = round(x_j / d)."""
    x = [n * 2.0**den_pow for n in xs_num]
    # x / d = n * 2**(den_pow - e_d)
    sh = den_pow - e_d
    q = [rh_away((n * 2**sh, 1)) if sh >= 0 else rh_away((n, 2**(-sh))) for n in xs_num]
    cases.append({"name": name, "x": x, "d_bits": f"{f16_bits_pow2(e_d):04x}", "q": q,
                  "derivation": note})


ints = [127, -127] + [(-1) ** j * (j * 7 % 127) for j in range(30)]
add("integers_amax_127", ints, 0, 0, "amax 127 -> d = 1, q = x")
add("negative_amax", [-127] + [j * 4 - 60 for j in range(31)], 0, 0, "amax from a negative value")
add("halves_d_half", [127] + [j * 8 - 124 for j in range(31)], -1, -1, "x = k/2, amax 63.5 -> d = 0.5, q = k")
add("pow2_scale_2^-6", [127, -3, 5] + list(range(-58, 58, 4)), -6, -6, "amax 127*2^-6 -> d = 2^-6")
add("ties_d1", [254, 1, -1, 3, -3, 5, -5, 253, -253] + [0] * 23, -1, 0,
    "d = 1: x = +-0.5, 1.5, 2.5, 126.5 round away from zero")
add("ties_d_half", [254, 1, -3, 5, -7, 9] + [0] * 26, -2, -1,
    "d = 0.5: x*2 = 0.5, -1.5, 2.5, -3.5, 4.5 round away from zero")
add("subnormal_d", [127] + list(range(-15, 16)), -20, -20, "d = 2^-20 is an f16 subnormal (bits 0x0010)")
add("tiny_subnormal_d", [127, -64, 63, 1, -1] + [0] * 27, -24, -24, "d = 2^-24, the smallest f16 subnormal")
cases.append({"name": "zeros", "x": [0.0] * 32, "d_bits": "0000", "q": [0] * 32,
              "derivation": "amax 0 -> d = 0, id = 0, q = 0"})
for c in cases:
    assert len(c["x"]) == 32 and len(c["q"]) == 32 and all(-128 <= v <= 127 for v in c["q"])

Path(__file__).with_name("q8_0_known_answers.json").write_text(
    json.dumps({"source": "constructed; see make_q8_0_known_answers.py", "cases": cases}, indent=1))
print(len(cases), "cases")
