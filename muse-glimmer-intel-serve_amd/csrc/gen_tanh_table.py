"""Writes the tanh table of mg_tanh_fast.hpp: kTanhTab[k] = tanh((k + 0.5) / 128)
rounded to the nearest double, k = 1..127, and kTanhTab[0] = tanh(0) = 0 (the
first interval's polynomial is taken about 0), evaluated in 60-digit decimal
arithmetic (tanh x = (e^2x - 1) / (e^2x + 1); CPython's Decimal -> float
conversion rounds correctly). Run: python3 gen_tanh_table.py > table.inc"""
from decimal import Decimal, getcontext

getcontext().prec = 60


def tanh_rn(x):
    e = (2 * x).exp()
    return float((e - 1) / (e + 1))


vals = [0.0] + [tanh_rn(Decimal(2 * k + 1) / Decimal(256)) for k in range(1, 128)]
print("    // tanh((k + 0.5) / 128), correctly rounded, and tanh(0) at k = 0 (gen_tanh_table.py)")
print("    alignas(16) inline constexpr double kTanhTab[128] = {")
for i in range(0, 128, 4):
    print("        " + ", ".join(v.hex() for v in vals[i:i + 4]) + ",")
print("    };")
