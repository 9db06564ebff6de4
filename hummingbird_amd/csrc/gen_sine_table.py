"""Writes the table kPow2Mod2Pi of glu_act.h: 2^e mod 2 pi for e = 9 .. 120, rounded to double. pi comes from
Machin's formula (pi = 16 atan(1/5) - 4 atan(1/239)) evaluated with 120 significant decimal digits, which leaves
more than 40 correct digits in 2^120 mod 2 pi. Run: python gen_sine_table.py > table.txt"""
from decimal import Decimal, getcontext

getcontext().prec = 120


def atan_inv(n: int) -> Decimal:
    x = Decimal(1) / n
    x2, s, t, k = x * x, x, x, 1
    while True:
        t, k = -t * x2, k + 2
        term = t / k
        if abs(term) < Decimal(10) ** -115:
            return s
        s += term


TWO_PI = 2 * (16 * atan_inv(5) - 4 * atan_inv(239))
print(",\n".join(repr(float((Decimal(2) ** e) % TWO_PI)) for e in range(9, 121)))
