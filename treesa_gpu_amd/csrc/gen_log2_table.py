"""Constants of the log2 core in tsa_math.h (TSA_LOG2_TAB, TSA_LOG2_A1..A6), printed as C.

For j = 0..127, c_j = 1 + j/128; entry j holds inv_j = 1/c_j rounded to double and t_j = -log2(inv_j)
rounded to double (so that log2(y) = t_j + log2(y * inv_j) exactly), both as IEEE-754 bit patterns.
A_k = (-1)^(k+1) / (k ln 2), the coefficients of log2(1 + z) = sum_k A_k z^k, rounded to double.
Rounding is exact (fractions.Fraction -> float rounds to nearest even); logarithms are evaluated with
60 significant decimal digits.  Run: python gen_log2_table.py
"""
import struct
from decimal import Decimal, getcontext
from fractions import Fraction

getcontext().prec = 60
LN2 = Decimal(2).ln()


def bits(x):
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def table():
    out = []
    for j in range(128):
        inv = float(Fraction(128, 128 + j))  # 1 / (1 + j/128), correctly rounded
        t = -(Decimal(Fraction(inv).numerator) / Decimal(Fraction(inv).denominator)).ln() / LN2
        out.append((bits(inv), bits(float(Fraction(t)))))
    return out


def coeffs():
    return [float(Fraction((-1) ** (k + 1)) / Fraction(Decimal(k) * LN2)) for k in range(1, 7)]


def main():
    print("#define TSA_LOG2_TAB \\")
    rows = table()
    print("  {" + ", \\\n   ".join(", ".join(f"0x{a:016x}ull, 0x{b:016x}ull" for a, b in rows[i:i + 2])
                                  for i in range(0, 128, 2)) + "}")
    for k, a in enumerate(coeffs(), 1):
        print(f"#define TSA_LOG2_A{k} {a.hex()}")


if __name__ == "__main__":
    main()
