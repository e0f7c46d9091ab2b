"""Prints the 32-entry table used by exp_det (src/vecmath.c:44-52 in the
reference): the bits of 2^(j/32), correctly rounded to binary64, minus j << 47
(so that adding k << 47 to entry k mod 32 yields the bits of 2^(k/32)).
Computed here from the mathematics with 60-digit decimal arithmetic; the test
suite checks the oracle's and the GPU library's constants against it."""
import struct
from decimal import Decimal, getcontext


def exp2_table():
    getcontext().prec = 60
    ln2 = Decimal(2).ln()
    out = []
    for j in range(32):
        d = float((ln2 * j / 32).exp())  # float(Decimal) rounds correctly
        bits = struct.unpack("<Q", struct.pack("<d", d))[0]
        out.append((bits - (j << 47)) & 0xFFFFFFFFFFFFFFFF)
    return out


if __name__ == "__main__":
    t = exp2_table()
    for i in range(0, 32, 4):
        print("    " + ", ".join(f"0x{v:016x}u" for v in t[i:i + 4]) + ",")
