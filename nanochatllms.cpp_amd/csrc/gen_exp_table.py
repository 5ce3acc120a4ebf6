"""Prints the 2^(i/128) table of exp_ref (nc_exp64.h).

Entry 2i is the double nearest to the relative tail t_i = 2^(i/128) / H_i - 1
and entry 2i + 1 is bits(H_i) - (i << 45), where H_i is the double nearest to
2^(i/128); both are computed from 80-digit decimal arithmetic and rounded
once.  This is the table layout of the published exp algorithm that glibc
ships (ARM optimized-routines, EXP_TABLE_BITS = 7).

    python gen_exp_table.py > table.inc
"""
import struct
from decimal import Decimal, getcontext
from fractions import Fraction


def bits(x):
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def table():
    getcontext().prec = 80
    ln2 = Decimal(2).ln()
    out = []
    for i in range(128):
        exact = Fraction((Decimal(i) / 128 * ln2).exp())
        h = float(exact)  # nearest double
        t = float(exact / Fraction(h) - 1)
        out += [bits(t), (bits(h) - (i << 45)) & (2**64 - 1)]
    return out


if __name__ == "__main__":
    t = table()
    print(",\n".join("    " + ", ".join(f"0x{v:016x}ull" for v in t[j:j + 4]) for j in range(0, 256, 4)))
