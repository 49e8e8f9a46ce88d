"""The 32-entry table of the softmax's exp (kExp2Table in nn-cpp_amd/src/kernels/hip/softmax_row.hpp), from its
definition: entry i = bits of 2^(i/32) rounded to the nearest double, minus i << 47 (mod 2^64). 2^(i/32) is
evaluated with 60-digit decimal arithmetic and converted by Python's correctly rounded float().

  python tests/golden/expf_table.py     # prints the table
"""
import struct
from decimal import Decimal, getcontext


def exp2_table():
    getcontext().prec = 60
    ln2 = Decimal(2).ln()
    out = []
    for i in range(32):
        d = float((Decimal(i) / 32 * ln2).exp())
        bits = struct.unpack("<Q", struct.pack("<d", d))[0]
        out.append((bits - (i << 47)) % (1 << 64))
    return out


if __name__ == "__main__":
    for i, v in enumerate(exp2_table()):
        print(f"{i:2d} 0x{v:016x}")
