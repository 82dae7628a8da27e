"""Writes fp8_e4m3_decode.bin: the 256 values of the reference's E4M3 decoder
(src/fp8.rs:94-112) as little-endian f32, computed here in the value domain
with Python floats (independent of the oracle's bit-level C decoder):

    0x7F (the reference's NaN sentinel, src/fp8.rs:33)  -> NaN (0x7FC00000)
    exponent field 0 (zero and would-be subnormals)     -> +0.0 for both signs
    otherwise  (-1)^s * 2^(e - 7) * (1 + m / 8)          (0xFF decodes to -480:
                                                         only 0x7F is NaN)

Run:  python tests/golden/make_fp8_decode.py  (rewrites the file beside it).
"""
import math
import os
import struct


def value(code: int) -> float:
    if code == 0x7F:
        return float("nan")
    s, e, m = code >> 7, (code >> 3) & 0xF, code & 0x7
    if e == 0:
        return 0.0
    return (-1.0 if s else 1.0) * math.ldexp(1.0 + m / 8.0, e - 7)


def table_bytes() -> bytes:
    out = bytearray()
    for c in range(256):
        v = value(c)
        out += struct.pack("<I", 0x7FC00000) if math.isnan(v) else struct.pack("<f", v)
    return bytes(out)


if __name__ == "__main__":
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fp8_e4m3_decode.bin")
    with open(path, "wb") as f:
        f.write(table_bytes())
