"""Writes known_blocks.json: hand-specified GGUF blocks and their values.

Each block is described by its integer fields (scales, mins, quants) and its
f16 super-scales; this script PACKS those fields into the GGUF byte layout
(an encoder written from the format description, independent of the
oracle's and the kernels' decoders) and records the expected values computed
from the integer fields, not from the bytes.  The tests decode the bytes and
must reproduce the values exactly.

Format description followed (GGUF block layouts, as written by the
reference's quantizer, tools/quantize.cpp:375-383):
  Q8_0  34 B : f16 d, int8 q[32];                   y = d*q
  Q4_K 144 B : f16 d, f16 dmin, u8 scales[12], u8 qs[128]
               (sc_j, m_j) 6-bit, j<4: low 6 bits of bytes j / j+4;
               j>=4: low nibble / high nibble of byte j+4, top 2 bits from
               the top bits of bytes j-4 / j; element e: chunk c=e//64 byte
               qs[32c + e%32], low nibble if e%64<32 else high nibble;
                                                    y = (d*sc_j)*q - dmin*m_j
  Q5_K 176 B : f16 d, f16 dmin, u8 scales[12], u8 qh[32], u8 qs[128]
               scales and the low 4 bits of each quant as Q4_K; the fifth
               bit of element e is bit e//32 of qh[e%32];
                                                    y = (d*sc_j)*q - dmin*m_j
  Q6_K 210 B : u8 ql[128], u8 qh[64], int8 sc[16], f16 d
               element e: h=e//128, t=(e%128)//32, l=e%32:
               low 4 bits in ql[64h+l+32(t&1)] (low nibble if t<2),
               high 2 bits in qh[32h+l] at bit 2t;   y = (d*sc[e//16])*(q-32)
Expected values are evaluated in float32 with the two roundings written
above (products formed left to right, no fused multiply-add).

Run:  python tests/golden/make_known_blocks.py
"""
import json
import pathlib

import numpy as np

OUT = pathlib.Path(__file__).resolve().parent / "known_blocks.json"


def f16bits(v):
    return int(np.array([v], dtype=np.float16).view(np.uint16)[0])


def f16val(bits):
    return np.array([bits], dtype=np.uint16).view(np.float16).astype(np.float32)[0]


def q8_0_block(d_bits, q):
    b = bytearray(34)
    b[0:2] = d_bits.to_bytes(2, "little")
    b[2:34] = np.array(q, dtype=np.int8).tobytes()
    d = f16val(d_bits)
    exp = [float(np.float32(d) * np.float32(v)) for v in q]
    return bytes(b), exp


def q4_K_block(d_bits, dmin_bits, sc, mn, q):
    assert len(sc) == len(mn) == 8 and len(q) == 256
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    qs = [0] * 128
    for e in range(256):
        c, r = e // 64, e % 64
        idx = 32 * c + (r % 32)
        if r < 32:
            qs[idx] |= q[e] & 15
        else:
            qs[idx] |= (q[e] & 15) << 4
    b = d_bits.to_bytes(2, "little") + dmin_bits.to_bytes(2, "little") + bytes(s) + bytes(qs)
    d, dmin = np.float32(f16val(d_bits)), np.float32(f16val(dmin_bits))
    exp = []
    for e in range(256):
        j = e // 32
        d1 = np.float32(d * np.float32(sc[j]))
        m1 = np.float32(dmin * np.float32(mn[j]))
        exp.append(float(np.float32(np.float32(d1 * np.float32(q[e])) - m1)))
    return b, exp


def q5_K_block(d_bits, dmin_bits, sc, mn, q):
    assert all(0 <= v < 32 for v in q)
    b4, exp = q4_K_block(d_bits, dmin_bits, sc, mn, q)
    # the 4-bit block holds d, dmin, scales, qs (low nibbles); splice qh in
    qh = [0] * 32
    for e in range(256):
        qh[e % 32] |= ((q[e] >> 4) & 1) << (e // 32)
    b = b4[:16] + bytes(qh) + b4[16:]
    assert len(b) == 176
    return b, exp


def q6_K_block(d_bits, sc, q):
    assert len(sc) == 16 and len(q) == 256
    ql = [0] * 128
    qh = [0] * 64
    for e in range(256):
        h, r = e // 128, e % 128
        t, l = r // 32, r % 32
        lo, hi = q[e] & 15, (q[e] >> 4) & 3
        idx = 64 * h + l + 32 * (t & 1)
        ql[idx] |= lo if t < 2 else lo << 4
        qh[32 * h + l] |= hi << (2 * t)
    b = bytes(ql) + bytes(qh) + np.array(sc, dtype=np.int8).tobytes() + d_bits.to_bytes(2, "little")
    d = np.float32(f16val(d_bits))
    exp = []
    for e in range(256):
        ds = np.float32(d * np.float32(sc[e // 16]))
        exp.append(float(np.float32(ds * np.float32(q[e] - 32))))
    return b, exp


def main():
    blocks = []
    # Q8_0: d = 1 with q spanning -127..127; d = 0.5; d = smallest f16 subnormal; d = 0
    q_span = [-127, -126, -100, -64, -33, -32, -17, -8, -2, -1, 0, 1, 2, 3, 7, 8,
              15, 16, 31, 32, 33, 63, 64, 65, 99, 100, 101, 120, 125, 126, 127, -128 + 1]
    for name, d_bits in [("q8_0_d1", f16bits(1.0)), ("q8_0_dhalf", f16bits(0.5)),
                         ("q8_0_dsub", 0x0001), ("q8_0_d0", 0x0000), ("q8_0_dneg", f16bits(-0.0123))]:
        b, e = q8_0_block(d_bits, q_span)
        blocks.append({"name": name, "type": 8, "ne0": 32, "hex": b.hex(), "expected": e})
    # Q4_K: exact small values first (d=1, dmin=0.5), exercising j<4 and j>=4 packing
    sc = [1, 2, 63, 17, 37, 48, 5, 63]
    mn = [0, 1, 5, 63, 2, 33, 60, 63]
    q = [(e * 7 + 3) % 16 for e in range(256)]
    b, e = q4_K_block(f16bits(1.0), f16bits(0.5), sc, mn, q)
    blocks.append({"name": "q4_K_exact", "type": 12, "ne0": 256, "hex": b.hex(), "expected": e})
    # Q4_K: generic f16 scales (two roundings matter), all-ones / all-max fields
    b, e = q4_K_block(f16bits(0.0123), f16bits(0.00771), [63] * 4 + [48, 16, 32, 1],
                      [0, 63, 31, 32, 63, 15, 16, 47], [15 - (e % 16) for e in range(256)])
    blocks.append({"name": "q4_K_f16", "type": 12, "ne0": 256, "hex": b.hex(), "expected": e})
    # Q5_K: the Q4_K fields with 5-bit quants (0..31), every qh bit position used
    q5 = [(e * 11 + 5) % 32 for e in range(256)]
    b, e = q5_K_block(f16bits(1.0), f16bits(0.5), sc, mn, q5)
    blocks.append({"name": "q5_K_exact", "type": 13, "ne0": 256, "hex": b.hex(), "expected": e})
    b, e = q5_K_block(f16bits(0.00417), f16bits(0.0213), [0, 63, 7, 40, 63, 1, 22, 9],
                      [63, 0, 12, 63, 5, 63, 31, 0], [31 - (e % 32) for e in range(256)])
    blocks.append({"name": "q5_K_f16", "type": 13, "ne0": 256, "hex": b.hex(), "expected": e})
    # Q6_K: d = 1, scales covering int8 extremes, quants 0..63 (values -32..31)
    sc6 = [-128, -64, -1, 0, 1, 2, 3, 7, 15, 31, 63, 64, 100, 126, 127, -100]
    q6 = [(e * 5 + 1) % 64 for e in range(256)]
    b, e = q6_K_block(f16bits(1.0), sc6, q6)
    blocks.append({"name": "q6_K_exact", "type": 14, "ne0": 256, "hex": b.hex(), "expected": e})
    b, e = q6_K_block(f16bits(0.000913), [(-1) ** i * (i * 9 % 128) for i in range(16)], [63 - (e % 64) for e in range(256)])
    blocks.append({"name": "q6_K_f16", "type": 14, "ne0": 256, "hex": b.hex(), "expected": e})
    OUT.write_text(json.dumps({"generator": "tests/golden/make_known_blocks.py", "blocks": blocks}, indent=1))
    print(f"wrote {OUT} ({len(blocks)} blocks)")


if __name__ == "__main__":
    main()
