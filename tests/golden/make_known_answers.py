"""Writes tests/golden/dequant_known_answers.json (run: python tests/golden/make_known_answers.py).

Known-answer GGUF blocks with expected fp32 outputs, as data:

1. The reference's own known answers (tests/test_dequant.py of Labeeb2339/pico-engine):
   q8_0_known_values (:21-27), q5_0_nibble_and_highbit (:30-41), q4_k_zero_nibbles_with_scale
   (:44-53), q6_k_zero_with_scale (:56-65). Where the reference asserts only some elements,
   the others are the values its comments state (untouched Q5_0 codes give -16; Q4_K
   sub-blocks 4..7 of that block have scale 1, min 0 and zero nibbles, so 0).
2. Hand-derived blocks for what those leave open -- Q4_K sub-blocks j >= 4 (6-bit scale/min
   split across bytes), Q6_K with non-zero qh and negative scales, Q8_0 with a negative scale,
   fp16-subnormal scales. The expected values come from per-element tables worked out by
   hand in the comments below (not from any dequantizer), so a wrong shift, index or sign in
   a restatement fails them.
"""

from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np


def f16(x: float) -> bytes:
    return struct.pack("<H", int(np.float16(x).view(np.uint16)))


def case(name, ggml_type, block: bytes, expected) -> dict:
    return {"name": name, "type": ggml_type, "n": len(expected), "block_hex": block.hex(),
            "expected": [float(v) for v in expected]}


def main() -> None:
    cases = []

    # -- reference known answers ----------------------------------------------------------
    qs = (np.arange(32) - 16).astype(np.int8)
    cases.append(case("ref_q8_0_known_values", 8, f16(0.5) + qs.tobytes(), qs.astype(np.float32) * 0.5))

    qh = 1 << 31
    q5 = np.zeros(16, np.uint8)
    q5[0] = 0x53
    exp = np.full(32, -16.0)
    exp[0], exp[16], exp[31] = -13.0, -11.0, 0.0
    cases.append(case("ref_q5_0_nibble_and_highbit", 6, f16(1.0) + struct.pack("<I", qh) + q5.tobytes(), exp))

    blk = f16(1.0) + f16(0.5) + bytes([0x01] * 12) + bytes(128)
    exp = np.concatenate([np.full(128, -0.5), np.zeros(128)])
    cases.append(case("ref_q4_k_zero_nibbles_with_scale", 12, blk, exp))

    blk = bytes(128) + bytes(64) + bytes([1] * 16) + f16(0.5)
    cases.append(case("ref_q6_k_zero_with_scale", 14, blk, np.full(256, -16.0)))

    # -- hand-derived ---------------------------------------------------------------------
    # Q8_0, negative scale d = -0.25, qs = 127, -128, 1, -1, 0, ... -> w = qs * d
    q = np.zeros(32, np.int8)
    q[:4] = [127, -128, 1, -1]
    cases.append(case("q8_0_negative_scale", 8, f16(-0.25) + q.tobytes(),
                      [-31.75, 32.0, -0.25, 0.25] + [0.0] * 28))

    # Q8_0 with an fp16-subnormal scale: bits 0x0003 = 3 * 2^-24; qs = 2 -> 6 * 2^-24
    q = np.full(32, 2, np.int8)
    cases.append(case("q8_0_subnormal_scale", 8, struct.pack("<H", 0x0003) + q.tobytes(),
                      [6 * 2.0 ** -24] * 32))

    # Q5_0: d = 2.0, qh = 0xFFFF0000 (5th bit set for elements 16..31),
    # qs[j] = j | (15 - j) << 4  ->  element j (<16): code j, w = (j - 16) * 2
    #                               element 16+j:   code (15 - j) | 16, w = (15 - j) * 2
    q5 = np.array([j | ((15 - j) << 4) for j in range(16)], np.uint8)
    exp = [(j - 16) * 2.0 for j in range(16)] + [(15 - j) * 2.0 for j in range(16)]
    cases.append(case("q5_0_ramp_highbits", 6, f16(2.0) + struct.pack("<I", 0xFFFF0000) + q5.tobytes(), exp))

    # Q4_K with all eight sub-block scales/mins distinct.  scales bytes:
    s = [0x41, 0x82, 0xC3, 0x04, 0x45, 0x86, 0xC7, 0x08, 0x21, 0x43, 0x65, 0x87]
    # worked by hand:
    #   j<4 : sc = s[j] & 63          -> 1, 2, 3, 4 ;   m = s[j+4] & 63 -> 5, 6, 7, 8
    #   j=4 : sc = (0x21&15)=1 | (0x41>>6=1)<<4 = 17 ;  m = (0x21>>4)=2 | (0x45>>6=1)<<4 = 18
    #   j=5 : sc = 3 | (0x82>>6=2)<<4 = 35            ;  m = 4 | (0x86>>6=2)<<4 = 36
    #   j=6 : sc = 5 | (0xC3>>6=3)<<4 = 53            ;  m = 6 | (0xC7>>6=3)<<4 = 54
    #   j=7 : sc = 7 | (0x04>>6=0)<<4 = 7             ;  m = 8 | (0x08>>6=0)<<4 = 8
    sc = [1, 2, 3, 4, 17, 35, 53, 7]
    mn = [5, 6, 7, 8, 18, 36, 54, 8]
    d, dmin = 0.25, 0.125
    # qs chunk c, byte i: low nibble = i % 16 (sub-block 2c), high nibble = 15 - i % 16 (2c+1)
    qsb = bytes([(i % 16) | ((15 - i % 16) << 4) for i in range(32)] * 4)
    exp = []
    for j in range(8):
        for i in range(32):
            nib = (i % 16) if j % 2 == 0 else (15 - i % 16)
            exp.append(d * sc[j] * nib - dmin * mn[j])
    cases.append(case("q4_k_all_subblocks", 12, f16(d) + f16(dmin) + bytes(s) + qsb, exp))

    # Q4_K with fp16-subnormal d and dmin (bits 0x0001 = 2^-24, 0x0002 = 2^-23), scales as above
    exp = []
    for j in range(8):
        for i in range(32):
            nib = (i % 16) if j % 2 == 0 else (15 - i % 16)
            exp.append(2.0 ** -24 * sc[j] * nib - 2.0 ** -23 * mn[j])
    cases.append(case("q4_k_subnormal_scales", 12,
                      struct.pack("<HH", 0x0001, 0x0002) + bytes(s) + qsb, exp))

    # Q6_K: d = 0.5, scales 1, -2, 3, -4, ... (sign alternates), 6-bit code of element e set to
    # e % 64 by ggml's packing: for half h and l < 32, codes c0..c3 of elements 128h + l + 32q:
    #   ql[64h + l] = c0 & 15 | (c2 & 15) << 4 ; ql[64h + 32 + l] = c1 & 15 | (c3 & 15) << 4
    #   qh[32h + l] = c0 >> 4 | (c1 >> 4) << 2 | (c2 >> 4) << 4 | (c3 >> 4) << 6
    # so element e is (e % 64 - 32) * 0.5 * scale[e // 16].
    code = [e % 64 for e in range(256)]
    ql = bytearray(128)
    qhb = bytearray(64)
    for h in range(2):
        for l in range(32):
            c0, c1, c2, c3 = (code[128 * h + l + 32 * q] for q in range(4))
            ql[64 * h + l] = (c0 & 15) | ((c2 & 15) << 4)
            ql[64 * h + 32 + l] = (c1 & 15) | ((c3 & 15) << 4)
            qhb[32 * h + l] = (c0 >> 4) | ((c1 >> 4) << 2) | ((c2 >> 4) << 4) | ((c3 >> 4) << 6)
    scales = [(i + 1) * (1 if i % 2 == 0 else -1) for i in range(16)]
    exp = [(code[e] - 32) * 0.5 * scales[e // 16] for e in range(256)]
    cases.append(case("q6_k_ramp_signed_scales", 14,
                      bytes(ql) + bytes(qhb) + np.array(scales, np.int8).tobytes() + f16(0.5), exp))

    out = {"doc": __doc__.strip().splitlines()[0], "cases": cases,
           "nbytes_for": [[8, 32, 34], [6, 32, 22], [12, 256, 144], [14, 256, 210],
                          [8, 896 * 4864, 4630528], [12, 4864 * 896, 2451456],
                          [14, 4864 * 896, 3575040], [6, 896 * 896, 551936]]}
    path = Path(__file__).with_name("dequant_known_answers.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path} ({len(cases)} cases)")


if __name__ == "__main__":
    main()
