"""Writes tests/golden/known_answers.json: known-answer vectors for the oracle, computed here in
plain Python / numpy, independently of the C oracle.

The reference commits no golden vectors (every test builds its inputs at run time from
``Rng`` in src/tensor.rs:155-199), and rie-core is not in this container, so the vectors are
restated from the definitions:

* SplitMix64 / Box-Muller streams (src/tensor.rs:163-186) in Python integers;
* hand-built GGUF blocks whose decoded values are exact in float32 (power-of-two scales, small
  integer codes), so the closed forms of the ggml formats give the expected floats exactly:
  Q4_0 (both nibbles), Q8_0, Q4_K (scale/min packing of sub-blocks 0-3 *and* 4-7), Q6_K (all
  four qh shifts, signed int8 scales);
* quantiser tie cases: Q8_0 rounds half away from zero (roundf), Q8_K rounds half to even and maps
  the signed largest element to -127;
* integer block sums by brute force.

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import math
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
M64 = (1 << 64) - 1


def splitmix(seed: int, n: int) -> list[int]:
    s = (seed ^ 0x9E3779B97F4A7C15) & M64
    out = []
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & M64
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        out.append(z ^ (z >> 31))
    return out


def uniform_from(u: int) -> float:
    return float(np.float32(u >> 40) / np.float32(1 << 24))


def f16bits(v: float) -> int:
    return int(np.array([v], dtype=np.float16).view(np.uint16)[0])


def hexb(b: bytes) -> str:
    return b.hex()


def q4_0_block(d: float, codes: list[int]) -> bytes:
    """codes[0..31] in [0, 15] -> 18-byte block; element j<16 low nibble of byte j, j+16 high."""
    qs = bytes((codes[j] & 0xF) | ((codes[j + 16] & 0xF) << 4) for j in range(16))
    return struct.pack("<H", f16bits(d)) + qs


def q8_0_block(d: float, codes: list[int]) -> bytes:
    return struct.pack("<H", f16bits(d)) + bytes((c & 0xFF) for c in codes)


def q4_k_block(d: float, dmin: float, sc: list[int], m: list[int], codes: list[int]) -> bytes:
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4)
    qs = bytearray(128)
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = (codes[64 * c + l] & 0xF) | ((codes[64 * c + 32 + l] & 0xF) << 4)
    return struct.pack("<HH", f16bits(d), f16bits(dmin)) + bytes(s) + bytes(qs)


def q4_k_values(d, dmin, sc, m, codes):
    return [d * sc[e // 32] * codes[e] - dmin * m[e // 32] for e in range(256)]


def q6_k_block(d: float, scales: list[int], codes: list[int]) -> bytes:
    """codes in [-32, 31]; element e uses scales[e // 16]."""
    L = [c + 32 for c in codes]
    ql = bytearray(128)
    qh = bytearray(64)
    for h in range(2):
        for l in range(32):
            q1, q2, q3, q4 = L[128 * h + l], L[128 * h + l + 32], L[128 * h + l + 64], L[128 * h + l + 96]
            ql[64 * h + l] = (q1 & 0xF) | ((q3 & 0xF) << 4)
            ql[64 * h + l + 32] = (q2 & 0xF) | ((q4 & 0xF) << 4)
            qh[32 * h + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    return bytes(ql) + bytes(qh) + bytes((s & 0xFF) for s in scales) + struct.pack("<H", f16bits(d))


def main() -> None:
    out: dict = {}
    # ---- Rng
    rng = {}
    for seed in (1, 2, 3, 9):
        us = splitmix(seed, 6)
        rng[str(seed)] = {"u64": [str(u) for u in us], "uniform": [uniform_from(u) for u in us]}
    out["rng"] = rng

    # ---- dequant known answers (values exact in f32)
    dq = []
    codes = [(7 * j + 3) % 16 for j in range(32)]
    dq.append({"type": 2, "k": 32, "blocks": hexb(q4_0_block(0.5, codes)), "values": [(c - 8) * 0.5 for c in codes]})
    codes = list(range(16)) + [15 - j for j in range(16)]
    dq.append({"type": 2, "k": 32, "blocks": hexb(q4_0_block(-0.125, codes)),
               "values": [(c - 8) * -0.125 for c in codes]})
    c8 = [((j * 37) % 255) - 127 for j in range(32)]
    dq.append({"type": 8, "k": 32, "blocks": hexb(q8_0_block(0.25, c8)), "values": [c * 0.25 for c in c8]})
    c8 = [-127, 127, 0, 1, -1] + [j - 13 for j in range(27)]
    dq.append({"type": 8, "k": 32, "blocks": hexb(q8_0_block(2.0 ** -10, c8)), "values": [c * 2.0 ** -10 for c in c8]})
    # Q4_K: sub-blocks 4..7 have sc, m >= 16 so the high bits live in bytes 0..7's top bits
    sc = [1, 7, 33, 63, 17, 48, 60, 31]
    m = [5, 0, 62, 9, 40, 19, 33, 63]
    c4 = [(11 * e + 5) % 16 for e in range(256)]
    dq.append({"type": 12, "k": 256, "blocks": hexb(q4_k_block(2.0 ** -6, 2.0 ** -8, sc, m, c4)),
               "values": q4_k_values(2.0 ** -6, 2.0 ** -8, sc, m, c4)})
    # Q6_K: codes exercise all 6 bits in every quarter (qh shifts 0, 2, 4, 6) and both halves
    s6 = [-128, 127, -1, 1, 64, -64, 3, -3, 100, -100, 7, 0, -17, 17, 42, -42]
    c6 = [((13 * e + 7) % 64) - 32 for e in range(256)]
    d6 = 2.0 ** -12
    dq.append({"type": 14, "k": 256, "blocks": hexb(q6_k_block(d6, s6, c6)),
               "values": [d6 * s6[e // 16] * c6[e] for e in range(256)]})
    out["dequant"] = dq

    # ---- quantiser known answers
    qa = []
    # Q8_0 (weights and activations): amax 127 -> d = 1, id = 1; ties round away from zero
    x = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5] + [float(j) - 12.0 for j in range(24)]
    q = [int(math.copysign(math.floor(abs(v) + 0.5), v)) for v in x]
    qa.append({"kind": "q8_0", "x": x, "d_bits": f16bits(1.0), "q": q})
    # Q8_0 zero block: d = 0 and codes 0
    qa.append({"kind": "q8_0", "x": [0.0] * 32, "d_bits": 0, "q": [0] * 32})
    # Q8_K: largest |x| is +127 -> iscale = -1, q = -x rounded half to even, d = -1
    x = [127.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 1.5] + [float((j * 5) % 31) - 15.0 for j in range(248)]
    qk = []
    for v in x:
        r = -v
        f = math.floor(r)
        rr = f + 1 if (r - f > 0.5 or (r - f == 0.5 and f % 2 != 0)) else f
        qk.append(int(min(127, rr)))
    bs = [sum(qk[16 * g:16 * g + 16]) for g in range(16)]
    qa.append({"kind": "q8_k", "x": x, "d": -1.0, "q": qk, "bsums": bs})
    # Q4_0 weight quantiser: max = -8 (signed largest) -> d = 1, id = 1, q = min(15, trunc(x + 8.5))
    x = [-8.0, 7.0, 7.4, 7.6, -7.5, 0.49, 0.5, -0.51] + [float(j % 15) - 7.0 for j in range(24)]
    xs = np.array(x, np.float32)
    q4 = [min(15, int(np.float32(v) * np.float32(1.0) + np.float32(8.5))) for v in xs]
    qa.append({"kind": "q4_0", "x": x, "d_bits": f16bits(1.0), "q": q4})
    out["quantise"] = qa

    # ---- integer block dot brute force (Q4_0 x Q8_0), small random codes
    r = np.random.default_rng(7)
    w_codes = r.integers(0, 16, 32).tolist()
    a_codes = r.integers(-127, 128, 32).tolist()
    out["isum_q4_0"] = {"w": hexb(q4_0_block(1.0, w_codes)), "a": hexb(q8_0_block(1.0, a_codes)),
                        "isum": int(sum((w - 8) * a for w, a in zip(w_codes, a_codes)))}
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", os.path.join(HERE, "known_answers.json"))


if __name__ == "__main__":
    main()
