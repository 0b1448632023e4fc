"""Known-answer blocks and expected values from the reference's own unit tests.

The byte patterns, scales, inputs and expected outputs below are the reference's test data
(tests/test_main.cpp:863-973 for Q8_0, :975-1054 Q4_K and Q5_K, :1056-1089 Q6_K, :1091-1112
BF16, :1295-1365 IQ1_S, :1367-1460 IQ2_XXS, :1663-1723 the Q4_K and MXFP4 blocks the reference
checked against ggml's own dequantize_row_q4_K / dequantize_row_mxfp4, :1725-1790 IQ2_S,
:1832-1907 IQ3_XXS),
regenerated here from the same formulas so that the oracle and the HIP decoders can be held to
the reference's pinned fingerprints and values.

Each entry: the storage type, its block size, the encoded blocks, the FNV-1a fingerprint of the
decoded floats (None where the reference pins the values only), exact and approximate sample
values, the matvec shape (rows, cols), input and expected outputs with tolerances, and the
bytes that make block 4 (element 4 for BF16) fail validation.
"""

from __future__ import annotations

import numpy as np

SCALES = (0x3C00, 0xB800, 0x3555, 0x4000, 0x0400, 0x0001)
MINIMUMS = (0x3800, 0xBC00, 0x3000, 0x3C00, 0x0001, 0x0400)


def fnv_f32(values: np.ndarray) -> int:
    """FNV-1a over the little-endian bytes of float32 values (test_main.cpp:878-888)."""
    h = 14695981039346656037
    for b in np.ascontiguousarray(values, np.float32).tobytes():
        h ^= b
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def kat_input(columns: int) -> np.ndarray:
    """(c % 29 - 14) * 0.03125 + (c % 3) * 0.0078125, in float (test_main.cpp:889-897)."""
    c = np.arange(columns)
    return (((c % 29) - 14).astype(np.float32) * np.float32(0.03125)
            + (c % 3).astype(np.float32) * np.float32(0.0078125)).astype(np.float32)


def q8_0_blocks() -> np.ndarray:
    out = np.zeros((len(SCALES), 34), np.uint8)
    for b, s in enumerate(SCALES):
        out[b, 0], out[b, 1] = s & 0xFF, s >> 8
        out[b, 2:] = [(b * 37 + i * 53 + 11) & 0xFF for i in range(32)]
    return out.reshape(-1)


def iq1_s_blocks() -> np.ndarray:
    out = np.zeros((len(SCALES), 50), np.uint8)
    for b, s in enumerate(SCALES):
        out[b, 0], out[b, 1] = s & 0xFF, s >> 8
        out[b, 2:34] = [(b * 37 + i * 53 + 11) & 0xFF for i in range(32)]
        for g in range(8):
            high = ((((g * 5 + b) & 7) << 12) | (0x8000 if ((g + b) & 1) else 0)
                    | ((b * 733 + g * 97 + 0x123) & 0x0FFF))
            out[b, 34 + 2 * g], out[b, 35 + 2 * g] = high & 0xFF, high >> 8
    return out.reshape(-1)


def iq2_xxs_blocks() -> np.ndarray:
    out = np.zeros((len(SCALES), 66), np.uint8)
    for b, s in enumerate(SCALES):
        out[b, 0], out[b, 1] = s & 0xFF, s >> 8
        for i in range(32):
            packed = (b * 733 + i * 977 + 0x1234) & 0xFFFF
            out[b, 2 + 2 * i], out[b, 3 + 2 * i] = packed & 0xFF, packed >> 8
    return out.reshape(-1)


def iq3_xxs_blocks() -> np.ndarray:
    out = np.zeros((len(SCALES), 98), np.uint8)
    for b, s in enumerate(SCALES):
        out[b, 0], out[b, 1] = s & 0xFF, s >> 8
        out[b, 2:66] = [(b * 37 + i * 53 + 11) & 0xFF for i in range(64)]
        for g in range(8):
            aux = ((b * 3 + g * 5) & 15) << 28
            for sb in range(4):
                aux |= ((b * 19 + g * 13 + sb * 23 + 7) & 127) << (7 * sb)
            out[b, 66 + 4 * g:70 + 4 * g] = [(aux >> (8 * k)) & 0xFF for k in range(4)]
    return out.reshape(-1)


def _k_head(out: np.ndarray, b: int, scale: int, minimum: int) -> None:
    out[b, 0], out[b, 1] = scale & 0xFF, scale >> 8
    out[b, 2], out[b, 3] = minimum & 0xFF, minimum >> 8


def q4_k_blocks() -> np.ndarray:
    out = np.zeros((len(SCALES), 144), np.uint8)
    for b in range(len(SCALES)):
        _k_head(out, b, SCALES[b], MINIMUMS[b])
        out[b, 4:16] = [(b * 29 + i * 47 + 7) & 0xFF for i in range(12)]
        out[b, 16:] = [(b * 37 + i * 53 + 11) & 0xFF for i in range(128)]
    return out.reshape(-1)


def q5_k_blocks() -> np.ndarray:
    out = np.zeros((len(SCALES), 176), np.uint8)
    for b in range(len(SCALES)):
        _k_head(out, b, SCALES[b], MINIMUMS[b])
        out[b, 4:16] = [(b * 29 + i * 47 + 7) & 0xFF for i in range(12)]
        out[b, 16:48] = [(b * 41 + i * 31 + 13) & 0xFF for i in range(32)]
        out[b, 48:] = [(b * 37 + i * 53 + 11) & 0xFF for i in range(128)]
    return out.reshape(-1)


def q6_k_blocks() -> np.ndarray:
    out = np.zeros((len(SCALES), 210), np.uint8)
    for b, s in enumerate(SCALES):
        out[b, :128] = [(b * 37 + i * 53 + 11) & 0xFF for i in range(128)]
        out[b, 128:192] = [(b * 41 + i * 31 + 13) & 0xFF for i in range(64)]
        out[b, 192:208] = [(b * 59 + i * 43 + 17) & 0xFF for i in range(16)]
        out[b, 208], out[b, 209] = s & 0xFF, s >> 8
    return out.reshape(-1)


def q4_k_ggml_blocks() -> np.ndarray:
    minimums = (0x3800, 0x3555, 0xBC00, 0x0001, 0x4200, 0x0400)
    out = np.zeros((len(SCALES), 144), np.uint8)
    for b in range(len(SCALES)):
        _k_head(out, b, SCALES[b], minimums[b])
        out[b, 4:16] = [(b * 37 + i * 53 + 0x2B) & 0xFF for i in range(12)]
        out[b, 16:] = [(b * 733 + i * 977 + 0x1234) & 0xFF for i in range(128)]
    return out.reshape(-1)


def mxfp4_ggml_blocks() -> np.ndarray:
    out = np.zeros((len(SCALES), 17), np.uint8)
    for b in range(len(SCALES)):
        out[b, 0] = 120 + 3 * b
        out[b, 1:] = [(b * 91 + i * 167 + 0x5A) & 0xFF for i in range(16)]
    return out.reshape(-1)


def iq2_s_blocks() -> np.ndarray:
    out = np.zeros((len(SCALES), 82), np.uint8)
    for b, s in enumerate(SCALES):
        out[b, 0], out[b, 1] = s & 0xFF, s >> 8
        out[b, 2:34] = [(b * 733 + i * 977 + 0x1234) & 0xFF for i in range(32)]
        out[b, 34:66] = [(b * 251 + i * 131 + 0x5AA5) & 0xFF for i in range(32)]
        out[b, 66:74] = [(b * 97 + i * 43 + 0x3C) & 0xFF for i in range(8)]
        out[b, 74:82] = [(b * 61 + i * 29 + 0x17) & 0xFF for i in range(8)]
    return out.reshape(-1)


def bf16_values() -> np.ndarray:
    return np.array([0x3F80, 0xC000, 0x3F00, 0x4080, 0xBF80, 0x4040, 0xBE80, 0x4000],
                    np.uint16).view(np.uint8)


# Expected decoded fingerprints, sample values and 3-row matvec outputs with their tolerances.
KAT = {
    "q8_0": dict(
        qtype=8, block_elements=32, blocks=q8_0_blocks, fnv=0x25EDD1A40129EE99,
        values={0: 11.0, 7: 126.0, 8: -77.0, 31: 118.0, 32: -24.0, 63: 50.5, 127: -54.0},
        cols=64, outputs=[(-168.55859375, 0.0), (-2.8284435272216797, 0.0),
                          (0.0058367089368402958, 0.0)]),
    "iq1_s": dict(
        qtype=19, block_elements=256, blocks=iq1_s_blocks, fnv=0x9B66DE452B7F3C8D,
        values={0: 0.125, 7: 0.125, 8: -0.875, 31: -0.875, 32: 9.625, 255: -7.875,
                256: 1.6875, 511: -0.5625},
        cols=512, outputs=[(-4.8994140625, 0.0), (22.142812728881836, 1e-6),
                           (-0.0021024104207754135, 1e-9)]),
    "iq2_xxs": dict(
        qtype=16, block_elements=256, blocks=iq2_xxs_blocks, fnv=0x9BCA8E03F48DAFE9,
        values={0: 9.375, 7: 3.0, 8: -16.125, 31: -3.0, 32: 5.0, 63: -5.0, 127: -9.0,
                255: 17.0, 256: 2.5, 511: 8.5},
        cols=512, outputs=[(-32.86767578125, 0.0), (-284.89828491210938, 0.0),
                           (-0.011499286629259586, 1e-9)]),
    "iq3_xxs": dict(
        qtype=18, block_elements=256, blocks=iq3_xxs_blocks, fnv=0xF36989DCC58B1664,
        values={0: -11.0, 7: -3.0, 8: 5.0, 31: -5.0, 32: 170.5, 255: 7.0, 256: -54.25,
                511: -19.5},
        cols=512, outputs=[(-347.998046875, 0.0), (2887.319580078125, 1e-4),
                           (0.064146831631660461, 1e-8)]),
    "q4_k": dict(
        qtype=12, block_elements=256, blocks=q4_k_blocks, fnv=0x84E8E84336EA0AD7,
        values={0: 75.5, 7: 96.5, 8: 19.5, 31: 40.5, 32: -25.0, 63: 353.0, 127: 12.0,
                255: 212.0, 256: 32.0, 511: -125.5},
        cols=512, outputs=[(281.6796875, 0.0), (-792.12872314453125, 0.0),
                           (0.0096547976136207581, 0.0)],
        poison={2: 0x00, 3: 0x7C}),  # dmin = +inf
    "q5_k": dict(
        qtype=13, block_elements=256, blocks=q5_k_blocks, fnv=0x3EC4A59589931118,
        values={0: 187.5, 7: 96.5, 8: 131.5, 31: 40.5, 32: -25.0, 63: 1217.0, 127: 332.0,
                255: 916.0, 256: 32.0, 511: -453.5},
        cols=512, outputs=[(668.2421875, 0.0), (1631.9100341796875, 0.0),
                           (-0.046117834746837616, 0.0)]),
    "q6_k": dict(
        qtype=14, block_elements=256, blocks=q6_k_blocks, fnv=0xCD39C3F1219AFBC9,
        values={0: -85.0, 7: 238.0, 8: -221.0, 31: 360.0, 32: 2781.0, 63: -2420.0, 127: 1054.0,
                255: -530.0, 511: 540.5},
        cols=512, outputs=[(-4684.79296875, 0.0), (7494.287109375, 0.0),
                           (0.5950310230255127, 0.0)],
        poison={208: 0x00, 209: 0x7C}),
    "q4_k_ggml": dict(
        qtype=12, block_elements=256, blocks=q4_k_ggml_blocks, fnv=0x4A61F0F8094737CC,
        values={0: 140.5, 1: 183.5, 31: 97.5, 32: 70.0, 127: 85.0, 255: 680.5},
        approx={256: (-19.9970703, 1e-4), 511: (-348.995361, 1e-3), 1024: (-56.9692383, 1e-4)},
        cols=512, outputs=[]),
    "mxfp4_ggml": dict(
        qtype=39, block_elements=32, blocks=mxfp4_ggml_blocks, fnv=0xCE2B9AA19EF0E448,
        values={0: -0.0078125, 1: 0.00390625, 2: 0.0, 3: -0.046875, 4: 0.03125},
        cols=64, outputs=[],
        poison={0: 0xFF, 1: 0x77}),  # scale 2^127 times a code of 12
    "iq2_s": dict(
        qtype=22, block_elements=256, blocks=iq2_s_blocks, fnv=0x785968D455DE0695,
        values={0: -15.0, 7: -15.0, 8: 15.0, 31: 3.0, 32: -9.0, 63: 21.875, 127: 40.625,
                255: -29.0, 256: -4.5, 511: -8.0625},
        cols=512, outputs=[(209.540527, 0.0), (274.050537, 0.0), (0.0192997903, 1e-9)]),
    "bf16": dict(
        qtype=30, block_elements=1, blocks=bf16_values, fnv=None, count=8,
        values={0: 1.0, 1: -2.0, 2: 0.5, 3: 4.0, 4: -1.0, 5: 3.0, 6: -0.25, 7: 2.0},
        rows=2, cols=4, x=np.array([0.25, -0.5, 2.0, 1.0], np.float32),
        outputs=[(6.25, 0.0), (-0.25, 0.0)],
        poison={0: 0x80, 1: 0x7F}),  # +inf
}


def kat_count(k: dict) -> int:
    """Decoded elements of an entry's blocks."""
    return k.get("count", 6 * k["block_elements"])


def kat_rows(k: dict) -> int:
    return k.get("rows", 3)


def kat_x(k: dict) -> np.ndarray:
    return k["x"] if "x" in k else kat_input(k["cols"])


def kat_poisoned(k: dict) -> np.ndarray:
    """The entry's blocks with block 4 made invalid (a non-finite scale or value)."""
    enc = k["blocks"]().copy()
    block_bytes = enc.size // (kat_count(k) // k["block_elements"])
    for off, v in k.get("poison", {0: 0x00, 1: 0x7C}).items():
        enc[4 * block_bytes + off] = v
    return enc
