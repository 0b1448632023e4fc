"""Known-answer blocks and expected values from the reference's own unit tests.

The byte patterns, scales, inputs and expected outputs below are the reference's test data
(tests/test_main.cpp:863-973 for Q8_0, :1295-1365 IQ1_S, :1367-1460 IQ2_XXS, :1832-1907
IQ3_XXS), regenerated here from the same formulas so that the oracle and the HIP decoders can
be held to the reference's pinned fingerprints and values.
"""

from __future__ import annotations

import numpy as np

SCALES = (0x3C00, 0xB800, 0x3555, 0x4000, 0x0400, 0x0001)


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
}
