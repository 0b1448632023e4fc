// Decode tables for the int8 MFMA decoders, derived at compile time from the compact codebooks.
//
// The kernels build each 8-lane sub-block as signed int8 with v_perm_b32: a per-format palette
// of signed values sits in two registers and every output byte is picked by a selector byte.
//   iq2_codes[i]  IQ2_XXS grid entry i as eight selector codes: 0 -> 8, 1 -> 25, 2 -> 43
//   sign_sel[s]   the 7-bit sign field s, parity bit added, as 0x04 in each negative lane; OR-ed
//                 into the codes it moves the pick to the negated half of the palette
//   iq3_pm[i]     IQ3_XXS grid entry i: low word the four magnitudes, high word their negations
//   iq3_sel[s]    selectors picking lane l from the low word (positive) or high word (negative)
//   iq1_codes[i]  IQ1_S grid entry i as eight selector codes: 0 -> q=0, 1 -> q=+1, 2 -> q=-1
// Sign fields and parity follow the reference decoders (ggml_quantization.cpp:262-270, :347-353).
#ifndef VL_TABLES_H
#define VL_TABLES_H

#include <stdint.h>

#include "iq_codebooks.h"

namespace vl {

struct DecodeTables {
    uint64_t iq2_codes[256];
    uint64_t sign_sel[128];
    uint64_t iq3_pm[256];
    uint64_t iq3_sel[128];
    uint64_t iq1_codes[2048];
};

constexpr unsigned parity_sign_byte(unsigned seven) {
    unsigned bits = 0;
    for (unsigned b = 0; b < 7; ++b) bits += (seven >> b) & 1u;
    return seven | ((bits & 1u) << 7);
}

constexpr DecodeTables make_decode_tables() {
    DecodeTables t{};
    constexpr uint16_t c2[256] = VL_IQ2XXS_CODES;
    constexpr uint16_t c3[256] = VL_IQ3XXS_CODES;
    constexpr uint16_t c1[2048] = VL_IQ1S_CODES;
    for (unsigned e = 0; e < 256; ++e) {
        uint64_t codes = 0;
        for (unsigned l = 0; l < 8; ++l) codes |= (uint64_t)((c2[e] >> (2 * l)) & 3u) << (8 * l);
        t.iq2_codes[e] = codes;
        uint64_t pos = 0, neg = 0;
        for (unsigned l = 0; l < 4; ++l) {
            const unsigned code = (c3[e] >> (3 * l)) & 7u;
            const unsigned m = 4u + 8u * code + (code == 7u ? 2u : 0u);
            pos |= (uint64_t)m << (8 * l);
            neg |= (uint64_t)((256u - m) & 0xffu) << (8 * l);
        }
        t.iq3_pm[e] = pos | (neg << 32);
    }
    for (unsigned s = 0; s < 128; ++s) {
        const unsigned sb = parity_sign_byte(s);
        uint64_t sel = 0, sel3 = 0;
        for (unsigned l = 0; l < 8; ++l) {
            const uint64_t neg = (sb >> l) & 1u;
            sel |= (neg * 4u) << (8 * l);
            sel3 |= ((l & 3u) + neg * 4u) << (8 * l);
        }
        t.sign_sel[s] = sel;
        t.iq3_sel[s] = sel3;
    }
    for (unsigned e = 0; e < 2048; ++e) {
        uint64_t codes = 0;
        for (unsigned l = 0; l < 8; ++l) codes |= (uint64_t)((c1[e] >> (2 * l)) & 3u) << (8 * l);
        t.iq1_codes[e] = codes;
    }
    return t;
}

// Palettes (low word = positive picks 0..3, high word = negated picks 4..7), as consumed by
// __builtin_amdgcn_perm(high, low, selector).
//   IQ2_XXS: magnitudes 8, 25, 43 and their negations.
constexpr uint32_t kIq2PalettePos = 0x002b1908u;
constexpr uint32_t kIq2PaletteNeg = 0x00d5e7f8u;
//   IQ1_S: 8*(q + delta) for q = 0, +1, -1; delta +1/8 in the low word, -1/8 in the high word.
constexpr uint32_t kIq1PalettePos = 0x00f90901u;  //  1,  9, -7
constexpr uint32_t kIq1PaletteNeg = 0x00f707ffu;  // -1,  7, -9

}  // namespace vl

#endif  // VL_TABLES_H
