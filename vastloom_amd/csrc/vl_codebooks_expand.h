/* Expansion of the compact IQ codebooks into the byte-lane tables a decoder indexes.
 *
 * Each expanded entry is bit-identical to the corresponding ggml grid entry: lane i of an
 * entry occupies bits 8i..8i+7, exactly as the reference's tables are laid out
 * (src/inference/ggml_quantization.cpp:28-42). vl_codebooks_fingerprints_ok() recomputes the
 * reference's FNV-1a fingerprints over the expanded tables (ggml_quantization.cpp:49-99), so a
 * caller can refuse to run with a corrupted codebook. Plain C99, header only.
 */
#ifndef VL_CODEBOOKS_EXPAND_H
#define VL_CODEBOOKS_EXPAND_H

#include <stdint.h>

#include "iq_codebooks.h"

typedef struct vl_expanded_codebooks {
    uint64_t iq2xxs[256];  /* eight unsigned magnitudes in {8, 25, 43} */
    uint32_t iq3xxs[256];  /* four unsigned magnitudes in {4, ..., 62} */
    uint64_t iq1s[2048];   /* eight int8 lanes in {-1, 0, +1} */
    uint64_t iq2s[1024];   /* eight unsigned magnitudes in {8, 25, 43} */
} vl_expanded_codebooks;

static inline uint64_t vl_fnv1a_lanes(const void* table, unsigned entries, unsigned lane_bytes) {
    uint64_t hash = 14695981039346656037ULL;
    for (unsigned e = 0; e < entries; ++e) {
        uint64_t v = lane_bytes == 8 ? ((const uint64_t*)table)[e] : ((const uint32_t*)table)[e];
        for (unsigned b = 0; b < lane_bytes; ++b) {
            hash ^= (uint8_t)(v >> (8u * b));
            hash *= 1099511628211ULL;
        }
    }
    return hash;
}

static inline void vl_codebooks_expand(vl_expanded_codebooks* out) {
    static const uint16_t c2[256] = VL_IQ2XXS_CODES;
    static const uint16_t c3[256] = VL_IQ3XXS_CODES;
    static const uint16_t c1[2048] = VL_IQ1S_CODES;
    static const uint16_t c2s[1024] = VL_IQ2S_CODES;
    static const uint8_t v2[4] = {8, 25, 43, 0};
    static const uint8_t v1[4] = {0x00, 0x01, 0xff, 0x00};
    for (unsigned e = 0; e < 256; ++e) {
        uint64_t g = 0;
        for (unsigned l = 0; l < 8; ++l) g |= (uint64_t)v2[(c2[e] >> (2u * l)) & 3u] << (8u * l);
        out->iq2xxs[e] = g;
        uint32_t h = 0;
        for (unsigned l = 0; l < 4; ++l) {
            unsigned code = (c3[e] >> (3u * l)) & 7u;
            h |= (uint32_t)(4u + 8u * code + (code == 7u ? 2u : 0u)) << (8u * l);
        }
        out->iq3xxs[e] = h;
    }
    for (unsigned e = 0; e < 2048; ++e) {
        uint64_t g = 0;
        for (unsigned l = 0; l < 8; ++l) g |= (uint64_t)v1[(c1[e] >> (2u * l)) & 3u] << (8u * l);
        out->iq1s[e] = g;
    }
    for (unsigned e = 0; e < 1024; ++e) {
        uint64_t g = 0;
        for (unsigned l = 0; l < 8; ++l) g |= (uint64_t)v2[(c2s[e] >> (2u * l)) & 3u] << (8u * l);
        out->iq2s[e] = g;
    }
}

static inline int vl_codebooks_fingerprints_ok(const vl_expanded_codebooks* t) {
    return vl_fnv1a_lanes(t->iq2xxs, 256, 8) == VL_IQ2XXS_GRID_FNV &&
           vl_fnv1a_lanes(t->iq3xxs, 256, 4) == VL_IQ3XXS_GRID_FNV &&
           vl_fnv1a_lanes(t->iq1s, 2048, 8) == VL_IQ1S_GRID_FNV &&
           vl_fnv1a_lanes(t->iq2s, 1024, 8) == VL_IQ2S_GRID_FNV;
}

#endif /* VL_CODEBOOKS_EXPAND_H */
