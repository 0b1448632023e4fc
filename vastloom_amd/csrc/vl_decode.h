// Device-side decoders: one lane's share of one 32-column group of one matrix row, produced as
// sixteen signed int8 weights (the lane's 32x32x32 int8 MFMA B fragment) plus the group's
// integer scale. With the superblock factor applied in float, each weight equals the
// reference's decoded float exactly:
//   IQ2_XXS  w = d/8 * (2s+1) * m * sign,     m in {8, 25, 43}        (ggml_quantization.cpp:250-283)
//   IQ3_XXS  w = d/4 * (2s+1) * m * sign,     m in {4, ..., 62}       (:336-379)
//   IQ1_S    w = d/8 * (2s+1) * (8q +- 1),    q in {-1, 0, 1}         (:217-248)
//   Q8_0     w = d * q,                        q int8                  (:419-433)
// In each case the reference's float operations round nothing: d is an fp16 value (11
// significant bits), the integer factor has at most 11 bits, and a power-of-two factor is
// exact, so the product fits in float's 24-bit significand.
//
// Lane layout: lane (n, hh) with n = lane % 32 the row within the tile and hh = lane / 32 the
// K half; it decodes sub-blocks 2hh and 2hh+1, i.e. columns 16hh .. 16hh+15 of the group, in
// column order (bytes 0..7 the first sub-block, 8..15 the second).
#ifndef VL_DECODE_H
#define VL_DECODE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vl_tables.h"

namespace vl {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

struct IqTables2 { uint64_t codes[256]; uint64_t sign[128]; };
struct IqTables3 { uint64_t pm[256]; uint64_t sel[128]; };
struct IqTables1 { uint64_t codes[2048]; };

__device__ __forceinline__ uint32_t lo32(uint64_t v) { return (uint32_t)v; }
__device__ __forceinline__ uint32_t hi32(uint64_t v) { return (uint32_t)(v >> 32); }

__device__ __forceinline__ uint32_t perm(uint32_t high, uint32_t low, uint32_t sel) {
    return __builtin_amdgcn_perm(high, low, sel);
}

// IQ2_XXS group: qs = four grid indices (one byte per sub-block), aux = four 7-bit sign fields
// and the 4-bit scale in the top nibble.
__device__ __forceinline__ i32x4 decode_iq2_xxs(uint32_t qs, uint32_t aux, int hh,
                                                const IqTables2& t) {
    const uint32_t q = qs >> (16 * hh);
    const uint32_t a = aux >> (14 * hh);
    const uint64_t s0 = t.codes[q & 0xffu] | t.sign[a & 0x7fu];
    const uint64_t s1 = t.codes[(q >> 8) & 0xffu] | t.sign[(a >> 7) & 0x7fu];
    i32x4 w;
    w[0] = (int)perm(kIq2PaletteNeg, kIq2PalettePos, lo32(s0));
    w[1] = (int)perm(kIq2PaletteNeg, kIq2PalettePos, hi32(s0));
    w[2] = (int)perm(kIq2PaletteNeg, kIq2PalettePos, lo32(s1));
    w[3] = (int)perm(kIq2PaletteNeg, kIq2PalettePos, hi32(s1));
    return w;
}

// IQ3_XXS group: qs8 = eight grid indices (two per sub-block, four lanes each), aux as IQ2_XXS.
__device__ __forceinline__ i32x4 decode_iq3_xxs(uint64_t qs8, uint32_t aux, int hh,
                                                const IqTables3& t) {
    const uint32_t q = (uint32_t)(qs8 >> (32 * hh));
    const uint32_t a = aux >> (14 * hh);
    const uint64_t sel0 = t.sel[a & 0x7fu];
    const uint64_t sel1 = t.sel[(a >> 7) & 0x7fu];
    const uint64_t g00 = t.pm[q & 0xffu], g01 = t.pm[(q >> 8) & 0xffu];
    const uint64_t g10 = t.pm[(q >> 16) & 0xffu], g11 = t.pm[q >> 24];
    i32x4 w;
    w[0] = (int)perm(hi32(g00), lo32(g00), lo32(sel0));
    w[1] = (int)perm(hi32(g01), lo32(g01), hi32(sel0));
    w[2] = (int)perm(hi32(g10), lo32(g10), lo32(sel1));
    w[3] = (int)perm(hi32(g11), lo32(g11), hi32(sel1));
    return w;
}

// IQ1_S group: qs4 = low 8 bits of the four 11-bit grid indices, qh = the group's 16-bit word
// (3 high index bits per sub-block, 3-bit scale at bit 12, delta sign at bit 15).
__device__ __forceinline__ i32x4 decode_iq1_s(uint32_t qs4, uint32_t qh, int hh,
                                              const IqTables1& t) {
    const int s0 = 2 * hh;
    const uint32_t i0 = ((qs4 >> (8 * s0)) & 0xffu) | (((qh >> (3 * s0)) & 7u) << 8);
    const uint32_t i1 = ((qs4 >> (8 * s0 + 8)) & 0xffu) | (((qh >> (3 * s0 + 3)) & 7u) << 8);
    const uint64_t dm = (qh & 0x8000u) ? 0x0404040404040404ull : 0ull;
    const uint64_t c0 = t.codes[i0] | dm;
    const uint64_t c1 = t.codes[i1] | dm;
    i32x4 w;
    w[0] = (int)perm(kIq1PaletteNeg, kIq1PalettePos, lo32(c0));
    w[1] = (int)perm(kIq1PaletteNeg, kIq1PalettePos, hi32(c0));
    w[2] = (int)perm(kIq1PaletteNeg, kIq1PalettePos, lo32(c1));
    w[3] = (int)perm(kIq1PaletteNeg, kIq1PalettePos, hi32(c1));
    return w;
}

// Exact binary16 -> binary32 (v_cvt_f32_f16; fp16 denormals are preserved on gfx9).
__device__ __forceinline__ float half_bits_to_float(uint16_t bits) {
    _Float16 h;
    __builtin_memcpy(&h, &bits, sizeof h);
    return (float)h;
}

}  // namespace vl

#endif  // VL_DECODE_H
