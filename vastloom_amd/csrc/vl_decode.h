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
//
// Decode tables live in LDS. The 256- and 128-entry tables of IQ2_XXS and IQ3_XXS are held in
// 16 copies, and lane l reads copy l % 16: the 16 lanes an LDS cycle serves for a b64 read then
// touch 16 different bank pairs whatever entries they look up, which removes the bank conflicts
// of random lookups (MI355X measures the same with 32 copies, and slower with 8). The two tables
// share 256-byte rows: grid entry e, copy c at byte e * 256 + c * 8 (the row's lower half) and
// sign entry e at e * 256 + 128 + c * 8 (the upper half of rows 0..127), 64 KiB in all. The
// address of entry e for a lane is (e << 8) | lane_off with lane_off = (l % 16) * 8, formed by
// one v_perm_b32 when e is a byte of a payload word and by a shift and a v_and_or_b32
// otherwise; the sign table's 128 rides in the DS instruction's immediate offset.
//
// LDS is addressed by plain byte addresses: the kernels that use these tables declare no static
// LDS (the launch code checks), so their dynamic LDS starts at address 0, the tables sit at its
// start, and the table bases fold into the DS instructions' immediate offsets.
#ifndef VL_DECODE_H
#define VL_DECODE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vl_tables.h"

namespace vl {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// LDS byte offsets of the replicated tables: A (256 grid entries) in the lower halves of 256
// rows of 256 bytes, B (128 sign entries) in the upper halves of the first 128 rows.
constexpr uint32_t kTabCopies = 16;
constexpr uint32_t kTabA = 0;
constexpr uint32_t kTabB = 128;
constexpr uint32_t kReplTableBytes = 256u * 256u;  // 64 KiB
constexpr uint32_t kIq1TableBytes = 2048u * 8u;            // 16 KiB, one copy

__device__ __forceinline__ uint32_t lo32(uint64_t v) { return (uint32_t)v; }
__device__ __forceinline__ uint32_t hi32(uint64_t v) { return (uint32_t)(v >> 32); }

__device__ __forceinline__ uint32_t perm(uint32_t high, uint32_t low, uint32_t sel) {
    return __builtin_amdgcn_perm(high, low, sel);
}

__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t width) {
    return __builtin_amdgcn_ubfe(v, off, width);
}

#define VL_LDS __attribute__((address_space(3)))

// Load of type T from LDS byte address addr.
template <typename T>
__device__ __forceinline__ T lds_load(uint32_t addr) {
    return *reinterpret_cast<const VL_LDS T*>((uintptr_t)addr);
}
__device__ __forceinline__ uint64_t lds_u64(uint32_t addr) { return lds_load<uint64_t>(addr); }

// (byte k of v) << 8 | lane_off, one v_perm_b32.
__device__ __forceinline__ uint32_t byte_entry(uint32_t v, int k, uint32_t lane_off) {
    return perm(v, lane_off, 0x0c0c0000u | ((4u + (uint32_t)k) << 8));
}

// IQ2_XXS group g of a superblock half (vl_layout.h): grid bytes in w[0..3], sign fields in
// w[4..7]. Codes select from the palette {8, 25, 43, -8, -25, -43}.
// IQ2_XXS group g in two halves: the table reads (fetch) and the B fragment from them (finish),
// so that a caller can have the next group's reads in flight while it finishes this one.
struct Iq2Fetch {
    uint64_t a0, b0, a1, b1;
};
__device__ __forceinline__ Iq2Fetch fetch_iq2_xxs(const uint32_t (&w)[8], int g, uint32_t lane_off) {
    const int q = g >> 1, odd = g & 1;
    const uint32_t gw = w[q], sw = w[4 + q];
    const uint32_t a0 = byte_entry(gw, 2 * odd, lane_off);
    const uint32_t a1 = byte_entry(gw, 2 * odd + 1, lane_off);
    const uint32_t b0 = ((odd ? sw >> 6 : sw << 8) & 0x7f00u) | lane_off;
    const uint32_t b1 = ((odd ? sw >> 13 : sw << 1) & 0x7f00u) | lane_off;
    return Iq2Fetch{lds_u64(kTabA + a0), lds_u64(kTabB + b0), lds_u64(kTabA + a1), lds_u64(kTabB + b1)};
}
__device__ __forceinline__ i32x4 finish_iq2_xxs(const Iq2Fetch& t) {
    const uint64_t s0 = t.a0 | t.b0, s1 = t.a1 | t.b1;
    i32x4 f;
    f[0] = (int)perm(kIq2PaletteNeg, kIq2PalettePos, lo32(s0));
    f[1] = (int)perm(kIq2PaletteNeg, kIq2PalettePos, hi32(s0));
    f[2] = (int)perm(kIq2PaletteNeg, kIq2PalettePos, lo32(s1));
    f[3] = (int)perm(kIq2PaletteNeg, kIq2PalettePos, hi32(s1));
    return f;
}

__device__ __forceinline__ i32x4 decode_iq2_xxs(const uint32_t (&w)[8], int g, uint32_t lane_off) {
    const int q = g >> 1, odd = g & 1;
    const uint32_t gw = w[q], sw = w[4 + q];
    const uint32_t a0 = byte_entry(gw, 2 * odd, lane_off);
    const uint32_t a1 = byte_entry(gw, 2 * odd + 1, lane_off);
    // Sign fields at bits 14*odd and 14*odd + 7, moved to bits 8..14: one shift, one and-or.
    const uint32_t b0 = ((odd ? sw >> 6 : sw << 8) & 0x7f00u) | lane_off;
    const uint32_t b1 = ((odd ? sw >> 13 : sw << 1) & 0x7f00u) | lane_off;
    const uint64_t s0 = lds_u64(kTabA + a0) | lds_u64(kTabB + b0);
    const uint64_t s1 = lds_u64(kTabA + a1) | lds_u64(kTabB + b1);
    i32x4 f;
    f[0] = (int)perm(kIq2PaletteNeg, kIq2PalettePos, lo32(s0));
    f[1] = (int)perm(kIq2PaletteNeg, kIq2PalettePos, hi32(s0));
    f[2] = (int)perm(kIq2PaletteNeg, kIq2PalettePos, lo32(s1));
    f[3] = (int)perm(kIq2PaletteNeg, kIq2PalettePos, hi32(s1));
    return f;
}

// IQ2_XXS scales of one superblock: own = this half's four scale bytes (top bytes of w[4..7],
// scale nibble in bits 4..7); lo/hi = the bytes of groups 0..3 and 4..7 once both halves'
// words are known.
__device__ __forceinline__ uint32_t iq2_scale_bytes(const uint32_t (&w)[8]) {
    return perm(w[5], w[4], 0x0c0c0703u) | perm(w[7], w[6], 0x07030c0cu);
}

// 2s+1 of four scale bytes (nibbles in bits 4..7), one per byte: (byte >> 3) | 1 bytewise.
__device__ __forceinline__ uint32_t odd_scales4(uint32_t bytes) {
    return ((bytes >> 3) & 0x1e1e1e1eu) | 0x01010101u;
}

// IQ3_XXS group: q = the lane's four grid bytes (two per sub-block), aux = the group's sign and
// scale word. Magnitude entries hold the four positive values in the low word and their
// negations in the high word; sign entries select per lane.
__device__ __forceinline__ i32x4 decode_iq3_xxs(uint32_t q, uint32_t aux, int hh, uint32_t lane_off) {
    const uint32_t a = aux >> (14 * hh);
    const uint64_t sel0 = lds_u64(kTabB + (((a << 8) & 0x7f00u) | lane_off));
    const uint64_t sel1 = lds_u64(kTabB + (((a << 1) & 0x7f00u) | lane_off));
    const uint64_t g00 = lds_u64(kTabA + byte_entry(q, 0, lane_off));
    const uint64_t g01 = lds_u64(kTabA + byte_entry(q, 1, lane_off));
    const uint64_t g10 = lds_u64(kTabA + byte_entry(q, 2, lane_off));
    const uint64_t g11 = lds_u64(kTabA + byte_entry(q, 3, lane_off));
    i32x4 f;
    f[0] = (int)perm(hi32(g00), lo32(g00), lo32(sel0));
    f[1] = (int)perm(hi32(g01), lo32(g01), hi32(sel0));
    f[2] = (int)perm(hi32(g10), lo32(g10), lo32(sel1));
    f[3] = (int)perm(hi32(g11), lo32(g11), hi32(sel1));
    return f;
}

// IQ1_S group: qs4 = low 8 bits of the four 11-bit grid indices, qh = the group's 16-bit word
// (3 high index bits per sub-block, 3-bit scale at bit 12, delta sign at bit 15).
__device__ __forceinline__ i32x4 decode_iq1_s(uint32_t qs4, uint32_t qh, int hh) {
    const int s0 = 2 * hh;
    const uint32_t i0 = ((qs4 >> (8 * s0)) & 0xffu) | (((qh >> (3 * s0)) & 7u) << 8);
    const uint32_t i1 = ((qs4 >> (8 * s0 + 8)) & 0xffu) | (((qh >> (3 * s0 + 3)) & 7u) << 8);
    const uint64_t dm = (qh & 0x8000u) ? 0x0404040404040404ull : 0ull;
    const uint64_t c0 = lds_u64(i0 * 8u) | dm;
    const uint64_t c1 = lds_u64(i1 * 8u) | dm;
    i32x4 f;
    f[0] = (int)perm(kIq1PaletteNeg, kIq1PalettePos, lo32(c0));
    f[1] = (int)perm(kIq1PaletteNeg, kIq1PalettePos, hi32(c0));
    f[2] = (int)perm(kIq1PaletteNeg, kIq1PalettePos, lo32(c1));
    f[3] = (int)perm(kIq1PaletteNeg, kIq1PalettePos, hi32(c1));
    return f;
}

// IQ1_S group in two halves (grid reads with the delta applied, then the fragment).
struct Iq1Fetch {
    uint64_t c0, c1;
};
__device__ __forceinline__ Iq1Fetch fetch_iq1_s(uint32_t qs4, uint32_t qh, int hh) {
    const int s0 = 2 * hh;
    const uint32_t i0 = ((qs4 >> (8 * s0)) & 0xffu) | (((qh >> (3 * s0)) & 7u) << 8);
    const uint32_t i1 = ((qs4 >> (8 * s0 + 8)) & 0xffu) | (((qh >> (3 * s0 + 3)) & 7u) << 8);
    const uint64_t dm = (qh & 0x8000u) ? 0x0404040404040404ull : 0ull;
    return Iq1Fetch{lds_u64(i0 * 8u) | dm, lds_u64(i1 * 8u) | dm};
}
__device__ __forceinline__ i32x4 finish_iq1_s(const Iq1Fetch& t) {
    i32x4 f;
    f[0] = (int)perm(kIq1PaletteNeg, kIq1PalettePos, lo32(t.c0));
    f[1] = (int)perm(kIq1PaletteNeg, kIq1PalettePos, hi32(t.c0));
    f[2] = (int)perm(kIq1PaletteNeg, kIq1PalettePos, lo32(t.c1));
    f[3] = (int)perm(kIq1PaletteNeg, kIq1PalettePos, hi32(t.c1));
    return f;
}

// Exact binary16 -> binary32 (v_cvt_f32_f16; fp16 denormals are preserved on gfx9).
__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    const uint16_t b = (uint16_t)bits;
    _Float16 h;
    __builtin_memcpy(&h, &b, sizeof h);
    return (float)h;
}

}  // namespace vl

#endif  // VL_DECODE_H
