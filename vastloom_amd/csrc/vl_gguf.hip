// HIP kernels for the storage types that stay in their GGUF bytes on the device: Q4_K, Q5_K,
// Q6_K, IQ2_S, MXFP4, BF16 and F32 (vl_type_tiled() is false for them).
//
//   k_gguf_dequant   GGUF matrix -> float32 rows, bit-identical to the reference decoders
//   k_gguf_matvec    y[token][row] = W x[token] for up to eight tokens, four rows per block
//
// These matrices are read as they are stored, row-major with each row's blocks contiguous, so
// making one resident is a device copy. A "piece" is eight consecutive weights of a row; a block
// holds a whole number of pieces (32 for the 256-weight K-quants, 4 for MXFP4), so a piece never
// crosses a block (the row products take 16-weight pieces of the K-quants when they carry one or
// two token slots). A 256-thread block takes four rows: thread i decodes the pieces i, i + 256,
// ... of each, two pieces per row at a time with all their loads issued before the first is
// decoded, and accumulates w * x in float per row and token (the activations of a piece are
// loaded once for the four rows; block and sub-block factors multiply the piece's sum of
// integer code times x rather than each weight); the block then adds its 256 partial sums per
// row and token in a fixed order.
// The dequantize kernel forms each weight exactly as the reference does (each product and
// difference rounded once, in the reference's order, fp contraction off) and is bit-exact; the
// matvec differs from the reference's float64 accumulation only by float rounding of its
// partial sums.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iq_codebooks.h"
#include "vl_kernels.h"
#include "vl_layout.h"
#include "vl_moe.h"
#include "vl_moe_dev.h"
#include "vl_stream.h"

namespace vl {

namespace {

// The IQ2_S grid (1024 entries of eight magnitudes in {8, 25, 43}, lane l in bits 8l..8l+7),
// expanded at compile time from the compact codes; identical to the reference's table, whose
// fingerprint the host-side expansion checks.
struct Iq2sGrid {
    uint64_t g[1024];
};
constexpr Iq2sGrid make_iq2s_grid() {
    Iq2sGrid t{};
    constexpr uint16_t codes[1024] = VL_IQ2S_CODES;
    constexpr uint8_t v[4] = {8, 25, 43, 0};
    for (unsigned e = 0; e < 1024; ++e) {
        uint64_t g = 0;
        for (unsigned l = 0; l < 8; ++l) g |= (uint64_t)v[(codes[e] >> (2 * l)) & 3u] << (8 * l);
        t.g[e] = g;
    }
    return t;
}
__device__ const Iq2sGrid kIq2sGrid = make_iq2s_grid();

__device__ __forceinline__ uint32_t ld_u8(const uint8_t* p) { return *gp(p); }
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {  // p 2-byte aligned
    return *gp(reinterpret_cast<const uint16_t*>(p));
}
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {  // p 4-byte aligned
    return *gp(reinterpret_cast<const uint32_t*>(p));
}
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint2 ld_u64(const uint8_t* p) {  // p 8-byte aligned
    const u32x2 v = *gp(reinterpret_cast<const u32x2*>(p));
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ u32x4 ld_u128(const uint8_t* p) {  // p 16-byte aligned
    return *gp(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ uint32_t byte_of(uint2 v, int i) {
    return ((i < 4 ? v.x : v.y) >> (8 * (i & 3))) & 0xffu;
}
__device__ __forceinline__ float bits_float(uint32_t b) { return __uint_as_float(b); }

// The 6-bit scale and minimum of sub-block j of a Q4_K/Q5_K superblock from its 12 scale bytes
// held as three little-endian words b (bytes 0-3), c (4-7), d (8-11): for j < 4 the low six bits
// of byte j (scale) and byte j + 4 (minimum); for j >= 4 the nibbles of byte j + 4 with the top
// two bits of bytes j - 4 (scale) and j (minimum) above them (ggml_quantization.cpp:435-455).
__device__ __forceinline__ void k_scale_min(uint32_t b, uint32_t c, uint32_t d, uint32_t j,
                                            uint32_t& sc, uint32_t& mn) {
    const uint32_t sh = 8u * (j & 3u);
    const uint32_t lb = b >> sh, lc = c >> sh, ld = d >> sh;
    if (j < 4u) {
        sc = lb & 63u;
        mn = lc & 63u;
    } else {
        sc = (ld & 15u) | ((lb >> 2) & 0x30u);
        mn = ((ld >> 4) & 15u) | ((lc >> 2) & 0x30u);
    }
}

// The raw bytes one piece needs, loaded before any of them is used.
struct RawPiece {
    uint32_t a, b, c, d;  // format-specific words
    uint2 q, h;           // quant bytes and high bits
};

// Weights per block and bytes per block of each format (the K-quants' 256-weight superblocks,
// MXFP4's 32-weight blocks; BF16 is handled per element).
template <uint32_t FMT> struct Fmt;
template <> struct Fmt<VL_TYPE_Q4_K> { static constexpr uint32_t be = 256, bb = 144; };
template <> struct Fmt<VL_TYPE_Q5_K> { static constexpr uint32_t be = 256, bb = 176; };
template <> struct Fmt<VL_TYPE_Q6_K> { static constexpr uint32_t be = 256, bb = 210; };
template <> struct Fmt<VL_TYPE_IQ2_S> { static constexpr uint32_t be = 256, bb = 82; };
template <> struct Fmt<VL_TYPE_MXFP4> { static constexpr uint32_t be = 32, bb = 17; };
template <> struct Fmt<VL_TYPE_BF16> { static constexpr uint32_t be = 1, bb = 2; };
template <> struct Fmt<VL_TYPE_F32> { static constexpr uint32_t be = 1, bb = 4; };

// Loads piece p of a row (row = the row's first byte). Offsets within the row are 32-bit (the
// launchers refuse rows of 4 GiB or more). A BF16 or F32 piece past the row's last column reads
// nothing for the missing columns.
template <uint32_t FMT>
__device__ __forceinline__ void load_piece(const uint8_t* row, uint32_t p, uint32_t cols, RawPiece& r) {
    if constexpr (FMT == VL_TYPE_F32) {
        const uint8_t* e = row + 32u * p;
        if ((cols & 7u) == 0u) {  // row bytes % 32 == 0: two 16-byte loads
            const u32x4 v0 = ld_u128(e), v1 = ld_u128(e + 16);
            r.a = v0.x; r.b = v0.y; r.c = v0.z; r.d = v0.w;
            r.q = make_uint2(v1.x, v1.y);
            r.h = make_uint2(v1.z, v1.w);
        } else {
            uint32_t w[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (8u * p + i < cols) w[i] = ld_u32(e + 4 * i);
            r.a = w[0]; r.b = w[1]; r.c = w[2]; r.d = w[3];
            r.q = make_uint2(w[4], w[5]);
            r.h = make_uint2(w[6], w[7]);
        }
    } else if constexpr (FMT == VL_TYPE_BF16) {
        const uint8_t* e = row + 16u * p;
        if ((cols & 7u) == 0u) {  // rows of whole pieces: one 16-byte load (row bytes % 16 == 0)
            const u32x4 v = ld_u128(e);
            r.a = v.x; r.b = v.y; r.c = v.z; r.d = v.w;
        } else {
            uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (8u * p + i < cols) w[i >> 1] |= ld_u16(e + 2 * i) << (16 * (i & 1));
            r.a = w[0]; r.b = w[1]; r.c = w[2]; r.d = w[3];
        }
    } else if constexpr (FMT == VL_TYPE_MXFP4) {
        // Piece q of a block: low nibbles (q < 2) or high nibbles (q >= 2) of code bytes
        // 1 + 8 (q & 1) .. +7. Blocks are 17 bytes, so every byte is loaded on its own.
        const uint32_t q = p & 3u;
        const uint8_t* blk = row + 17u * (p >> 2);
        const uint8_t* c = blk + 1u + 8u * (q & 1u);
        r.a = ld_u8(blk);
        r.q.x = ld_u8(c) | ld_u8(c + 1) << 8 | ld_u8(c + 2) << 16 | ld_u8(c + 3) << 24;
        r.q.y = ld_u8(c + 4) | ld_u8(c + 5) << 8 | ld_u8(c + 6) << 16 | ld_u8(c + 7) << 24;
    } else if constexpr (FMT == VL_TYPE_IQ2_S) {
        // Piece q of a block is sub-block s = q & 3 of group g = q >> 2: its grid index byte,
        // sign byte, the group's high-index byte and scale byte, and the block's d (82-byte
        // blocks: d is 2-byte aligned, the rest are single bytes).
        const uint32_t q = p & 31u, g = q >> 2, sb = q & 3u;
        const uint8_t* blk = row + 82u * (p >> 5);
        r.a = ld_u16(blk);
        r.b = ld_u8(blk + 2u + 4u * g + sb);
        r.c = ld_u8(blk + 34u + 4u * g + sb);
        r.d = ld_u8(blk + 66u + g) | ld_u8(blk + 74u + g) << 8;
    } else if constexpr (FMT == VL_TYPE_Q6_K) {
        // Blocks are 210 bytes: 2-byte aligned loads only. Piece q = 16h + 4k + l0/8.
        const uint32_t q = p & 31u, h = q >> 4, k = (q >> 2) & 3u, l0 = (q & 3u) * 8u;
        const uint32_t b0 = 210u * (p >> 5);
        const uint8_t* blk = row + b0;
        const uint8_t* lo = row + (b0 + 64u * h + 32u * (k & 1u) + l0);
        const uint8_t* hi = row + (b0 + 128u + 32u * h + l0);
        r.q.x = ld_u16(lo) | ld_u16(lo + 2) << 16;
        r.q.y = ld_u16(lo + 4) | ld_u16(lo + 6) << 16;
        r.h.x = ld_u16(hi) | ld_u16(hi + 2) << 16;
        r.h.y = ld_u16(hi + 4) | ld_u16(hi + 6) << 16;
        r.a = ld_u16(blk + 208u);
        r.b = ld_u8(blk + 192u + 8u * h + (l0 >> 4) + 2u * k);
    } else {  // Q4_K, Q5_K: 144- and 176-byte blocks keep 16-byte alignment
        const uint32_t q = p & 31u, j = q >> 2, l0 = (q & 3u) * 8u;
        const uint32_t b0 = Fmt<FMT>::bb * (p >> 5);
        const u32x4 head = ld_u128(row + b0);  // d, dmin and the 12 scale bytes
        r.a = head.x; r.b = head.y; r.c = head.z; r.d = head.w;
        if constexpr (FMT == VL_TYPE_Q5_K) {
            r.h = ld_u64(row + (b0 + 16u + l0));
            r.q = ld_u64(row + (b0 + 48u + 32u * (j >> 1) + l0));
        } else {
            r.q = ld_u64(row + (b0 + 16u + 32u * (j >> 1) + l0));
        }
    }
}

// The eight weights of piece p, exactly as the reference decoders produce them
// (ggml_quantization.cpp:285-334, :381-413, :435-589).
template <uint32_t FMT>
__device__ __forceinline__ void decode_piece(const RawPiece& r, uint32_t p, float w[8]) {
#pragma clang fp contract(off)
    if constexpr (FMT == VL_TYPE_F32) {
        const uint32_t v[8] = {r.a, r.b, r.c, r.d, r.q.x, r.q.y, r.h.x, r.h.y};
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = bits_float(v[i]);
    } else if constexpr (FMT == VL_TYPE_BF16) {
        const uint32_t v[4] = {r.a, r.b, r.c, r.d};
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = bits_float((i & 1) ? (v[i >> 1] & 0xffff0000u) : (v[i >> 1] << 16));
    } else if constexpr (FMT == VL_TYPE_MXFP4) {
        // Scale: E8M0 with the half of the doubled code table folded in; codes: twice E2M1.
        const uint32_t e = r.a;
        const float s = bits_float(e < 2u ? 0x00200000u << e : (e - 1u) << 23);
        const uint32_t shift = 4u * ((p & 3u) >> 1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = (byte_of(r.q, i) >> shift) & 15u, m = c & 7u;
            const int mag = m < 4u ? (int)m : (int)((m & 1u ? 6u : 4u) << ((m - 4u) >> 1));
            w[i] = (float)(c & 8u ? -mag : mag) * s;
        }
    } else if constexpr (FMT == VL_TYPE_IQ2_S) {
        const uint32_t sb = p & 3u;
        const uint32_t index = r.b | ((r.d >> (2u * sb)) & 3u) << 8;
        const uint64_t grid = *gp(&kIq2sGrid.g[index]);
        const uint32_t nib = sb < 2u ? (r.d >> 8) & 15u : (r.d >> 12) & 15u;
        const float ls = half_bits_to_float(r.a) * (0.5f + (float)nib) * 0.25f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float mag = (float)((uint32_t)(grid >> (8 * i)) & 0xffu);
            w[i] = ls * mag * ((r.c >> i) & 1u ? -1.0f : 1.0f);
        }
    } else if constexpr (FMT == VL_TYPE_Q6_K) {
        const uint32_t q = p & 31u, k = (q >> 2) & 3u;
        const float d = half_bits_to_float(r.a);
        const float ds = d * (float)(int)(int8_t)(uint8_t)r.b;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lb = byte_of(r.q, i);
            const uint32_t nib = k < 2u ? (lb & 15u) : (lb >> 4);
            const int v = (int)(nib | ((byte_of(r.h, i) >> (2u * k)) & 3u) << 4) - 32;
            w[i] = ds * (float)v;
        }
    } else {  // Q4_K, Q5_K
        const uint32_t j = (p & 31u) >> 2;
        const float d = half_bits_to_float(r.a), dmin = half_bits_to_float(r.a >> 16);
        // Sub-block j's 6-bit scale and minimum from the 12 packed bytes (words b, c, d).
        uint32_t sc, mn;
        k_scale_min(r.b, r.c, r.d, j, sc, mn);
        const float dj = d * (float)sc, mj = dmin * (float)mn;
        const uint32_t shift = 4u * (j & 1u);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t v = (byte_of(r.q, i) >> shift) & 15u;
            if constexpr (FMT == VL_TYPE_Q5_K) v += ((byte_of(r.h, i) >> j) & 1u) << 4;
            w[i] = dj * (float)v - mj;
        }
    }
}

template <uint32_t FMT>
__device__ __forceinline__ uint64_t row_bytes(uint32_t cols) {
    return (uint64_t)(cols / Fmt<FMT>::be) * Fmt<FMT>::bb;
}

// One thread per piece of the matrix.
template <uint32_t FMT>
__global__ void __launch_bounds__(256) k_gguf_dequant(vl_tiled_layout L, const uint8_t* __restrict__ w,
                                                      float* __restrict__ out) {
    const uint32_t ppr = (L.cols + 7u) / 8u;
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i >= (uint64_t)L.rows * ppr) return;
    const uint32_t row = (uint32_t)(i / ppr), p = (uint32_t)(i % ppr);
    RawPiece r;
    load_piece<FMT>(w + (uint64_t)row * row_bytes<FMT>(L.cols), p, L.cols, r);
    float v[8];
    decode_piece<FMT>(r, p, v);
    float* dst = out + (uint64_t)row * L.cols + 8u * p;
    if (8u * p + 8u <= L.cols) {
#pragma unroll
        for (int k = 0; k < 8; ++k) dst[k] = v[k];
    } else {
        for (uint32_t k = 0; 8u * p + k < L.cols; ++k) dst[k] = v[k];
    }
}

// Four unsigned bytes of a word as floats (v_cvt_f32_ubyte0..3).
__device__ __forceinline__ void bytes_float(uint32_t v, float* f) {
    // Opaque to the compiler, so that the masks and shifts that formed v are not folded into a
    // bit-field extract per byte: each byte then converts with one v_cvt_f32_ubyteN.
    asm("" : "+v"(v));
    f[0] = (float)(v & 0xffu);
    f[1] = (float)((v >> 8) & 0xffu);
    f[2] = (float)((v >> 16) & 0xffu);
    f[3] = (float)(v >> 24);
}

// acc[t] += sum_i w_i x[t][i] over piece p, for the matvec. The block and sub-block factors are
// taken out of the sum: K-quant pieces are d_j * sum q_i x_i - m_j * sum x_i (Q6_K:
// d_s * (sum q_i x_i - 32 sum x_i)), MXFP4 pieces s * sum v_i x_i, with the small integer codes
// converted straight from their bytes (IQ2_S pieces: ls * sum (+/-grid magnitude) x_i);
// sx[t] = sum_i x[t][i] is shared by the block's rows.
// Only the rounding of these partial sums differs from forming each weight first.
template <uint32_t FMT, int NT>
__device__ __forceinline__ void piece_dot(const RawPiece& r, uint32_t p, const float (&xv)[NT][8],
                                          const float (&sx)[NT], float (&acc)[NT]) {
    if constexpr (FMT == VL_TYPE_F32 || FMT == VL_TYPE_BF16) {
        float w[8];
        decode_piece<FMT>(r, p, w);
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[t] = fmaf(w[i], xv[t][i], acc[t]);
    } else if constexpr (FMT == VL_TYPE_IQ2_S) {
        const uint32_t sb = p & 3u;
        const uint32_t index = r.b | ((r.d >> (2u * sb)) & 3u) << 8;
        const uint64_t grid = *gp(&kIq2sGrid.g[index]);
        const uint32_t nib = sb < 2u ? (r.d >> 8) & 15u : (r.d >> 12) & 15u;
        const float ls = half_bits_to_float(r.a) * (0.5f + (float)nib) * 0.25f;
        float v[8];
        bytes_float((uint32_t)grid, v);
        bytes_float((uint32_t)(grid >> 32), v + 4);
        // Sign bit i of the sign byte flips the sign of activation i.
        uint32_t neg[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) neg[i] = (r.c << (31 - i)) & 0x80000000u;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) d = fmaf(v[i], __uint_as_float(__float_as_uint(xv[t][i]) ^ neg[i]), d);
            acc[t] = fmaf(ls, d, acc[t]);
        }
    } else if constexpr (FMT == VL_TYPE_MXFP4) {
        // Four codes per word, one per byte: v_perm_b32 picks each code's magnitude (0, 1, 2, 3,
        // 4, 6, 8, 12 for codes & 7) out of an eight-byte table, and the code's sign bit flips
        // the sign of the matching activation.
        const uint32_t e = r.a;
        const float s = bits_float(e < 2u ? 0x00200000u << e : (e - 1u) << 23);
        const uint32_t shift = 4u * ((p & 3u) >> 1);
        const uint32_t c0 = (r.q.x >> shift) & 0x0f0f0f0fu, c1 = (r.q.y >> shift) & 0x0f0f0f0fu;
        float v[8];
        bytes_float(__builtin_amdgcn_perm(0x0c080604u, 0x03020100u, c0 & 0x07070707u), v);
        bytes_float(__builtin_amdgcn_perm(0x0c080604u, 0x03020100u, c1 & 0x07070707u), v + 4);
        uint32_t neg[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            neg[i] = (c0 << (28 - 8 * i)) & 0x80000000u;      // bit 3 of byte i -> bit 31
            neg[i + 4] = (c1 << (28 - 8 * i)) & 0x80000000u;
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) d = fmaf(v[i], __uint_as_float(__float_as_uint(xv[t][i]) ^ neg[i]), d);
            acc[t] = fmaf(s, d, acc[t]);
        }
    } else {
        float q[8];
        float scale, offset;  // acc += scale * (sum q x) - offset * (sum x)
        if constexpr (FMT == VL_TYPE_Q6_K) {
            const uint32_t k = ((p & 31u) >> 2) & 3u;
            const uint32_t sh = k < 2u ? 0u : 4u;
            const uint32_t lo = (r.q.x >> sh) & 0x0f0f0f0fu, hi = (r.q.y >> sh) & 0x0f0f0f0fu;
            bytes_float(lo | ((r.h.x >> (2u * k)) & 0x03030303u) << 4, q);
            bytes_float(hi | ((r.h.y >> (2u * k)) & 0x03030303u) << 4, q + 4);
            scale = half_bits_to_float(r.a) * (float)(int)(int8_t)(uint8_t)r.b;
            offset = 32.0f * scale;
        } else {  // Q4_K, Q5_K
            const uint32_t j = (p & 31u) >> 2;
            const float d = half_bits_to_float(r.a), dmin = half_bits_to_float(r.a >> 16);
            uint32_t sc, mn;
            k_scale_min(r.b, r.c, r.d, j, sc, mn);
            const uint32_t sh = 4u * (j & 1u);
            uint32_t lo = (r.q.x >> sh) & 0x0f0f0f0fu, hi = (r.q.y >> sh) & 0x0f0f0f0fu;
            if constexpr (FMT == VL_TYPE_Q5_K) {
                lo |= ((r.h.x >> j) & 0x01010101u) << 4;
                hi |= ((r.h.y >> j) & 0x01010101u) << 4;
            }
            bytes_float(lo, q);
            bytes_float(hi, q + 4);
            scale = d * (float)sc;
            offset = dmin * (float)mn;
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) d = fmaf(q[i], xv[t][i], d);
            acc[t] = fmaf(scale, d, fmaf(-offset, sx[t], acc[t]));
        }
    }
}

__global__ void k_gguf_clear_status(uint32_t* status) {
    if (threadIdx.x == 0) *status = 0u;
}

constexpr int kPiecesInFlight = 2;

constexpr uint32_t kRowsPerBlock = 4;

// Weights per piece in the row products: 16 for the K-quants with at most two token slots, so
// that one header load and one scale unpacking serve 16 weights of a sub-block; 8 otherwise.
template <uint32_t FMT, int NT>
constexpr int piece_width() {
    return (FMT == VL_TYPE_Q4_K || FMT == VL_TYPE_Q5_K || FMT == VL_TYPE_Q6_K) && NT <= 2 ? 16 : 8;
}

// The raw bytes of a 16-weight K-quant piece. Q4_K/Q5_K: the block header and the 16 quant (and
// high-bit) bytes of half a sub-block, all 16-byte aligned (144- and 176-byte blocks). Q6_K: the
// 16 low-nibble and 16 high-bit bytes of the piece, its scale byte and d (210-byte blocks: 2-byte
// loads).
struct RawWide {
    uint32_t a, b, c, d;
    u32x4 q, h;
};

template <uint32_t FMT>
__device__ __forceinline__ void load_wide(const uint8_t* row, uint32_t p, RawWide& r) {
    if constexpr (FMT == VL_TYPE_Q6_K) {
        // Piece q = 8h + 2k + l0/16 holds weights 128h + 32k + l0 .. +15 of its block.
        const uint32_t q = p & 15u, h = q >> 3, k = (q >> 1) & 3u, l0 = (q & 1u) * 16u;
        const uint32_t b0 = 210u * (p >> 4);
        const uint8_t* lo = row + (b0 + 64u * h + 32u * (k & 1u) + l0);
        const uint8_t* hi = row + (b0 + 128u + 32u * h + l0);
        uint32_t lw[4], hw[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            lw[w] = ld_u16(lo + 4 * w) | ld_u16(lo + 4 * w + 2) << 16;
            hw[w] = ld_u16(hi + 4 * w) | ld_u16(hi + 4 * w + 2) << 16;
        }
        r.q = u32x4{lw[0], lw[1], lw[2], lw[3]};
        r.h = u32x4{hw[0], hw[1], hw[2], hw[3]};
        r.a = ld_u16(row + (b0 + 208u));
        r.b = ld_u8(row + (b0 + 192u + 8u * h + (l0 >> 4) + 2u * k));
        return;
    }
    const uint32_t q = p & 15u, j = q >> 1, l0 = (q & 1u) * 16u;
    const uint32_t b0 = Fmt<FMT>::bb * (p >> 4);
    const u32x4 head = ld_u128(row + b0);
    r.a = head.x; r.b = head.y; r.c = head.z; r.d = head.w;
    if constexpr (FMT == VL_TYPE_Q5_K) {
        r.h = ld_u128(row + (b0 + 16u + l0));
        r.q = ld_u128(row + (b0 + 48u + 32u * (j >> 1) + l0));
    } else {
        r.q = ld_u128(row + (b0 + 16u + 32u * (j >> 1) + l0));
    }
}

// acc[t] += d_j * sum q_i x[t][i] - m_j * sum x[t][i] over the 16 weights of piece p.
template <uint32_t FMT, int NT, int PW>
__device__ __forceinline__ void wide_dot(const RawWide& r, uint32_t p, const float (&xv)[NT][PW],
                                         const float (&sx)[NT], float (&acc)[NT]) {
    if constexpr (FMT == VL_TYPE_Q6_K) {
        // acc[t] += (d * scale) * (sum q_i x[t][i] - 32 sum x[t][i]), q_i the 6-bit codes.
        const uint32_t k = ((p & 15u) >> 1) & 3u, sh = k < 2u ? 0u : 4u;
        const uint32_t lw[4] = {r.q.x, r.q.y, r.q.z, r.q.w}, hw[4] = {r.h.x, r.h.y, r.h.z, r.h.w};
        float q[16];
#pragma unroll
        for (int w = 0; w < 4; ++w)
            bytes_float(((lw[w] >> sh) & 0x0f0f0f0fu) | ((hw[w] >> (2u * k)) & 0x03030303u) << 4, q + 4 * w);
        const float scale = half_bits_to_float(r.a) * (float)(int)(int8_t)(uint8_t)r.b;
        const float offset = 32.0f * scale;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) s = fmaf(q[i], xv[t][i], s);
            acc[t] = fmaf(scale, s, fmaf(-offset, sx[t], acc[t]));
        }
        return;
    }
    const uint32_t j = (p & 15u) >> 1;
    const float d = half_bits_to_float(r.a), dmin = half_bits_to_float(r.a >> 16);
    uint32_t sc, mn;
    k_scale_min(r.b, r.c, r.d, j, sc, mn);
    const uint32_t sh = 4u * (j & 1u);
    const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    float q[16];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t v = (qw[w] >> sh) & 0x0f0f0f0fu;
        if constexpr (FMT == VL_TYPE_Q5_K) {
            const uint32_t hw = w == 0 ? r.h.x : w == 1 ? r.h.y : w == 2 ? r.h.z : r.h.w;
            v |= ((hw >> j) & 0x01010101u) << 4;
        }
        bytes_float(v, q + 4 * w);
    }
    const float scale = d * (float)sc, offset = dmin * (float)mn;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) s = fmaf(q[i], xv[t][i], s);
        acc[t] = fmaf(scale, s, fmaf(-offset, sx[t], acc[t]));
    }
}

// Per-block LDS of the row products: each wave's sums, then the block's.
template <int NT>
struct RowsLds {
    float part[4][kRowsPerBlock][NT];
    float sum[kRowsPerBlock][NT];
    uint32_t bad[4];
};

// The products of nrows (<= kRowsPerBlock) rows of W, starting at rp with row stride rb, with the
// activation rows xs[0 .. ntok-1]; the result lands in lds.sum[row][t] (valid on return for
// every thread), and whether any activation was non-finite is returned. Thread i takes pieces i,
// i + 256, ... of each row, so that the activations it loads for a piece serve all the rows, and
// issues the loads of kPiecesInFlight pieces of every row before it decodes the first. Each wave
// adds its lanes; the four waves' sums are added in wave order.
template <uint32_t FMT, int NT, int NTS, bool CHECK_X = true>
__device__ __forceinline__ bool block_rows_dot(const uint8_t* rp, uint64_t rb, uint32_t nrows,
                                               uint32_t cols, const float* const (&xs)[NTS],
                                               uint32_t ntok, RowsLds<NTS>& lds) {
    static_assert(NT <= NTS, "token slots beyond the LDS rows");
    constexpr uint32_t R = kRowsPerBlock;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t ppr = (cols + 7u) / 8u;
    const bool whole = (cols & 7u) == 0u;
    float acc[R][NT];
#pragma unroll
    for (uint32_t rr = 0; rr < R; ++rr)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[rr][t] = 0.0f;
    bool bad_x = false;
    constexpr int PW = piece_width<FMT, NT>();
    if constexpr (PW > 8) {
        const uint32_t ppw = cols / PW;  // K-quant rows are whole 256-weight blocks
        for (uint32_t base = tid; base < ppw; base += 256u * kPiecesInFlight) {
            RawWide r[kPiecesInFlight][R];  // PW-weight pieces
#pragma unroll
            for (int u = 0; u < kPiecesInFlight; ++u) {
                const uint32_t p = base + 256u * u;
#pragma unroll
                for (uint32_t rr = 0; rr < R; ++rr)
                    if (p < ppw && rr < nrows) load_wide<FMT>(rp + rr * rb, p, r[u][rr]);
            }
#pragma unroll
            for (int u = 0; u < kPiecesInFlight; ++u) {
                const uint32_t p = base + 256u * u;
                if (p >= ppw) break;
                float xv[NT][PW];
                float sx[NT];
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const float* xp = xs[t] + (uint32_t)PW * p;
#pragma unroll
                    for (int k = 0; k < PW / 4; ++k) {
                        const f32x4 v = t < (int)ntok ? *gp(reinterpret_cast<const f32x4*>(xp + 4 * k))
                                                      : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                        xv[t][4 * k] = v.x; xv[t][4 * k + 1] = v.y; xv[t][4 * k + 2] = v.z; xv[t][4 * k + 3] = v.w;
                    }
                    if constexpr (CHECK_X) {
#pragma unroll
                        for (int i = 0; i < PW; ++i) bad_x |= !__builtin_isfinite(xv[t][i]);
                    }
                    float h[PW / 2];
#pragma unroll
                    for (int i = 0; i < PW / 2; ++i) h[i] = xv[t][2 * i] + xv[t][2 * i + 1];
                    sx[t] = 0.0f;
#pragma unroll
                    for (int i = 0; i < PW / 2; ++i) sx[t] += h[i];
                }
#pragma unroll
                for (uint32_t rr = 0; rr < R; ++rr) {
                    if (rr >= nrows) break;
                    wide_dot<FMT, NT, PW>(r[u][rr], p, xv, sx, acc[rr]);
                }
            }
        }
    } else
    for (uint32_t base = tid; base < ppr; base += 256u * kPiecesInFlight) {
        RawPiece r[kPiecesInFlight][R];
#pragma unroll
        for (int u = 0; u < kPiecesInFlight; ++u) {
            const uint32_t p = base + 256u * u;
#pragma unroll
            for (uint32_t rr = 0; rr < R; ++rr)
                if (p < ppr && rr < nrows) load_piece<FMT>(rp + rr * rb, p, cols, r[u][rr]);
        }
#pragma unroll
        for (int u = 0; u < kPiecesInFlight; ++u) {
            const uint32_t p = base + 256u * u;
            if (p >= ppr) break;
            float xv[NT][8];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float* xp = xs[t] + 8u * p;
                if (t >= (int)ntok) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) xv[t][i] = 0.0f;
                } else if (whole) {
                    const f32x4 a = *gp(reinterpret_cast<const f32x4*>(xp));
                    const f32x4 b = *gp(reinterpret_cast<const f32x4*>(xp + 4));
                    xv[t][0] = a.x; xv[t][1] = a.y; xv[t][2] = a.z; xv[t][3] = a.w;
                    xv[t][4] = b.x; xv[t][5] = b.y; xv[t][6] = b.z; xv[t][7] = b.w;
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) xv[t][i] = 8u * p + i < cols ? xp[i] : 0.0f;
                }
                if constexpr (CHECK_X) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) bad_x |= !__builtin_isfinite(xv[t][i]);
                }
            }
            float sx[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t)
                sx[t] = ((xv[t][0] + xv[t][1]) + (xv[t][2] + xv[t][3])) +
                        ((xv[t][4] + xv[t][5]) + (xv[t][6] + xv[t][7]));
#pragma unroll
            for (uint32_t rr = 0; rr < R; ++rr) {
                if (rr >= nrows) break;
                piece_dot<FMT, NT>(r[u][rr], p, xv, sx, acc[rr]);
            }
        }
    }
#pragma unroll
    for (uint32_t rr = 0; rr < R; ++rr)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) acc[rr][t] += __shfl_xor(acc[rr][t], off, 64);
    const bool wave_bad = __ballot(bad_x) != 0ull;
    if (lane == 0) {
#pragma unroll
        for (uint32_t rr = 0; rr < R; ++rr)
#pragma unroll
            for (int t = 0; t < NT; ++t) lds.part[wave][rr][t] = acc[rr][t];
        lds.bad[wave] = wave_bad ? 1u : 0u;
    }
    __syncthreads();
    if (tid < R * NT) {
        const uint32_t rr = tid / NT, t = tid % NT;
        lds.sum[rr][t] = ((lds.part[0][rr][t] + lds.part[1][rr][t]) + lds.part[2][rr][t]) + lds.part[3][rr][t];
    }
    const bool any_bad = (lds.bad[0] | lds.bad[1] | lds.bad[2] | lds.bad[3]) != 0u;
    __syncthreads();
    return any_bad;
}

// kRowsPerBlock rows per 256-thread block (block_rows_dot). NT = token slots (tokens <= NT).
template <uint32_t FMT, int NT>
__global__ void __launch_bounds__(256) k_gguf_matvec(vl_tiled_layout L, const uint8_t* __restrict__ W,
                                                     const float* __restrict__ x, uint32_t tokens,
                                                     float* __restrict__ y, uint32_t* status) {
    __shared__ RowsLds<NT> lds;
    const uint32_t row0 = blockIdx.x * kRowsPerBlock;  // grid = ceil(rows / kRowsPerBlock)
    const uint32_t nrows = L.rows - row0 < kRowsPerBlock ? L.rows - row0 : kRowsPerBlock;
    const uint64_t rb = row_bytes<FMT>(L.cols);
    const float* xs[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) xs[t] = x + (uint64_t)t * L.cols;
    const bool bad_x = block_rows_dot<FMT, NT, NT>(W + (uint64_t)row0 * rb, rb, nrows, L.cols, xs, tokens, lds);
    if (threadIdx.x == 0) {
        uint32_t bits = bad_x ? kStatusNonFiniteInput : 0u;
        for (uint32_t rr = 0; rr < nrows; ++rr)
            for (uint32_t t = 0; t < tokens && t < (uint32_t)NT; ++t) {
                const float v = lds.sum[rr][t];
                y[(uint64_t)t * L.rows + row0 + rr] = v;
                if (!__builtin_isfinite(v)) bits |= kStatusNonFiniteOutput;
            }
        if (bits) or_bits(status, bits);
    }
}

// block_rows_dot with as many token slots as the group has tokens (1, 2, 4 or 8): a group's
// token count is uniform over the block. The layer's plan has already checked the activations
// (a non-finite one refuses the layer), and h is checked where it is formed.
template <uint32_t FMT>
__device__ __forceinline__ void rows_dot_slots(const uint8_t* rp, uint64_t rb, uint32_t nrows, uint32_t cols,
                                               const float* const (&xs)[kMoeMaxTokens], uint32_t ntok,
                                               RowsLds<kMoeMaxTokens>& lds) {
    constexpr int S = kMoeMaxTokens;
    if (ntok <= 1) block_rows_dot<FMT, 1, S, false>(rp, rb, nrows, cols, xs, ntok, lds);
    else if (ntok <= 2) block_rows_dot<FMT, 2, S, false>(rp, rb, nrows, cols, xs, ntok, lds);
    else if (ntok <= 4) block_rows_dot<FMT, 4, S, false>(rp, rb, nrows, cols, xs, ntok, lds);
    else block_rows_dot<FMT, 8, S, false>(rp, rb, nrows, cols, xs, ntok, lds);
}

// MoE layer stages for GGUF-layout experts, on the grouped layer's plan (the active groups of up
// to kMoeMaxTokens tokens of one expert, their weight pointers and the combine entries), with
// the grouped layer's h [group][slot][inter] and per-slot down outputs [group][slot][width] that
// k_moe_combine adds. Block (bx, a): rows 4 bx .. 4 bx + 3 of group a; groups past the plan's
// count leave at once.
template <uint32_t FMT>
__global__ void __launch_bounds__(256) k_gguf_moe_gateup(const MoeShape s, const MoeInputs in,
                                                         const MoeWorkspace w) {
    constexpr int NT = kMoeMaxTokens;
    __shared__ RowsLds<NT> lg, lu;
    const uint32_t a = blockIdx.y;
    if (a >= *gp(&ws_ptr<const MoeHeader>(w, w.off_header)->n_active)) return;  // whole block
    const ActiveExpert* ae = ws_ptr<const ActiveExpert>(w, w.off_active) + a;
    const MoeExpert ex = ws_ptr<const MoeExpert>(w, w.off_gweights)[a];
    const uint32_t F = s.inter, H = s.width, ntok = *gp(&ae->ntok);
    const uint32_t row0 = blockIdx.x * kRowsPerBlock;
    const uint32_t nrows = F - row0 < kRowsPerBlock ? F - row0 : kRowsPerBlock;
    const uint64_t rb = row_bytes<FMT>(H);
    const float* xs[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) xs[t] = in.x + (uint64_t)(t < (int)ntok ? *gp(&ae->tok[t]) : 0u) * H;
    rows_dot_slots<FMT>(ex.gate + (uint64_t)row0 * rb, rb, nrows, H, xs, ntok, lg);
    rows_dot_slots<FMT>(ex.up + (uint64_t)row0 * rb, rb, nrows, H, xs, ntok, lu);
    const uint32_t tid = threadIdx.x, rr = tid / NT, t = tid % NT;
    bool bad = false;
    if (tid < kRowsPerBlock * NT && rr < nrows && t < ntok) {
        const float g = lg.sum[rr][t], u = lu.sum[rr][t];
        const float h = swiglu(s.semantics, g, u, *gp(&ae->limit), *gp(&ae->apply_w) != 0u, *gp(&ae->route_w[t]));
        bad = !__builtin_isfinite(g) || !__builtin_isfinite(u) || !__builtin_isfinite(h);
        *gp(ws_ptr<float>(w, w.off_h) + ((uint64_t)a * NT + t) * F + row0 + rr) = h;
    }
    if (__any(bad) && (tid & 63u) == 0)
        or_bits(&ws_ptr<MoeHeader>(w, w.off_header)->status, kStatusNonFiniteOutput);
}

template <uint32_t FMT>
__global__ void __launch_bounds__(256) k_gguf_moe_down(const MoeShape s, const MoeInputs in,
                                                       const MoeWorkspace w) {
    constexpr int NT = kMoeMaxTokens;
    __shared__ RowsLds<NT> ld;
    const uint32_t a = blockIdx.y;
    if (a >= *gp(&ws_ptr<const MoeHeader>(w, w.off_header)->n_active)) return;  // whole block
    const ActiveExpert* ae = ws_ptr<const ActiveExpert>(w, w.off_active) + a;
    const MoeExpert ex = ws_ptr<const MoeExpert>(w, w.off_gweights)[a];
    const uint32_t F = s.inter, H = s.width, ntok = *gp(&ae->ntok);
    const uint32_t row0 = blockIdx.x * kRowsPerBlock;
    const uint32_t nrows = H - row0 < kRowsPerBlock ? H - row0 : kRowsPerBlock;
    const uint64_t rb = row_bytes<FMT>(F);
    const float* h = ws_ptr<const float>(w, w.off_h);
    const float* xs[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) xs[t] = h + ((uint64_t)a * NT + t) * F;
    rows_dot_slots<FMT>(ex.down + (uint64_t)row0 * rb, rb, nrows, F, xs, ntok, ld);
    const uint32_t tid = threadIdx.x, rr = tid / NT, t = tid % NT;
    if (tid < kRowsPerBlock * NT && rr < nrows && t < ntok)
        *gp(ws_ptr<float>(w, w.off_ypart) + ((uint64_t)a * NT + t) * H + row0 + rr) = ld.sum[rr][t];
}

// Whether rows of `cols` columns of this type fit the kernels' 32-bit offsets.
template <uint32_t FMT>
bool rows_fit(uint32_t cols) {
    return (uint64_t)(cols / Fmt<FMT>::be) * Fmt<FMT>::bb + 64u <= 0xffffffffull;
}

template <uint32_t FMT>
hipError_t dequant_fmt(const vl_tiled_layout& L, const uint8_t* w, float* out, hipStream_t st) {
    if (!rows_fit<FMT>(L.cols)) return hipErrorInvalidValue;
    const uint64_t n = (uint64_t)L.rows * ((L.cols + 7u) / 8u);
    hipLaunchKernelGGL(k_gguf_dequant<FMT>, dim3((uint32_t)((n + 255u) / 256u)), dim3(256), 0, st, L, w, out);
    return hipGetLastError();
}

template <uint32_t FMT, int NT>
hipError_t matvec_nt(const vl_tiled_layout& L, const uint8_t* w, const float* x, uint32_t tokens,
                     float* y, uint32_t* status, hipStream_t st) {
    hipLaunchKernelGGL((k_gguf_matvec<FMT, NT>), dim3((L.rows + kRowsPerBlock - 1u) / kRowsPerBlock), dim3(256), 0, st, L, w, x,
                       tokens, y, status);
    return hipGetLastError();
}

template <uint32_t FMT>
hipError_t matvec_fmt(const vl_tiled_layout& L, const uint8_t* w, const float* x, uint32_t tokens,
                      float* y, uint32_t* status, hipStream_t st) {
    if (!rows_fit<FMT>(L.cols)) return hipErrorInvalidValue;
    switch (limb_slots(tokens)) {
        case 1: return matvec_nt<FMT, 1>(L, w, x, tokens, y, status, st);
        case 2: return matvec_nt<FMT, 2>(L, w, x, tokens, y, status, st);
        case 4: return matvec_nt<FMT, 4>(L, w, x, tokens, y, status, st);
        default: return matvec_nt<FMT, 8>(L, w, x, tokens, y, status, st);
    }
}

template <uint32_t FMT>
hipError_t moe_gateup_fmt(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w, hipStream_t st) {
    if (!rows_fit<FMT>(s.width)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_gguf_moe_gateup<FMT>, dim3((s.inter + kRowsPerBlock - 1u) / kRowsPerBlock, w.max_active),
                       dim3(256), 0, st, s, in, w);
    return hipGetLastError();
}

template <uint32_t FMT>
hipError_t moe_down_fmt(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w, hipStream_t st) {
    if (!rows_fit<FMT>(s.inter)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_gguf_moe_down<FMT>, dim3((s.width + kRowsPerBlock - 1u) / kRowsPerBlock, w.max_active),
                       dim3(256), 0, st, s, in, w);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gguf_moe_gateup(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                                  hipStream_t stream) {
    switch (s.gate_type) {
        case VL_TYPE_Q4_K: return moe_gateup_fmt<VL_TYPE_Q4_K>(s, in, w, stream);
        case VL_TYPE_Q5_K: return moe_gateup_fmt<VL_TYPE_Q5_K>(s, in, w, stream);
        case VL_TYPE_Q6_K: return moe_gateup_fmt<VL_TYPE_Q6_K>(s, in, w, stream);
        case VL_TYPE_IQ2_S: return moe_gateup_fmt<VL_TYPE_IQ2_S>(s, in, w, stream);
        case VL_TYPE_MXFP4: return moe_gateup_fmt<VL_TYPE_MXFP4>(s, in, w, stream);
        case VL_TYPE_BF16: return moe_gateup_fmt<VL_TYPE_BF16>(s, in, w, stream);
        case VL_TYPE_F32: return moe_gateup_fmt<VL_TYPE_F32>(s, in, w, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gguf_moe_down(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                                hipStream_t stream) {
    switch (s.down_type) {
        case VL_TYPE_Q4_K: return moe_down_fmt<VL_TYPE_Q4_K>(s, in, w, stream);
        case VL_TYPE_Q5_K: return moe_down_fmt<VL_TYPE_Q5_K>(s, in, w, stream);
        case VL_TYPE_Q6_K: return moe_down_fmt<VL_TYPE_Q6_K>(s, in, w, stream);
        case VL_TYPE_IQ2_S: return moe_down_fmt<VL_TYPE_IQ2_S>(s, in, w, stream);
        case VL_TYPE_MXFP4: return moe_down_fmt<VL_TYPE_MXFP4>(s, in, w, stream);
        case VL_TYPE_BF16: return moe_down_fmt<VL_TYPE_BF16>(s, in, w, stream);
        case VL_TYPE_F32: return moe_down_fmt<VL_TYPE_F32>(s, in, w, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gguf_copy_rows(const vl_tiled_layout& L, const uint8_t* gguf_row0, uint8_t* dst,
                                 uint32_t row0, uint32_t row1, hipStream_t stream) {
    if (row0 >= row1 || row1 > L.rows) return hipErrorInvalidValue;
    const uint64_t rb = L.gguf_bytes / L.rows;
    return hipMemcpyAsync(dst + (uint64_t)row0 * rb, gguf_row0, (uint64_t)(row1 - row0) * rb,
                          hipMemcpyDeviceToDevice, stream);
}

hipError_t launch_gguf_dequant(const vl_tiled_layout& L, const uint8_t* w, float* out, hipStream_t stream) {
    switch (L.type) {
        case VL_TYPE_Q4_K: return dequant_fmt<VL_TYPE_Q4_K>(L, w, out, stream);
        case VL_TYPE_Q5_K: return dequant_fmt<VL_TYPE_Q5_K>(L, w, out, stream);
        case VL_TYPE_Q6_K: return dequant_fmt<VL_TYPE_Q6_K>(L, w, out, stream);
        case VL_TYPE_IQ2_S: return dequant_fmt<VL_TYPE_IQ2_S>(L, w, out, stream);
        case VL_TYPE_MXFP4: return dequant_fmt<VL_TYPE_MXFP4>(L, w, out, stream);
        case VL_TYPE_BF16: return dequant_fmt<VL_TYPE_BF16>(L, w, out, stream);
        case VL_TYPE_F32: return dequant_fmt<VL_TYPE_F32>(L, w, out, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gguf_matvec(const vl_tiled_layout& L, const uint8_t* w, const float* x, uint32_t tokens,
                              float* y, uint8_t* workspace, hipStream_t stream) {
    if (tokens == 0 || tokens > 8) return hipErrorInvalidValue;
    uint32_t* status = reinterpret_cast<uint32_t*>(workspace);
    hipLaunchKernelGGL(k_gguf_clear_status, dim3(1), dim3(64), 0, stream, status);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    switch (L.type) {
        case VL_TYPE_Q4_K: return matvec_fmt<VL_TYPE_Q4_K>(L, w, x, tokens, y, status, stream);
        case VL_TYPE_Q5_K: return matvec_fmt<VL_TYPE_Q5_K>(L, w, x, tokens, y, status, stream);
        case VL_TYPE_Q6_K: return matvec_fmt<VL_TYPE_Q6_K>(L, w, x, tokens, y, status, stream);
        case VL_TYPE_IQ2_S: return matvec_fmt<VL_TYPE_IQ2_S>(L, w, x, tokens, y, status, stream);
        case VL_TYPE_MXFP4: return matvec_fmt<VL_TYPE_MXFP4>(L, w, x, tokens, y, status, stream);
        case VL_TYPE_BF16: return matvec_fmt<VL_TYPE_BF16>(L, w, x, tokens, y, status, stream);
        case VL_TYPE_F32: return matvec_fmt<VL_TYPE_F32>(L, w, x, tokens, y, status, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace vl
