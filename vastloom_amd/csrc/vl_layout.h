// Device-resident ("tiled") layout of a quantized expert matrix, shared by host and device code.
//
// Q4_K, Q5_K, Q6_K, IQ2_S, MXFP4, BF16 and F32 matrices are not rearranged: they stay in their GGUF bytes
// (vl_type_tiled); everything below describes the four tiled types.
//
// The GGUF block bytes of a matrix are rearranged once, when the matrix becomes resident, into
// planes that the matvec kernels read with aligned 16-byte loads. The rearrangement moves whole
// bit fields and never changes a value: the tiled matrix holds exactly the GGUF bytes (66, 98,
// 50 or 34 per block), plus zero rows when the row count is not a multiple of 32. Rows are
// grouped into tiles of 32 (the N dimension of one 32x32x32 int8 MFMA); a "group" is 32 columns
// (the K of one MFMA): one Q8_0 block, or one eighth of an IQ superblock.
//
// Planes, in order, for a matrix of R rows (Rp = R rounded up to 32, T = Rp/32 tiles), K
// columns, NB = K/256 superblocks and NG = K/32 groups per row; j is the row within its tile:
//
//   IQ2_XXS  P: [T][NB][2 h][32 j][32 B]  half h of row j's superblock (see below)
//            S: [T][NB][32 j] u16           superblock scale d
//   IQ3_XXS  Q: [T][NG/2][32 j][16 B]  two groups' 8 grid-index bytes
//            A: [T][NG/4][32 j][16 B]  four groups' sign/scale words
//            S: [T][NB][32 j] u16
//   IQ1_S    Q: [T][NG/4][32 j][16 B]  four groups' 4 low index bytes
//            H: [T][NB][32 j][16 B]    the superblock's eight 16-bit high words
//            S: [T][NB][32 j] u16
//   Q8_0     Q: [T][NG][32 j][32 B]    the block's 32 int8 quants
//            S: [T][NG][32 j] u16      block scale d
//
// IQ2_XXS half h of a superblock row holds what the MFMA lane that takes K half h of every
// group needs: sub-blocks 2h and 2h+1 of each of the 8 groups, as eight 32-bit words
//   w[q]     q = 0..3: grid bytes of groups 2q and 2q+1: g(2q,2h), g(2q,2h+1), g(2q+1,2h),
//            g(2q+1,2h+1) in bytes 0..3
//   w[4+q]   q = 0..3: the 7-bit sign fields of the same four sub-blocks at bits 0, 7, 14 and
//            21, and at bits 28..31 the 4-bit scale of group 4h+q
// so that each of the 32 lanes of a half-wave loads its own 32 contiguous bytes, and the two
// halves of a row exchange their four scales once per superblock.
#ifndef VL_LAYOUT_H
#define VL_LAYOUT_H

#include <stdint.h>

#define VL_TYPE_F32 0u
#define VL_TYPE_Q8_0 8u
#define VL_TYPE_IQ2_XXS 16u
#define VL_TYPE_IQ3_XXS 18u
#define VL_TYPE_IQ1_S 19u
#define VL_TYPE_Q4_K 12u
#define VL_TYPE_Q5_K 13u
#define VL_TYPE_Q6_K 14u
#define VL_TYPE_IQ2_S 22u
#define VL_TYPE_BF16 30u
#define VL_TYPE_MXFP4 39u

#define VL_TILE_ROWS 32u

#ifdef __HIPCC__
#define VL_HD __host__ __device__
#else
#define VL_HD
#endif

typedef struct vl_tiled_layout {
    uint32_t type;
    uint32_t rows, rows_padded, tiles;
    uint32_t cols, superblocks, groups;
    uint32_t block_elements, block_bytes;
    uint64_t plane0, plane1, plane2;  // byte offsets of the planes
    uint64_t bytes;                   // total tiled bytes
    uint64_t gguf_bytes;              // bytes of the GGUF (untiled) matrix
} vl_tiled_layout;

static inline VL_HD int vl_block_shape(uint32_t type, uint32_t* elements, uint32_t* bytes) {
    switch (type) {
        case VL_TYPE_Q8_0: *elements = 32u; *bytes = 34u; return 1;
        case VL_TYPE_IQ2_XXS: *elements = 256u; *bytes = 66u; return 1;
        case VL_TYPE_IQ3_XXS: *elements = 256u; *bytes = 98u; return 1;
        case VL_TYPE_IQ1_S: *elements = 256u; *bytes = 50u; return 1;
        case VL_TYPE_Q4_K: *elements = 256u; *bytes = 144u; return 1;
        case VL_TYPE_Q5_K: *elements = 256u; *bytes = 176u; return 1;
        case VL_TYPE_Q6_K: *elements = 256u; *bytes = 210u; return 1;
        case VL_TYPE_IQ2_S: *elements = 256u; *bytes = 82u; return 1;
        case VL_TYPE_MXFP4: *elements = 32u; *bytes = 17u; return 1;
        case VL_TYPE_BF16: *elements = 1u; *bytes = 2u; return 1;
        case VL_TYPE_F32: *elements = 1u; *bytes = 4u; return 1;
        default: return 0;
    }
}

// Whether a type is rearranged into the tiled planes above (the types the MFMA matvec and the
// MoE layer kernels read). The other types keep their GGUF bytes unchanged on the device: the
// layout's "tiled" matrix is then the GGUF matrix itself (rows_padded = rows, one plane).
static inline VL_HD int vl_type_tiled(uint32_t type) {
    return type == VL_TYPE_Q8_0 || type == VL_TYPE_IQ2_XXS || type == VL_TYPE_IQ3_XXS ||
           type == VL_TYPE_IQ1_S;
}

// Fills *out; returns 0 for an unsupported type or a column count that is not a whole number
// of blocks.
static inline VL_HD int vl_make_layout(uint32_t type, uint32_t rows, uint32_t cols,
                                       vl_tiled_layout* out) {
    uint32_t be = 0, bb = 0;
    if (!vl_block_shape(type, &be, &bb) || rows == 0 || cols == 0 || cols % be != 0) return 0;
    vl_tiled_layout L;
    L.type = type;
    L.rows = rows;
    L.rows_padded = vl_type_tiled(type) ? (rows + VL_TILE_ROWS - 1u) / VL_TILE_ROWS * VL_TILE_ROWS
                                        : rows;
    L.tiles = L.rows_padded / VL_TILE_ROWS;
    L.cols = cols;
    L.block_elements = be;
    L.block_bytes = bb;
    L.groups = cols / 32u;
    L.superblocks = cols / 256u;
    const uint64_t rp = L.rows_padded;
    L.gguf_bytes = (uint64_t)rows * (cols / be) * bb;
    if (!vl_type_tiled(type)) {
        L.plane0 = L.plane1 = L.plane2 = 0;
        L.bytes = L.gguf_bytes;
        *out = L;
        return 1;
    }
    switch (type) {
        case VL_TYPE_IQ2_XXS:
            L.plane0 = 0;
            L.plane1 = rp * L.superblocks * 64u;
            L.plane2 = L.plane1;
            L.bytes = L.plane1 + rp * L.superblocks * 2u;
            break;
        case VL_TYPE_IQ3_XXS:
            L.plane0 = 0;
            L.plane1 = rp * L.groups * 8u;
            L.plane2 = L.plane1 + rp * L.groups * 4u;
            L.bytes = L.plane2 + rp * L.superblocks * 2u;
            break;
        case VL_TYPE_IQ1_S:
            L.plane0 = 0;
            L.plane1 = rp * L.groups * 4u;
            L.plane2 = L.plane1 + rp * L.superblocks * 16u;
            L.bytes = L.plane2 + rp * L.superblocks * 2u;
            break;
        default: /* Q8_0 */
            L.plane0 = 0;
            L.plane1 = rp * L.groups * 32u;
            L.plane2 = L.plane1;
            L.bytes = L.plane1 + rp * L.groups * 2u;
            break;
    }
    *out = L;
    return 1;
}

#endif  // VL_LAYOUT_H
