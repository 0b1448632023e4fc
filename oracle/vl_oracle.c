/* CPU oracle for the quantized routed-expert path. TEST INFRASTRUCTURE ONLY: the checker for
 * the HIP product, never part of it. See vl_oracle.h for what pins each function.
 *
 * Built with -ffp-contract=off and no fast-math, the reference's own host FP semantics
 * (cmake/VastloomWarnings.cmake): every product and sum below rounds exactly once, in the
 * order written.
 */
#include "vl_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "../vastloom_amd/csrc/vl_codebooks_expand.h"

/* ----------------------------------------------------------------------------------------- */
/* Codebooks and scalar helpers                                                                */
/* ----------------------------------------------------------------------------------------- */

static vl_expanded_codebooks g_books;
static int g_books_ok = -1;
static pthread_once_t g_books_once = PTHREAD_ONCE_INIT;

static void books_init(void) {
    vl_codebooks_expand(&g_books);
    g_books_ok = vl_codebooks_fingerprints_ok(&g_books);
}

int vlo_codebooks_ok(void) {
    pthread_once(&g_books_once, books_init);
    return g_books_ok;
}

/* Exact binary16 -> binary32, subnormals renormalised (ggml_quantization.cpp:101-124). */
float vlo_fp16_to_f32(uint16_t value) {
    uint32_t sign = (uint32_t)(value & 0x8000u) << 16;
    uint32_t exponent = (value >> 10) & 0x1fu;
    uint32_t mantissa = value & 0x3ffu;
    uint32_t bits = sign;
    if (exponent == 0u) {
        if (mantissa != 0u) {
            uint32_t e = 113u;
            while ((mantissa & 0x400u) == 0u) {
                mantissa <<= 1;
                --e;
            }
            bits |= e << 23;
            bits |= (mantissa & 0x3ffu) << 13;
        }
    } else if (exponent == 0x1fu) {
        bits |= 0x7f800000u | (mantissa << 13);
    } else {
        bits |= (exponent + 112u) << 23;
        bits |= mantissa << 13;
    }
    float out;
    memcpy(&out, &bits, sizeof out);
    return out;
}

static inline uint16_t le16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t le32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* Eight sign bits for one 8-lane sub-block: seven stored, the eighth makes the parity even
 * (ggml_quantization.cpp:266-269, :350-353). */
static inline unsigned sign_byte(uint32_t seven) {
    return seven | ((unsigned)(__builtin_popcount(seven) & 1) << 7);
}

/* ----------------------------------------------------------------------------------------- */
/* Block decoders: one block into float[block_elements]                                       */
/* ----------------------------------------------------------------------------------------- */

typedef void (*block_decoder)(const uint8_t* block, float* out);

/* Q8_0: 34 bytes -> 32 weights, w = d * (float)int8 (ggml_quantization.cpp:419-433). */
static void decode_q8_0(const uint8_t* block, float* out) {
    const float d = vlo_fp16_to_f32(le16(block));
    for (int i = 0; i < 32; ++i) out[i] = d * (float)(int8_t)block[2 + i];
}

/* IQ2_XXS: 66 bytes -> 256 weights (ggml_quantization.cpp:250-283). Eight groups of eight
 * bytes: four grid indices, then a word holding four 7-bit sign fields and a 4-bit scale. */
static void decode_iq2_xxs(const uint8_t* block, float* out) {
    const float d = vlo_fp16_to_f32(le16(block));
    for (int g = 0; g < 8; ++g) {
        const uint8_t* group = block + 2 + 8 * g;
        const uint32_t aux = le32(group + 4);
        const float ls = d * (0.5f + (float)(aux >> 28)) * 0.25f;
        for (int s = 0; s < 4; ++s) {
            const uint64_t grid = g_books.iq2xxs[group[s]];
            const unsigned signs = sign_byte((aux >> (7 * s)) & 127u);
            for (int l = 0; l < 8; ++l) {
                const float mag = (float)((grid >> (8 * l)) & 0xffu);
                const float sg = (signs >> l) & 1u ? -1.0f : 1.0f;
                out[32 * g + 8 * s + l] = ls * mag * sg;
            }
        }
    }
}

/* IQ3_XXS: 98 bytes -> 256 weights (ggml_quantization.cpp:336-379). 64 grid-index bytes
 * (two per sub-block, four lanes each), then eight scale/sign words. */
static void decode_iq3_xxs(const uint8_t* block, float* out) {
    const float d = vlo_fp16_to_f32(le16(block));
    const uint8_t* qs = block + 2;
    const uint8_t* words = block + 66;
    for (int g = 0; g < 8; ++g) {
        const uint32_t aux = le32(words + 4 * g);
        const float ls = d * (0.5f + (float)(aux >> 28)) * 0.5f;
        for (int s = 0; s < 4; ++s) {
            const unsigned signs = sign_byte((aux >> (7 * s)) & 127u);
            const uint32_t first = g_books.iq3xxs[qs[8 * g + 2 * s]];
            const uint32_t second = g_books.iq3xxs[qs[8 * g + 2 * s + 1]];
            for (int l = 0; l < 4; ++l) {
                const float s0 = (signs >> l) & 1u ? -1.0f : 1.0f;
                const float s1 = (signs >> (l + 4)) & 1u ? -1.0f : 1.0f;
                out[32 * g + 8 * s + l] = ls * (float)((first >> (8 * l)) & 0xffu) * s0;
                out[32 * g + 8 * s + 4 + l] = ls * (float)((second >> (8 * l)) & 0xffu) * s1;
            }
        }
    }
}

/* IQ1_S: 50 bytes -> 256 weights (ggml_quantization.cpp:217-248). 32 low index bytes, then
 * eight 16-bit words: 3 high index bits per sub-block, a 3-bit scale, and the delta sign. */
static void decode_iq1_s(const uint8_t* block, float* out) {
    const float d = vlo_fp16_to_f32(le16(block));
    const uint8_t* qs = block + 2;
    const uint8_t* qh = block + 34;
    for (int g = 0; g < 8; ++g) {
        const uint16_t h = le16(qh + 2 * g);
        const float ls = d * (float)(2u * ((h >> 12) & 7u) + 1u);
        const float delta = (h & 0x8000u) ? -0.125f : 0.125f;
        for (int s = 0; s < 4; ++s) {
            const unsigned index = qs[4 * g + s] | (((h >> (3 * s)) & 7u) << 8);
            const uint64_t grid = g_books.iq1s[index];
            for (int l = 0; l < 8; ++l) {
                const float q = (float)(int8_t)((grid >> (8 * l)) & 0xffu);
                out[32 * g + 8 * s + l] = ls * (q + delta);
            }
        }
    }
}

/* F32: little-endian float elements, one per "block" (ggml_quantization.cpp:381-417). Used for
 * routers, shared experts stored unquantized, and the float-weight operator fixtures. */
static void decode_f32(const uint8_t* block, float* out) {
    const uint32_t bits = le32(block);
    memcpy(out, &bits, sizeof bits);
}

/* IQ2_S: 82 bytes -> 256 weights (ggml_quantization.cpp:285-334). fp16 d, 32 low index bytes,
 * 32 explicit sign bytes, 8 high-bit bytes (two index bits per sub-block) and 8 scale bytes
 * (low nibble for sub-blocks 0-1 of a group, high nibble for 2-3):
 * w = ((d * (0.5 + nibble)) * 0.25) * grid magnitude * sign. */
static void decode_iq2_s(const uint8_t* block, float* out) {
    const float d = vlo_fp16_to_f32(le16(block));
    const uint8_t* qs = block + 2;
    const uint8_t* signs = block + 34;
    const uint8_t* high = block + 66;
    const uint8_t* scales = block + 74;
    for (unsigned g = 0; g < 8u; ++g) {
        const float ls_low = d * (0.5f + (float)(scales[g] & 15u)) * 0.25f;
        const float ls_high = d * (0.5f + (float)(scales[g] >> 4)) * 0.25f;
        for (unsigned s = 0; s < 4u; ++s) {
            const unsigned index = qs[4u * g + s] | (((unsigned)high[g] >> (2u * s)) & 3u) << 8;
            const uint64_t grid = g_books.iq2s[index];
            const unsigned sg = signs[4u * g + s];
            const float ls = s < 2u ? ls_low : ls_high;
            for (unsigned l = 0; l < 8u; ++l) {
                const float mag = (float)((grid >> (8u * l)) & 0xffu);
                out[32u * g + 8u * s + l] = ls * mag * ((sg >> l) & 1u ? -1.0f : 1.0f);
            }
        }
    }
}

/* The 6-bit scale and minimum of sub-block j of a Q4_K/Q5_K superblock, packed into 12 bytes:
 * bytes 0..3 hold scales 0..3 in their low six bits, bytes 4..7 minimums 0..3 likewise; for
 * j >= 4 the low four bits come from byte j+4 (scale: low nibble, minimum: high nibble) and the
 * top two from the spare high bits of bytes j-4 (scale) and j (minimum)
 * (ggml_quantization.cpp:435-455). */
static void k_scale_min(const uint8_t* s, unsigned j, unsigned* sc, unsigned* mn) {
    if (j < 4u) {
        *sc = s[j] & 63u;
        *mn = s[j + 4u] & 63u;
    } else {
        *sc = (s[j + 4u] & 15u) | ((unsigned)(s[j - 4u] >> 6) << 4);
        *mn = (unsigned)(s[j + 4u] >> 4) | ((unsigned)(s[j] >> 6) << 4);
    }
}

/* Q4_K: 144 bytes -> 256 weights (ggml_quantization.cpp:457-493). fp16 d and dmin, 12 scale
 * bytes, 128 quant bytes; sub-block j (32 weights) takes the low (even j) or high (odd j)
 * nibbles of quant bytes 32*(j/2) .. +31, w = (d*sc) * q - (dmin*m). */
static void decode_q4_k(const uint8_t* block, float* out) {
    const float d = vlo_fp16_to_f32(le16(block)), dmin = vlo_fp16_to_f32(le16(block + 2));
    for (unsigned j = 0; j < 8u; ++j) {
        unsigned sc, mn;
        k_scale_min(block + 4, j, &sc, &mn);
        const float dj = d * (float)sc, mj = dmin * (float)mn;
        const uint8_t* q = block + 16 + 32u * (j / 2u);
        for (unsigned l = 0; l < 32u; ++l)
            out[32u * j + l] = dj * (float)((q[l] >> (4u * (j & 1u))) & 15u) - mj;
    }
}

/* Q5_K: 176 bytes -> 256 weights (ggml_quantization.cpp:495-539). As Q4_K with 32 high-bit
 * bytes before the nibbles: bit j of high byte l adds 16 to weight l of sub-block j. */
static void decode_q5_k(const uint8_t* block, float* out) {
    const float d = vlo_fp16_to_f32(le16(block)), dmin = vlo_fp16_to_f32(le16(block + 2));
    const uint8_t* high = block + 16;
    for (unsigned j = 0; j < 8u; ++j) {
        unsigned sc, mn;
        k_scale_min(block + 4, j, &sc, &mn);
        const float dj = d * (float)sc, mj = dmin * (float)mn;
        const uint8_t* q = block + 48 + 32u * (j / 2u);
        for (unsigned l = 0; l < 32u; ++l) {
            const unsigned v = ((q[l] >> (4u * (j & 1u))) & 15u) + (((high[l] >> j) & 1u) << 4);
            out[32u * j + l] = dj * (float)v - mj;
        }
    }
}

/* Q6_K: 210 bytes -> 256 weights (ggml_quantization.cpp:541-589). 128 low-nibble bytes, 64
 * high-bit bytes (2 bits per weight), 16 int8 scales (one per 16 weights), fp16 d at byte 208.
 * Half h (128 weights) reads low bytes 64h.., high bytes 128+32h.. and scales 192+8h..; its
 * quarter k takes weight l's low bits from low byte l (k = 0, 2) or l+32 (k = 1, 3), low nibble
 * for k < 2 and high nibble after, and bits 2k..2k+1 of high byte l on top;
 * w = (d * scale) * (q - 32). */
static void decode_q6_k(const uint8_t* block, float* out) {
    const float d = vlo_fp16_to_f32(le16(block + 208));
    for (unsigned h = 0; h < 2u; ++h) {
        const uint8_t* low = block + 64u * h;
        const uint8_t* high = block + 128u + 32u * h;
        const int8_t* sc = (const int8_t*)(block + 192u + 8u * h);
        for (unsigned k = 0; k < 4u; ++k) {
            for (unsigned l = 0; l < 32u; ++l) {
                const uint8_t lb = low[l + 32u * (k & 1u)];
                const unsigned nib = k < 2u ? (lb & 15u) : (unsigned)(lb >> 4);
                const int q = (int)(nib | (((unsigned)(high[l] >> (2u * k)) & 3u) << 4)) - 32;
                out[128u * h + 32u * k + l] = d * (float)sc[l / 16u + 2u * k] * (float)q;
            }
        }
    }
}

/* E8M0 block scale of MXFP4 with the one-half factor of the doubled value table folded in:
 * byte v >= 2 is 2^(v-128) (exponent field v-1), bytes 0 and 1 the subnormals 2^-128 and
 * 2^-127 (ggml_quantization.cpp:126-133). */
static float e8m0_half(uint8_t v) {
    const uint32_t bits = v < 2u ? 0x00200000u << v : (uint32_t)(v - 1u) << 23;
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* Twice the E2M1 values, indexed by the 4-bit code (ggml_quantization.cpp:44-47). */
static const int8_t kE2m1Doubled[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

/* MXFP4: 17 bytes -> 32 weights (ggml_quantization.cpp:381-399). One E8M0 scale byte, then
 * 16 bytes whose low nibbles are weights 0..15 and high nibbles weights 16..31. */
static void decode_mxfp4(const uint8_t* block, float* out) {
    const float s = e8m0_half(block[0]);
    for (unsigned i = 0; i < 16u; ++i) {
        out[i] = (float)kE2m1Doubled[block[1 + i] & 15u] * s;
        out[i + 16u] = (float)kE2m1Doubled[block[1 + i] >> 4] * s;
    }
}

/* BF16: the upper half of a binary32 (ggml_quantization.cpp:411-413). */
static void decode_bf16(const uint8_t* block, float* out) {
    const uint32_t bits = (uint32_t)le16(block) << 16;
    memcpy(out, &bits, sizeof bits);
}

/* Whether a block passes the reference's pre-decode validation. */
typedef int (*block_check)(const uint8_t* block);

/* validate_block_scales (ggml_quantization.cpp:206-215): the fp16 scale leads the block. */
static int check_lead_scale(const uint8_t* block) { return isfinite(vlo_fp16_to_f32(le16(block))); }
/* Q4_K/Q5_K validators (:1140-1156, :1180-1196): d and dmin. */
static int check_d_dmin(const uint8_t* block) {
    return isfinite(vlo_fp16_to_f32(le16(block))) && isfinite(vlo_fp16_to_f32(le16(block + 2)));
}
/* Q6_K validator (:1220-1234): d at byte 208. */
static int check_q6_k(const uint8_t* block) { return isfinite(vlo_fp16_to_f32(le16(block + 208))); }
/* validate_mxfp4_blocks (:400-409): every decoded value. */
static int check_mxfp4(const uint8_t* block) {
    float v[32];
    decode_mxfp4(block, v);
    for (int i = 0; i < 32; ++i)
        if (!isfinite(v[i])) return 0;
    return 1;
}
/* validate_dense_values (:856-871): every element of a dense matrix. */
static int check_f32(const uint8_t* block) {
    float v;
    decode_f32(block, &v);
    return isfinite(v);
}
static int check_bf16(const uint8_t* block) {
    float v;
    decode_bf16(block, &v);
    return isfinite(v);
}

/* Block shape, decoder and validator of each storage type (ggml_storage_bytes,
 * ggml_quantization.cpp:1052-1113, and the per-type entry points at :1115-1500). */
static int layout_checked(uint32_t type, size_t* elements, size_t* bytes, block_decoder* decoder,
                          block_check* check) {
    *check = check_lead_scale;
    switch (type) {
        case VLO_F32: *elements = 1; *bytes = 4; *decoder = decode_f32; *check = check_f32; return VLO_OK;
        case VLO_Q8_0: *elements = 32; *bytes = 34; *decoder = decode_q8_0; return VLO_OK;
        case VLO_Q4_K: *elements = 256; *bytes = 144; *decoder = decode_q4_k; *check = check_d_dmin; return VLO_OK;
        case VLO_Q5_K: *elements = 256; *bytes = 176; *decoder = decode_q5_k; *check = check_d_dmin; return VLO_OK;
        case VLO_Q6_K: *elements = 256; *bytes = 210; *decoder = decode_q6_k; *check = check_q6_k; return VLO_OK;
        case VLO_IQ2_XXS: *elements = 256; *bytes = 66; *decoder = decode_iq2_xxs; return VLO_OK;
        case VLO_IQ3_XXS: *elements = 256; *bytes = 98; *decoder = decode_iq3_xxs; return VLO_OK;
        case VLO_IQ1_S: *elements = 256; *bytes = 50; *decoder = decode_iq1_s; return VLO_OK;
        case VLO_IQ2_S: *elements = 256; *bytes = 82; *decoder = decode_iq2_s; return VLO_OK;
        case VLO_BF16: *elements = 1; *bytes = 2; *decoder = decode_bf16; *check = check_bf16; return VLO_OK;
        case VLO_MXFP4: *elements = 32; *bytes = 17; *decoder = decode_mxfp4; *check = check_mxfp4; return VLO_OK;
        default: return VLO_E_UNSUPPORTED;
    }
}

static int layout(uint32_t type, size_t* elements, size_t* bytes, block_decoder* decoder) {
    block_check c;
    return layout_checked(type, elements, bytes, decoder, &c);
}

int vlo_block_layout(uint32_t type, size_t* block_elements, size_t* block_bytes) {
    block_decoder d;
    return layout(type, block_elements, block_bytes, &d);
}

/* checked_matrix_elements + checked_encoded_bytes (ggml_quantization.cpp:175-204). */
static int checked_bytes(size_t rows, size_t cols, size_t block_elements, size_t block_bytes,
                         size_t max_elements, size_t* out) {
    if (max_elements == 0 || rows == 0 || cols == 0 || cols % block_elements != 0)
        return VLO_E_INVALID_ARGUMENT;
    if (rows > max_elements / cols) return VLO_E_RESOURCE_EXHAUSTED;
    *out = rows * cols / block_elements * block_bytes;
    return VLO_OK;
}

int vlo_storage_bytes(uint32_t type, size_t rows, size_t cols, size_t max_elements, size_t* bytes) {
    size_t be, bb;
    block_decoder d;
    int st = layout(type, &be, &bb, &d);
    if (st) return st;
    return checked_bytes(rows, cols, be, bb, max_elements, bytes);
}

/* The type's pre-decode validation over every block of an encoded span. */
static int blocks_valid(uint32_t type, const uint8_t* encoded, size_t bytes) {
    size_t be, bb;
    block_decoder d;
    block_check check;
    if (layout_checked(type, &be, &bb, &d, &check)) return 0;
    for (size_t off = 0; off < bytes; off += bb)
        if (!check(encoded + off)) return 0;
    return 1;
}

int vlo_dequantize(uint32_t type, const uint8_t* encoded, size_t encoded_bytes, float* out,
                   size_t out_elements, size_t max_elements) {
    vlo_codebooks_ok();
    size_t be, bb;
    block_decoder decode;
    int st = layout(type, &be, &bb, &decode);
    if (st) return st;
    /* dequantize_blocked (ggml_quantization.cpp:601-628). */
    if (out_elements == 0 || out_elements % be != 0 || out_elements > max_elements)
        return VLO_E_INVALID_ARGUMENT;
    if (encoded_bytes != out_elements / be * bb) return VLO_E_INVALID_FORMAT;
    if (!blocks_valid(type, encoded, encoded_bytes)) return VLO_E_INVALID_FORMAT;
    for (size_t b = 0; b < out_elements / be; ++b) decode(encoded + b * bb, out + b * be);
    return VLO_OK;
}

/* dequantize_ggml_row_f32 (ggml_quantization.cpp:1536-1583). */
int vlo_dequantize_row(uint32_t type, const uint8_t* encoded, size_t encoded_bytes, size_t rows,
                       size_t cols, size_t row, float* out, size_t out_elements) {
    size_t total, row_bytes;
    if (row >= rows || out_elements != cols) return VLO_E_INVALID_ARGUMENT;
    int st = vlo_storage_bytes(type, rows, cols, VLO_DEFAULT_MAX_ELEMENTS, &total);
    if (st) return st;
    if (encoded_bytes != total) return VLO_E_INVALID_FORMAT;
    st = vlo_storage_bytes(type, 1, cols, cols, &row_bytes);
    if (st) return st;
    return vlo_dequantize(type, encoded + row * row_bytes, row_bytes, out, cols,
                          VLO_DEFAULT_MAX_ELEMENTS);
}

/* ----------------------------------------------------------------------------------------- */
/* Matvec: per row, blocks in order, lanes in order, sum += (double)w * (double)x             */
/* ----------------------------------------------------------------------------------------- */

typedef struct row_job {
    const uint8_t* encoded;
    size_t first, last, blocks_per_row, be, bb;
    block_decoder decode;
    const float* x;
    float* y;
    int status;
} row_job;

/* The per-row loop of matvec_blocked (ggml_quantization.cpp:793-817). */
static void* run_rows(void* arg) {
    row_job* job = (row_job*)arg;
    float decoded[256];
    for (size_t r = job->first; r < job->last; ++r) {
        double sum = 0.0;
        for (size_t b = 0; b < job->blocks_per_row; ++b) {
            job->decode(job->encoded + (r * job->blocks_per_row + b) * job->bb, decoded);
            const float* xs = job->x + b * job->be;
            for (size_t c = 0; c < job->be; ++c) sum += (double)decoded[c] * (double)xs[c];
        }
        const float v = (float)sum;
        if (!isfinite(v)) {
            job->status = VLO_E_INVALID_FORMAT;
            return NULL;
        }
        job->y[r] = v;
    }
    return NULL;
}

int vlo_matvec(uint32_t type, const uint8_t* encoded, size_t encoded_bytes, size_t rows,
               size_t cols, const float* x, size_t x_len, float* y, size_t y_len,
               size_t max_elements, unsigned max_threads) {
    vlo_codebooks_ok();
    size_t be, bb, need;
    block_decoder decode;
    int st = layout(type, &be, &bb, &decode);
    if (st) return st;
    st = checked_bytes(rows, cols, be, bb, max_elements, &need);
    if (st) return st;
    if (encoded_bytes != need || x_len != cols || y_len != rows) return VLO_E_INVALID_ARGUMENT;
    for (size_t i = 0; i < cols; ++i)
        if (!isfinite(x[i])) return VLO_E_INVALID_ARGUMENT;
    if (!blocks_valid(type, encoded, encoded_bytes)) return VLO_E_INVALID_FORMAT;

    /* Computed into scratch and published on success, as matvec_ggml_f32_transactional
     * (ggml_quantization.cpp:1585-1676) does for every graph call. */
    float* scratch = (float*)malloc(rows * sizeof(float));
    if (!scratch) return VLO_E_RESOURCE_EXHAUSTED;

    /* Row split of matvec_blocked (:819-853): min(rows / 64, threads) workers, contiguous
     * rows each. IQ1_S and IQ3_XXS never split (:1331-1458). Results do not depend on it. */
    unsigned workers = max_threads ? max_threads : 1u;
    if (rows / 64 < workers) workers = (unsigned)(rows / 64);
    if (workers < 1u) workers = 1u;
    if (type == VLO_IQ1_S || type == VLO_IQ3_XXS) workers = 1u;
    if (workers > 64u) workers = 64u;

    row_job jobs[64];
    pthread_t threads[64];
    const size_t per = (rows + workers - 1) / workers;
    for (unsigned w = 0; w < workers; ++w) {
        size_t first = (size_t)w * per < rows ? (size_t)w * per : rows;
        size_t last = first + per < rows ? first + per : rows;
        jobs[w] = (row_job){encoded, first, last, cols / be, be, bb, decode, x, scratch, VLO_OK};
    }
    unsigned started = 0;
    for (unsigned w = 1; w < workers; ++w) {
        if (pthread_create(&threads[w], NULL, run_rows, &jobs[w]) != 0) break;
        started = w;
    }
    run_rows(&jobs[0]);
    for (unsigned w = 1; w <= started; ++w) pthread_join(threads[w], NULL);
    for (unsigned w = started + 1; w < workers; ++w) run_rows(&jobs[w]);
    for (unsigned w = 0; w < workers; ++w)
        if (jobs[w].status) st = jobs[w].status;
    if (!st) memcpy(y, scratch, rows * sizeof(float));
    free(scratch);
    return st;
}

static int matrix_matvec(const vlo_matrix* m, size_t rows, size_t cols, const float* x, float* y,
                         unsigned threads) {
    return vlo_matvec(m->type, m->data, m->bytes, rows, cols, x, cols, y, rows,
                      VLO_DEFAULT_MAX_ELEMENTS, threads);
}

/* ----------------------------------------------------------------------------------------- */
/* Expert FFNs                                                                                  */
/* ----------------------------------------------------------------------------------------- */

/* routed_expert_iq1_s_iq3_xxs_f32 (ggml_quantization.cpp:1678-1745): IQ1_S gate and up, f32
 * g / (1 + expf(-g)) * u with no clamp and no route weight, IQ3_XXS down. */
int vlo_routed_expert_iq1s_iq3xxs(const vlo_matrix* gate, const vlo_matrix* up,
                                  const vlo_matrix* down, size_t width, size_t expert_width,
                                  const float* x, float* y) {
    if (width == 0 || expert_width == 0) return VLO_E_INVALID_ARGUMENT;
    if (gate->type != VLO_IQ1_S || up->type != VLO_IQ1_S || down->type != VLO_IQ3_XXS)
        return VLO_E_INVALID_ARGUMENT;
    float* g = (float*)malloc(expert_width * sizeof(float));
    float* u = (float*)malloc(expert_width * sizeof(float));
    float* out = (float*)malloc(width * sizeof(float));
    int st = (g && u && out) ? VLO_OK : VLO_E_RESOURCE_EXHAUSTED;
    if (!st) st = matrix_matvec(gate, expert_width, width, x, g, 1);
    if (!st) st = matrix_matvec(up, expert_width, width, x, u, 1);
    for (size_t i = 0; !st && i < expert_width; ++i) {
        const float a = g[i] / (1.0f + expf(-g[i])) * u[i];
        if (!isfinite(a)) st = VLO_E_INVALID_FORMAT;
        g[i] = a;
    }
    if (!st) st = matrix_matvec(down, width, expert_width, g, out, 1);
    if (!st) memcpy(y, out, width * sizeof(float));
    free(g);
    free(u);
    free(out);
    return st;
}

/* execute_expert (deepseek_v4_graph.cpp:1826-1894): w1 (gate) and w3 (up) per token row, the
 * SwiGLU in float64 with the optional clamp (gate capped above, up clamped both ways) and the
 * route weight applied before the down projection w2. routing == NULL means no route weight
 * (the shared expert). */
int vlo_expert_deepseek(const vlo_matrix* w1, const vlo_matrix* w3, const vlo_matrix* w2,
                        size_t width, size_t intermediate, const float* x, size_t tokens,
                        const float* routing, float swiglu_limit, float* y, unsigned threads) {
    if (tokens == 0 || !isfinite(swiglu_limit) || swiglu_limit < 0.0f)
        return VLO_E_INVALID_ARGUMENT;
    if (routing)
        for (size_t t = 0; t < tokens; ++t)
            if (!isfinite(routing[t])) return VLO_E_INVALID_ARGUMENT;
    float* g = (float*)malloc(intermediate * sizeof(float));
    float* u = (float*)malloc(intermediate * sizeof(float));
    float* out = (float*)malloc(tokens * width * sizeof(float));
    int st = (g && u && out) ? VLO_OK : VLO_E_RESOURCE_EXHAUSTED;
    for (size_t t = 0; !st && t < tokens; ++t) {
        const float* xt = x + t * width;
        st = matrix_matvec(w1, intermediate, width, xt, g, threads);
        if (!st) st = matrix_matvec(w3, intermediate, width, xt, u, threads);
        for (size_t c = 0; !st && c < intermediate; ++c) {
            double gv = (double)g[c];
            double uv = (double)u[c];
            if (swiglu_limit > 0.0f) {
                const double lim = (double)swiglu_limit;
                gv = gv < lim ? gv : lim;
                uv = uv < -lim ? -lim : (uv > lim ? lim : uv);
            }
            double v = gv / (1.0 + exp(-gv)) * uv;
            if (routing) v *= (double)routing[t];
            g[c] = (float)v;
            if (!isfinite(g[c])) st = VLO_E_INVALID_FORMAT;
        }
        if (!st) st = matrix_matvec(w2, width, intermediate, g, out + t * width, threads);
    }
    if (!st) memcpy(y, out, tokens * width * sizeof(float));
    free(g);
    free(u);
    free(out);
    return st;
}

/* sigmoid_f / silu_f (qwen3_8_flash_next_reference.cpp:244-255), float throughout. */
float vlo_silu_f(float v) {
    float s;
    if (v >= 0.0f) {
        s = 1.0f / (1.0f + expf(-v));
    } else {
        const float z = expf(v);
        s = z / (1.0f + z);
    }
    return v * s;
}

/* qwen38_expert_mlp_q8 (qwen3_8_flash_next_reference.cpp:1317-1342) over linear_from_q8
 * (:352-399): the weight is (float)q * d, the same value the Q8_0 decoder produces, and every
 * row keeps its float64 column-order sum, so the matvec is the shared one. */
int vlo_expert_qwen(const vlo_matrix* gate, const vlo_matrix* up, const vlo_matrix* down,
                    size_t width, size_t intermediate, const float* x, float* y,
                    unsigned threads) {
    if (width == 0 || intermediate == 0) return VLO_E_INVALID_ARGUMENT;
    float* g = (float*)malloc(intermediate * sizeof(float));
    float* u = (float*)malloc(intermediate * sizeof(float));
    float* out = (float*)malloc(width * sizeof(float));
    int st = (g && u && out) ? VLO_OK : VLO_E_RESOURCE_EXHAUSTED;
    if (!st) st = matrix_matvec(gate, intermediate, width, x, g, threads);
    if (!st) st = matrix_matvec(up, intermediate, width, x, u, threads);
    for (size_t i = 0; !st && i < intermediate; ++i) g[i] = vlo_silu_f(g[i]) * u[i];
    if (!st) st = matrix_matvec(down, width, intermediate, g, out, threads);
    if (!st) memcpy(y, out, width * sizeof(float));
    free(g);
    free(u);
    free(out);
    return st;
}

/* ----------------------------------------------------------------------------------------- */
/* Routing                                                                                      */
/* ----------------------------------------------------------------------------------------- */

/* sqrt(softplus(x)) in float64 (deepseek_v4_reference.cpp:65-69). */
float vlo_sqrt_softplus(float value) {
    const double p = (double)value;
    const double sp = (p > 0.0 ? p : 0.0) + log1p(exp(-fabs(p)));
    return (float)sqrt(sp);
}

/* The reference's float64 logistic (deepseek_v4_reference.cpp:71-78). */
float vlo_sigmoid(float value) {
    const double p = (double)value;
    if (p >= 0.0) return (float)(1.0 / (1.0 + exp(-p)));
    const double e = exp(p);
    return (float)(e / (1.0 + e));
}

/* Gate logits: float64 accumulation per output, one rounding (linear_f,
 * qwen3_8_flash_next_reference.cpp:311-345; deepseek gate_logits likewise). */
int vlo_linear_f64(const float* weight, const float* x, size_t tokens, size_t in_width,
                   size_t out_width, float* out) {
    if (tokens == 0 || in_width == 0 || out_width == 0) return VLO_E_INVALID_ARGUMENT;
    for (size_t t = 0; t < tokens; ++t)
        for (size_t o = 0; o < out_width; ++o) {
            double acc = 0.0;
            const float* w = weight + o * in_width;
            const float* xt = x + t * in_width;
            for (size_t i = 0; i < in_width; ++i) acc += (double)w[i] * (double)xt[i];
            out[t * out_width + o] = (float)acc;
        }
    return VLO_OK;
}

static float score(float logit, int fn) {
    return fn == VLO_SCORE_SIGMOID ? vlo_sigmoid(logit) : vlo_sqrt_softplus(logit);
}

/* route_from_indices (deepseek_v4_reference.cpp:80-121): weights are the selected scores over
 * their float64 sum, times the route scale, each rounded once to float. */
static int weights_from_indices(const float* scores, const uint32_t* indices, size_t tokens,
                                size_t experts, size_t top_k, float route_scale,
                                float* weights) {
    if (!isfinite(route_scale) || route_scale <= 0.0f) return VLO_E_INVALID_ARGUMENT;
    for (size_t t = 0; t < tokens; ++t) {
        double sum = 0.0;
        for (size_t s = 0; s < top_k; ++s) {
            const uint32_t e = indices[t * top_k + s];
            if (e >= experts) return VLO_E_INVALID_ARGUMENT;
            sum += (double)scores[t * experts + e];
        }
        if (!isfinite(sum) || sum <= 0.0) return VLO_E_INVALID_ARGUMENT;
        for (size_t s = 0; s < top_k; ++s) {
            const double v = (double)scores[t * experts + indices[t * top_k + s]];
            weights[t * top_k + s] = (float)(v / sum * (double)route_scale);
        }
    }
    return VLO_OK;
}

static float* activate(const float* logits, size_t n, int fn) {
    float* scores = (float*)malloc(n * sizeof(float));
    if (!scores) return NULL;
    for (size_t i = 0; i < n; ++i) scores[i] = score(logits[i], fn);
    return scores;
}

static int logits_finite(const float* logits, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!isfinite(logits[i])) return 0;
    return 1;
}

/* deepseek_v4_route_learned_logits (deepseek_v4_reference.cpp:223-255): top-k of
 * score + bias, ties to the lower expert id; weights from the unbiased scores. */
int vlo_route_learned(const float* logits, const float* bias, size_t tokens, size_t experts,
                      size_t top_k, float route_scale, int score_fn, uint32_t* indices,
                      float* weights) {
    if (top_k == 0 || top_k > experts || experts == 0 || tokens == 0)
        return VLO_E_INVALID_ARGUMENT;
    if (!logits_finite(logits, tokens * experts)) return VLO_E_INVALID_ARGUMENT;
    if (bias && !logits_finite(bias, experts)) return VLO_E_INVALID_ARGUMENT;
    float* scores = activate(logits, tokens * experts, score_fn);
    if (!scores) return VLO_E_RESOURCE_EXHAUSTED;
    unsigned char* taken = (unsigned char*)malloc(experts);
    if (!taken) {
        free(scores);
        return VLO_E_RESOURCE_EXHAUSTED;
    }
    for (size_t t = 0; t < tokens; ++t) {
        memset(taken, 0, experts);
        for (size_t s = 0; s < top_k; ++s) {
            size_t best = experts;
            float best_key = 0.0f;
            for (size_t e = 0; e < experts; ++e) {
                if (taken[e]) continue;
                const float key = scores[t * experts + e] + (bias ? bias[e] : 0.0f);
                if (best == experts || key > best_key) {
                    best = e;
                    best_key = key;
                }
            }
            taken[best] = 1;
            indices[t * top_k + s] = (uint32_t)best;
        }
    }
    int st = weights_from_indices(scores, indices, tokens, experts, top_k, route_scale, weights);
    free(taken);
    free(scores);
    return st;
}

/* deepseek_v4_route_hash_logits (deepseek_v4_reference.cpp:275-307): the token's row of the
 * table picks the experts, the gate scores weight them. */
int vlo_route_hash(const float* logits, const uint32_t* token_ids, const uint32_t* table,
                   size_t tokens, size_t vocabulary, size_t experts, size_t top_k,
                   float route_scale, int score_fn, uint32_t* indices, float* weights) {
    if (top_k == 0 || top_k > experts || tokens == 0 || vocabulary == 0 || experts == 0)
        return VLO_E_INVALID_ARGUMENT;
    if (!logits_finite(logits, tokens * experts)) return VLO_E_INVALID_ARGUMENT;
    for (size_t t = 0; t < tokens; ++t) {
        if (token_ids[t] >= vocabulary) return VLO_E_INVALID_ARGUMENT;
        for (size_t s = 0; s < top_k; ++s)
            indices[t * top_k + s] = table[(size_t)token_ids[t] * top_k + s];
    }
    float* scores = activate(logits, tokens * experts, score_fn);
    if (!scores) return VLO_E_RESOURCE_EXHAUSTED;
    int st = weights_from_indices(scores, indices, tokens, experts, top_k, route_scale, weights);
    free(scores);
    return st;
}

/* qwen38_moe_route after its logits (qwen3_8_flash_next_reference.cpp:1198-1239): float64
 * softmax, descending probability with ties to the lower id, optional renormalisation of the
 * top-k by 1 / sum as (float)((double)(float)p * scale). */
int vlo_route_softmax(const float* logits, size_t experts, size_t top_k, int renormalize,
                      uint32_t* indices, float* weights) {
    if (experts == 0 || top_k == 0 || top_k > experts) return VLO_E_INVALID_ARGUMENT;
    double max_l = (double)logits[0];
    for (size_t e = 0; e < experts; ++e)
        if ((double)logits[e] > max_l) max_l = (double)logits[e];
    double* probs = (double*)malloc(experts * sizeof(double));
    unsigned char* taken = (unsigned char*)calloc(experts, 1);
    if (!probs || !taken) {
        free(probs);
        free(taken);
        return VLO_E_RESOURCE_EXHAUSTED;
    }
    double sum = 0.0;
    for (size_t e = 0; e < experts; ++e) {
        probs[e] = exp((double)logits[e] - max_l);
        sum += probs[e];
    }
    const double inv = sum > 0.0 ? 1.0 / sum : 0.0;
    for (size_t e = 0; e < experts; ++e) probs[e] = probs[e] * inv;
    double top_sum = 0.0;
    for (size_t s = 0; s < top_k; ++s) {
        size_t best = experts;
        for (size_t e = 0; e < experts; ++e)
            if (!taken[e] && (best == experts || probs[e] > probs[best])) best = e;
        taken[best] = 1;
        indices[s] = (uint32_t)best;
        weights[s] = (float)probs[best];
        top_sum += probs[best];
    }
    if (renormalize && top_sum > 0.0) {
        const double scale = 1.0 / top_sum;
        for (size_t s = 0; s < top_k; ++s) weights[s] = (float)((double)weights[s] * scale);
    }
    free(probs);
    free(taken);
    return VLO_OK;
}

/* ----------------------------------------------------------------------------------------- */
/* MoE layers                                                                                   */
/* ----------------------------------------------------------------------------------------- */

/* moe_forward's expert loop and combine (deepseek_v4_graph.cpp:2129-2266): ascending expert
 * id, then token, then slot; each routed output added in float; the shared expert (computed
 * without a route weight) added last. expert_matrices holds w1, w3, w2 per expert. */
int vlo_moe_deepseek(const float* x, size_t tokens, size_t width, size_t intermediate,
                     size_t experts, size_t top_k, const uint32_t* indices,
                     const float* weights, const vlo_matrix* expert_matrices,
                     const vlo_matrix* shared, float routed_limit, float shared_limit,
                     float* out, unsigned threads) {
    if (tokens == 0 || width == 0 || experts == 0 || top_k == 0) return VLO_E_INVALID_ARGUMENT;
    for (size_t i = 0; i < tokens * top_k; ++i)
        if (indices[i] >= experts) return VLO_E_INVALID_FORMAT;
    float* acc = (float*)calloc(tokens * width, sizeof(float));
    float* y = (float*)malloc(tokens * width * sizeof(float));
    int st = (acc && y) ? VLO_OK : VLO_E_RESOURCE_EXHAUSTED;
    for (size_t e = 0; !st && e < experts; ++e) {
        const vlo_matrix* m = expert_matrices + 3 * e;
        for (size_t t = 0; !st && t < tokens; ++t)
            for (size_t s = 0; !st && s < top_k; ++s) {
                if (indices[t * top_k + s] != e) continue;
                st = vlo_expert_deepseek(&m[0], &m[1], &m[2], width, intermediate, x + t * width,
                                         1, &weights[t * top_k + s], routed_limit, y, threads);
                for (size_t c = 0; !st && c < width; ++c) acc[t * width + c] += y[c];
            }
    }
    if (!st && shared) {
        st = vlo_expert_deepseek(&shared[0], &shared[1], &shared[2], width, intermediate, x,
                                 tokens, NULL, shared_limit, y, threads);
        for (size_t i = 0; !st && i < tokens * width; ++i) acc[i] += y[i];
    }
    for (size_t i = 0; !st && i < tokens * width; ++i)
        if (!isfinite(acc[i])) st = VLO_E_INVALID_FORMAT;
    if (!st) memcpy(out, acc, tokens * width * sizeof(float));
    free(acc);
    free(y);
    return st;
}

/* qwen38_moe_block (qwen3_8_flash_next_reference.cpp:1377-1421) and the CLI's Q8_0 combine
 * (src/cli/main.cpp:2600-2615): out[d] += y[d] * w in route-slot order, then the shared
 * expert. One token. expert_matrices holds gate, up, down per expert. */
int vlo_moe_qwen(const float* x, size_t width, size_t intermediate, size_t experts,
                 size_t top_k, const uint32_t* indices, const float* weights,
                 const vlo_matrix* expert_matrices, const vlo_matrix* shared, float* out,
                 unsigned threads) {
    if (width == 0 || experts == 0 || top_k == 0) return VLO_E_INVALID_ARGUMENT;
    float* acc = (float*)calloc(width, sizeof(float));
    float* y = (float*)malloc(width * sizeof(float));
    int st = (acc && y) ? VLO_OK : VLO_E_RESOURCE_EXHAUSTED;
    for (size_t s = 0; !st && s < top_k; ++s) {
        if (indices[s] >= experts) {
            st = VLO_E_INVALID_ARGUMENT;
            break;
        }
        const vlo_matrix* m = expert_matrices + 3 * indices[s];
        st = vlo_expert_qwen(&m[0], &m[1], &m[2], width, intermediate, x, y, threads);
        for (size_t d = 0; !st && d < width; ++d) acc[d] += y[d] * weights[s];
    }
    if (!st && shared) {
        st = vlo_expert_qwen(&shared[0], &shared[1], &shared[2], width, intermediate, x, y,
                             threads);
        for (size_t d = 0; !st && d < width; ++d) acc[d] += y[d];
    }
    if (!st) memcpy(out, acc, width * sizeof(float));
    free(acc);
    free(y);
    return st;
}
