// HIP kernels for the quantized routed-expert path on gfx950 (MI355X).
//
//   k_pack          GGUF block bytes -> tiled device layout (vl_layout.h), once per resident matrix
//   k_dequant       tiled matrix -> float32 rows, through the same decoders as the matvec; used to
//                   prove the decode bit-exact against the reference
//   k_prep_limbs    float32 activations -> int8 limbs + per-token exponent (the MFMA A operand)
//   k_qmv           batched quantized matvec: per 32-row tile, int8 32x32x32 MFMA with the
//                   decoded weights as B and up to 8 tokens x 4 limbs as A
//
// Numerics of k_qmv: every product w*x is formed exactly in integers (weights are exact small
// integers times a per-group float factor, activations are 30-bit fixed point per token); each
// group's int32 MFMA result is scaled by the group's integer scale, summed exactly over the
// superblock, converted to float once per superblock, and the four waves' K partials are added
// in a fixed order. The result is deterministic and its error is a few float roundings of the
// row's partial sums, well inside 1e-5 * |w| * |x|.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vl_decode.h"
#include "vl_kernels.h"
#include "vl_layout.h"
#include "vl_tables.h"

namespace vl {

__device__ const DecodeTables g_tables = make_decode_tables();

// ------------------------------------------------------------------------------------------
// Pack: GGUF -> tiled. One thread per (row, superblock) for the IQ formats and per (row,
// block) for Q8_0; padded rows are written as zeros.
// ------------------------------------------------------------------------------------------

__device__ __forceinline__ void copy_bytes(uint8_t* dst, const uint8_t* src, int n, bool zero) {
    for (int i = 0; i < n; ++i) dst[i] = zero ? 0 : src[i];
}

__global__ void k_pack(vl_tiled_layout L, const uint8_t* __restrict__ gguf,
                       uint8_t* __restrict__ out) {
    const uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool q8 = L.type == VL_TYPE_Q8_0;
    const uint32_t units = q8 ? L.groups : L.superblocks;  // blocks per row
    if (id >= (uint64_t)L.rows_padded * units) return;
    const uint32_t r = (uint32_t)(id / units), b = (uint32_t)(id % units);
    const uint32_t t = r / 32u, j = r % 32u;
    const bool pad = r >= L.rows;
    // Padded rows read nothing; their source pointer stays on the first block.
    const uint8_t* src = pad ? gguf : gguf + ((uint64_t)r * units + b) * L.block_bytes;
    const uint32_t NG = L.groups, NB = L.superblocks;
    uint8_t* S = out + L.plane2;
    switch (L.type) {
        case VL_TYPE_IQ2_XXS: {
            S = out + L.plane1;
            for (uint32_t g = 0; g < 8; ++g) {
                const uint32_t G = 8u * b + g;
                uint8_t* dst = out + (((uint64_t)t * (NG / 2) + G / 2) * 32u + j) * 16u + (G % 2) * 8u;
                copy_bytes(dst, src + 2 + 8 * g, 8, pad);
            }
            copy_bytes(S + (((uint64_t)t * NB + b) * 32u + j) * 2u, src, 2, pad);
            break;
        }
        case VL_TYPE_IQ3_XXS: {
            for (uint32_t g = 0; g < 8; ++g) {
                const uint32_t G = 8u * b + g;
                uint8_t* q = out + (((uint64_t)t * (NG / 2) + G / 2) * 32u + j) * 16u + (G % 2) * 8u;
                copy_bytes(q, src + 2 + 8 * g, 8, pad);
                uint8_t* a = out + L.plane1 +
                             (((uint64_t)t * (NG / 4) + G / 4) * 32u + j) * 16u + (G % 4) * 4u;
                copy_bytes(a, src + 66 + 4 * g, 4, pad);
            }
            copy_bytes(S + (((uint64_t)t * NB + b) * 32u + j) * 2u, src, 2, pad);
            break;
        }
        case VL_TYPE_IQ1_S: {
            for (uint32_t g = 0; g < 8; ++g) {
                const uint32_t G = 8u * b + g;
                uint8_t* q = out + (((uint64_t)t * (NG / 4) + G / 4) * 32u + j) * 16u + (G % 4) * 4u;
                copy_bytes(q, src + 2 + 4 * g, 4, pad);
            }
            copy_bytes(out + L.plane1 + (((uint64_t)t * NB + b) * 32u + j) * 16u, src + 34, 16, pad);
            copy_bytes(S + (((uint64_t)t * NB + b) * 32u + j) * 2u, src, 2, pad);
            break;
        }
        default: {  // Q8_0: b is the block (= group) index
            S = out + L.plane1;
            copy_bytes(out + (((uint64_t)t * NG + b) * 32u + j) * 32u, src + 2, 32, pad);
            copy_bytes(S + (((uint64_t)t * NG + b) * 32u + j) * 2u, src, 2, pad);
            break;
        }
    }
}

hipError_t launch_pack(const vl_tiled_layout& L, const uint8_t* gguf, uint8_t* tiled,
                       hipStream_t stream) {
    const uint64_t units = (uint64_t)L.rows_padded * (L.type == VL_TYPE_Q8_0 ? L.groups : L.superblocks);
    const uint32_t block = 256;
    const uint64_t grid = (units + block - 1) / block;
    hipLaunchKernelGGL(k_pack, dim3((uint32_t)grid), dim3(block), 0, stream, L, gguf, tiled);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// Group access: one lane's decoded B fragment, integer group scale and superblock factor.
// ------------------------------------------------------------------------------------------

union LdsTables {
    IqTables2 iq2;
    IqTables3 iq3;
    IqTables1 iq1;
};

template <uint32_t FMT>
__device__ __forceinline__ void load_tables(LdsTables& lds) {
    const int tid = threadIdx.x, nthreads = blockDim.x;
    if (FMT == VL_TYPE_IQ2_XXS) {
        for (int i = tid; i < 256; i += nthreads) lds.iq2.codes[i] = g_tables.iq2_codes[i];
        for (int i = tid; i < 128; i += nthreads) lds.iq2.sign[i] = g_tables.sign_sel[i];
    } else if (FMT == VL_TYPE_IQ3_XXS) {
        for (int i = tid; i < 256; i += nthreads) lds.iq3.pm[i] = g_tables.iq3_pm[i];
        for (int i = tid; i < 128; i += nthreads) lds.iq3.sel[i] = g_tables.iq3_sel[i];
    } else if (FMT == VL_TYPE_IQ1_S) {
        for (int i = tid; i < 2048; i += nthreads) lds.iq1.codes[i] = g_tables.iq1_codes[i];
    }
}

// Register payload of one unit (a superblock for IQ formats, a block for Q8_0) for one lane.
struct UnitPayload {
    uint4 p[4];
    uint16_t d;
};

template <uint32_t FMT>
__device__ __forceinline__ void load_unit(const vl_tiled_layout& L, const uint8_t* __restrict__ w,
                                          uint32_t t, uint32_t n, int hh, uint32_t u,
                                          UnitPayload& up) {
    const uint32_t NG = L.groups, NB = L.superblocks;
    if (FMT == VL_TYPE_IQ2_XXS) {
        const uint4* P = reinterpret_cast<const uint4*>(w) + ((uint64_t)t * (NG / 2) + 4u * u) * 32u + n;
#pragma unroll
        for (int q = 0; q < 4; ++q) up.p[q] = P[q * 32];
        up.d = reinterpret_cast<const uint16_t*>(w + L.plane1)[((uint64_t)t * NB + u) * 32u + n];
    } else if (FMT == VL_TYPE_IQ3_XXS) {
        // Grid indices here; the sign/scale words come from load_iq3_aux.
        const uint4* Q = reinterpret_cast<const uint4*>(w) + ((uint64_t)t * (NG / 2) + 4u * u) * 32u + n;
#pragma unroll
        for (int q = 0; q < 4; ++q) up.p[q] = Q[q * 32];
        up.d = reinterpret_cast<const uint16_t*>(w + L.plane2)[((uint64_t)t * NB + u) * 32u + n];
    } else if (FMT == VL_TYPE_IQ1_S) {
        const uint4* Q = reinterpret_cast<const uint4*>(w) + ((uint64_t)t * (NG / 4) + 2u * u) * 32u + n;
        up.p[0] = Q[0];
        up.p[1] = Q[32];
        up.p[2] = reinterpret_cast<const uint4*>(w + L.plane1)[((uint64_t)t * NB + u) * 32u + n];
        up.d = reinterpret_cast<const uint16_t*>(w + L.plane2)[((uint64_t)t * NB + u) * 32u + n];
    } else {  // Q8_0: unit = one block; this lane's 16 bytes
        up.p[0] = reinterpret_cast<const uint4*>(w)[(((uint64_t)t * NG + u) * 32u + n) * 2u + hh];
        up.d = reinterpret_cast<const uint16_t*>(w + L.plane1)[((uint64_t)t * NG + u) * 32u + n];
    }
}

// IQ3_XXS keeps its eight aux words in a second pair of quads.
__device__ __forceinline__ void load_iq3_aux(const vl_tiled_layout& L, const uint8_t* __restrict__ w,
                                             uint32_t t, uint32_t n, uint32_t u, uint4& a0,
                                             uint4& a1) {
    const uint4* A = reinterpret_cast<const uint4*>(w + L.plane1) +
                     ((uint64_t)t * (L.groups / 4) + 2u * u) * 32u + n;
    a0 = A[0];
    a1 = A[32];
}

__device__ __forceinline__ uint32_t quad_word(const uint4& q, int i) {
    return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
}

// Decoded fragment and integer scale of group g (0..7) of an IQ unit.
template <uint32_t FMT>
__device__ __forceinline__ i32x4 decode_group(const UnitPayload& up, const uint4& a0,
                                              const uint4& a1, int g, int hh,
                                              const LdsTables& lds, int& sc) {
    if (FMT == VL_TYPE_IQ2_XXS) {
        const uint4& q = up.p[g >> 1];
        const uint32_t qs = (g & 1) ? q.z : q.x;
        const uint32_t aux = (g & 1) ? q.w : q.y;
        sc = 2 * (int)(aux >> 28) + 1;
        return decode_iq2_xxs(qs, aux, hh, lds.iq2);
    } else if (FMT == VL_TYPE_IQ3_XXS) {
        const uint4& q = up.p[g >> 1];
        const uint64_t qs8 = (g & 1) ? ((uint64_t)q.w << 32 | q.z) : ((uint64_t)q.y << 32 | q.x);
        const uint32_t aux = quad_word(g < 4 ? a0 : a1, g & 3);
        sc = 2 * (int)(aux >> 28) + 1;
        return decode_iq3_xxs(qs8, aux, hh, lds.iq3);
    } else {  // IQ1_S
        const uint32_t qs4 = quad_word(up.p[g >> 2], g & 3);
        const uint32_t qh = (quad_word(up.p[2], g >> 1) >> (16 * (g & 1))) & 0xffffu;
        sc = 2 * (int)((qh >> 12) & 7u) + 1;
        return decode_iq1_s(qs4, qh, hh, lds.iq1);
    }
}

template <uint32_t FMT>
__device__ __forceinline__ float unit_factor() {
    return FMT == VL_TYPE_IQ3_XXS ? 0.25f : FMT == VL_TYPE_Q8_0 ? 1.0f : 0.125f;
}

// ------------------------------------------------------------------------------------------
// Dequantize (tiled -> float rows), one wave per (tile, unit). Lane (n, hh) writes 16 weights of
// every group of the unit: w = (float)(q * sc) * (d * factor), the reference value exactly.
// ------------------------------------------------------------------------------------------

template <uint32_t FMT>
__global__ void __launch_bounds__(256) k_dequant(vl_tiled_layout L, const uint8_t* __restrict__ w,
                                                 float* __restrict__ out) {
#pragma clang fp contract(off)
    __shared__ LdsTables lds;
    load_tables<FMT>(lds);
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = lane & 31;
    const int hh = lane >> 5;
    const uint32_t units = FMT == VL_TYPE_Q8_0 ? L.groups : L.superblocks;
    const uint64_t item = (uint64_t)blockIdx.x * 4u + wave;
    if (item >= (uint64_t)L.tiles * units) return;
    const uint32_t t = (uint32_t)(item / units), u = (uint32_t)(item % units);
    const uint32_t row = t * 32u + n;
    UnitPayload up;
    load_unit<FMT>(L, w, t, n, hh, u, up);
    uint4 a0 = make_uint4(0, 0, 0, 0), a1 = a0;
    if (FMT == VL_TYPE_IQ3_XXS) load_iq3_aux(L, w, t, n, u, a0, a1);
    const float df = half_bits_to_float(up.d) * unit_factor<FMT>();
    if (row >= L.rows) return;
    const int ngroups = FMT == VL_TYPE_Q8_0 ? 1 : 8;
    for (int g = 0; g < ngroups; ++g) {
        int sc = 1;
        i32x4 frag;
        if (FMT == VL_TYPE_Q8_0) {
            frag[0] = (int)up.p[0].x; frag[1] = (int)up.p[0].y;
            frag[2] = (int)up.p[0].z; frag[3] = (int)up.p[0].w;
        } else {
            frag = decode_group<FMT>(up, a0, a1, g, hh, lds, sc);
        }
        const uint64_t col0 = (uint64_t)u * (FMT == VL_TYPE_Q8_0 ? 32u : 256u) + 32u * g + 16u * hh;
        float* dst = out + (uint64_t)row * L.cols + col0;
        for (int e = 0; e < 16; ++e) {
            const int q = (int)(int8_t)((uint32_t)frag[e >> 2] >> (8 * (e & 3)));
            dst[e] = (float)(q * sc) * df;
        }
    }
}

hipError_t launch_dequant(const vl_tiled_layout& L, const uint8_t* tiled, float* out,
                          hipStream_t stream) {
    const uint64_t units = (uint64_t)L.tiles * (L.type == VL_TYPE_Q8_0 ? L.groups : L.superblocks);
    const dim3 grid((uint32_t)((units + 3) / 4)), block(256);
    switch (L.type) {
        case VL_TYPE_IQ2_XXS: hipLaunchKernelGGL(k_dequant<VL_TYPE_IQ2_XXS>, grid, block, 0, stream, L, tiled, out); break;
        case VL_TYPE_IQ3_XXS: hipLaunchKernelGGL(k_dequant<VL_TYPE_IQ3_XXS>, grid, block, 0, stream, L, tiled, out); break;
        case VL_TYPE_IQ1_S: hipLaunchKernelGGL(k_dequant<VL_TYPE_IQ1_S>, grid, block, 0, stream, L, tiled, out); break;
        case VL_TYPE_Q8_0: hipLaunchKernelGGL(k_dequant<VL_TYPE_Q8_0>, grid, block, 0, stream, L, tiled, out); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// Activations -> limbs. One block per (set, token): max |x|, exponent, then the four digits.
// ------------------------------------------------------------------------------------------

__device__ __forceinline__ float block_max(float v, float* scratch) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float m = 0.0f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) m = fmaxf(m, scratch[i]);
    __syncthreads();
    return m;
}

__global__ void __launch_bounds__(256) k_prep_limbs(const float* __restrict__ x, uint32_t tokens,
                                                    uint32_t cols, uint64_t x_stride,
                                                    uint64_t set_stride, int8_t* __restrict__ xl,
                                                    int* __restrict__ xe, uint32_t* status) {
    __shared__ float scratch[16];
    const uint32_t tok = blockIdx.x, set = blockIdx.y;
    const uint32_t slots = tokens <= 1 ? 1u : tokens <= 2 ? 2u : tokens <= 4 ? 4u : 8u;
    const float* xs = x + set * set_stride + tok * x_stride;
    int8_t* out = xl + (uint64_t)set * (cols / 32u) * slots * 128u;
    float m = 0.0f;
    bool finite = true;
    for (uint32_t k = threadIdx.x; k < cols; k += blockDim.x) {
        const float v = xs[k];
        finite &= isfinite(v);
        m = fmaxf(m, fabsf(v));
    }
    if (!finite) atomicOr(status, kStatusNonFiniteInput);
    m = block_max(finite ? m : 0.0f, scratch);
    int q = 0;
    frexpf(m, &q);
    const int e = m > 0.0f ? 30 - q : 0;
    if (threadIdx.x == 0) xe[set * 8u + tok] = e;
    for (uint32_t k4 = threadIdx.x * 4u; k4 < cols; k4 += blockDim.x * 4u) {
        uint32_t packed[4] = {0, 0, 0, 0};
        for (int i = 0; i < 4; ++i) {
            const float v = xs[k4 + i];
            int X = isfinite(v) ? (int)rintf(ldexpf(v, e)) : 0;
            for (int l = 0; l < 4; ++l) {
                const int digit = l < 3 ? (int)(int8_t)(X & 0xff) : X;
                packed[l] |= ((uint32_t)digit & 0xffu) << (8 * i);
                X = (X - digit) >> 8;
            }
        }
        const uint64_t base = ((uint64_t)(k4 / 32u) * slots + tok) * 128u + (k4 % 32u);
        for (int l = 0; l < 4; ++l) *reinterpret_cast<uint32_t*>(out + base + 32u * l) = packed[l];
    }
}

hipError_t launch_prep_limbs(const float* x, uint32_t sets, uint32_t tokens, uint32_t cols,
                             uint64_t x_stride, uint64_t set_stride, int8_t* xl, int* xe,
                             uint32_t* status, hipStream_t stream) {
    if (tokens == 0 || tokens > 8 || cols % 32u != 0 || sets == 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_prep_limbs, dim3(tokens, sets), dim3(256), 0, stream, x, tokens, cols,
                       x_stride, set_stride, xl, xe, status);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// Batched quantized matvec.
// Block = 4 waves on one 32-row tile of one job; wave w takes a contiguous quarter of the
// units (superblocks, or Q8_0 blocks). Lane (n, hh): row n of the tile, K half hh of each
// group; for the A operand it supplies limb (n % 4) of token 2*(n/8) + (n/4)%2.
// ------------------------------------------------------------------------------------------

template <int NT>
struct Acc {
    static constexpr int kSlots = (NT + 1) / 2;  // tokens hh, hh+2, ... per lane
};

__device__ __forceinline__ float limbs_to_float(int a0, int a1, int a2, int a3) {
    return (((float)a3 * 256.0f + (float)a2) * 256.0f + (float)a1) * 256.0f + (float)a0;
}

template <uint32_t FMT, int NT>
__global__ void __launch_bounds__(256) k_qmv(const QmvBatch batch, uint32_t* status) {
    __shared__ LdsTables lds;
    __shared__ float partial[4][NT][32];
    const QmvJob job = batch.device_jobs ? batch.device_jobs[blockIdx.y]
                                         : batch.inline_jobs[blockIdx.y];
    vl_tiled_layout L;
    vl_make_layout(FMT, job.rows, job.cols, &L);
    const uint32_t t = blockIdx.x;
    if (t >= L.tiles) return;
    load_tables<FMT>(lds);
    __syncthreads();

    constexpr int S = Acc<NT>::kSlots;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = lane & 31;
    const int hh = lane >> 5;
    const uint32_t units = FMT == VL_TYPE_Q8_0 ? L.groups : L.superblocks;
    const uint32_t u0 = units * wave / 4u, u1 = units * (wave + 1) / 4u;

    // A operand: this lane's token and limb.
    const int a_tok = 2 * (int)(n / 8u) + (int)((n / 4u) & 1u);
    const int a_limb = (int)(n & 3u);
    const bool a_on = a_tok < (int)job.tokens;
    const int8_t* abase = job.xl + ((uint64_t)a_tok * 4u + a_limb) * 32u + 16u * hh;
    constexpr uint64_t kGroupStride = (uint64_t)NT * 128u;

    float accf[S];
#pragma unroll
    for (int i = 0; i < S; ++i) accf[i] = 0.0f;
    const i32x16 zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const i32x4 zero4 = {0, 0, 0, 0};

    for (uint32_t u = u0; u < u1; ++u) {
        UnitPayload up;
        load_unit<FMT>(L, job.w, t, n, hh, u, up);
        uint4 a0 = make_uint4(0, 0, 0, 0), a1 = a0;
        if (FMT == VL_TYPE_IQ3_XXS) load_iq3_aux(L, job.w, t, n, u, a0, a1);
        constexpr int G = FMT == VL_TYPE_Q8_0 ? 1 : 8;
        i32x4 afr[G];
        const uint64_t group0 = (uint64_t)u * G;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            afr[g] = zero4;
            if (a_on) afr[g] = *reinterpret_cast<const i32x4*>(abase + (group0 + g) * kGroupStride);
        }
        if (FMT == VL_TYPE_Q8_0) {
            i32x4 bfr;
            bfr[0] = (int)up.p[0].x; bfr[1] = (int)up.p[0].y;
            bfr[2] = (int)up.p[0].z; bfr[3] = (int)up.p[0].w;
            const i32x16 c = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr[0], bfr, zero16, 0, 0, 0);
            const float d = half_bits_to_float(up.d);
#pragma unroll
            for (int i = 0; i < S; ++i)
                accf[i] += d * limbs_to_float(c[4 * i], c[4 * i + 1], c[4 * i + 2], c[4 * i + 3]);
        } else {
            int acc[S][4];
#pragma unroll
            for (int i = 0; i < S; ++i) acc[i][0] = acc[i][1] = acc[i][2] = acc[i][3] = 0;
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                int sc;
                const i32x4 bfr = decode_group<FMT>(up, a0, a1, g, hh, lds, sc);
                const i32x16 c = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr[g], bfr, zero16, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < S; ++i)
#pragma unroll
                    for (int l = 0; l < 4; ++l) acc[i][l] += sc * c[4 * i + l];
            }
            const float df = half_bits_to_float(up.d) * unit_factor<FMT>();
#pragma unroll
            for (int i = 0; i < S; ++i)
                accf[i] += df * limbs_to_float(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
        }
    }

#pragma unroll
    for (int i = 0; i < S; ++i) {
        const int tok = 2 * i + hh;
        if (tok < NT) partial[wave][tok][n] = accf[i];
    }
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < NT * 32) {
        const int tok = tid / 32, r = tid % 32;
        const uint32_t row = t * 32u + r;
        if (tok < (int)job.tokens && row < job.rows) {
            const float s = ((partial[0][tok][r] + partial[1][tok][r]) + partial[2][tok][r]) +
                            partial[3][tok][r];
            const float y = ldexpf(s, -job.xe[tok]);
            if (!isfinite(y)) atomicOr(status, kStatusNonFiniteOutput);
            job.y[(uint64_t)tok * job.y_stride + row] = y;
        }
    }
}

template <uint32_t FMT>
static hipError_t launch_qmv_fmt(uint32_t slots, const QmvBatch& jobs, uint32_t njobs,
                                 uint32_t max_tiles, uint32_t* status, hipStream_t stream) {
    const dim3 grid(max_tiles, njobs), block(256);
    switch (slots) {
        case 1: hipLaunchKernelGGL((k_qmv<FMT, 1>), grid, block, 0, stream, jobs, status); break;
        case 2: hipLaunchKernelGGL((k_qmv<FMT, 2>), grid, block, 0, stream, jobs, status); break;
        case 4: hipLaunchKernelGGL((k_qmv<FMT, 4>), grid, block, 0, stream, jobs, status); break;
        case 8: hipLaunchKernelGGL((k_qmv<FMT, 8>), grid, block, 0, stream, jobs, status); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_qmv(uint32_t type, uint32_t token_slots, const QmvBatch& jobs, uint32_t njobs,
                      uint32_t max_tiles, uint32_t* status, hipStream_t stream) {
    if (njobs == 0 || max_tiles == 0) return hipSuccess;
    if (!jobs.device_jobs && njobs > kInlineJobs) return hipErrorInvalidValue;
    switch (type) {
        case VL_TYPE_IQ2_XXS: return launch_qmv_fmt<VL_TYPE_IQ2_XXS>(token_slots, jobs, njobs, max_tiles, status, stream);
        case VL_TYPE_IQ3_XXS: return launch_qmv_fmt<VL_TYPE_IQ3_XXS>(token_slots, jobs, njobs, max_tiles, status, stream);
        case VL_TYPE_IQ1_S: return launch_qmv_fmt<VL_TYPE_IQ1_S>(token_slots, jobs, njobs, max_tiles, status, stream);
        case VL_TYPE_Q8_0: return launch_qmv_fmt<VL_TYPE_Q8_0>(token_slots, jobs, njobs, max_tiles, status, stream);
        default: return hipErrorInvalidValue;
    }
}

__global__ void k_fill_u32(uint32_t* dst, uint32_t count, uint32_t value) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) dst[i] = value;
}

hipError_t launch_fill_u32(uint32_t* dst, uint32_t count, uint32_t value, hipStream_t stream) {
    if (count == 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_u32, dim3((count + 255) / 256), dim3(256), 0, stream, dst, count, value);
    return hipGetLastError();
}

}  // namespace vl
