// Shared device code of the quantized matvec kernels: per-format LDS decode tables, the loads
// of one lane's share of a unit (an IQ superblock or a Q8_0 block) of a tiled matrix, and the
// per-wave MFMA loop over a range of units of one 32-row tile.
#ifndef VL_QMV_CORE_H
#define VL_QMV_CORE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vl_decode.h"
#include "vl_layout.h"
#include "vl_tables.h"

namespace vl {

static __device__ const DecodeTables g_tables = make_decode_tables();

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

template <int NT>
struct Acc {
    static constexpr int kSlots = (NT + 1) / 2;  // tokens hh, hh+2, ... per lane
};

__device__ __forceinline__ float limbs_to_float(int a0, int a1, int a2, int a3) {
    return (((float)a3 * 256.0f + (float)a2) * 256.0f + (float)a1) * 256.0f + (float)a0;
}

// Partial dot products of one wave over units [u0, u1) of tile t. On return accf[i] holds, for
// lane (n, hh), row n of the tile against token slot 2i + hh, in units of 2^-e of that token.
// abase: this lane's A-operand source (its token's limb row, K half hh) or null when the lane's
// token slot is unused; a_stride: bytes between consecutive groups of that source.
template <uint32_t FMT, int NT>
__device__ __forceinline__ void tile_partial(const vl_tiled_layout& L, const uint8_t* __restrict__ w,
                                             uint32_t t, uint32_t u0, uint32_t u1,
                                             const int8_t* abase, uint64_t a_stride,
                                             const LdsTables& lds, float* accf) {
    constexpr int S = Acc<NT>::kSlots;
    const int lane = threadIdx.x & 63;
    const uint32_t n = lane & 31;
    const int hh = lane >> 5;
    const i32x16 zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const i32x4 zero4 = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < S; ++i) accf[i] = 0.0f;
    for (uint32_t u = u0; u < u1; ++u) {
        UnitPayload up;
        load_unit<FMT>(L, w, t, n, hh, u, up);
        uint4 a0 = make_uint4(0, 0, 0, 0), a1 = a0;
        if (FMT == VL_TYPE_IQ3_XXS) load_iq3_aux(L, w, t, n, u, a0, a1);
        constexpr int G = FMT == VL_TYPE_Q8_0 ? 1 : 8;
        i32x4 afr[G];
        const uint64_t group0 = (uint64_t)u * G;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            afr[g] = zero4;
            if (abase) afr[g] = *reinterpret_cast<const i32x4*>(abase + (group0 + g) * a_stride);
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
}

// A-operand row of lane (n, hh): token slot 2*(n/8) + (n/4)%2, limb n%4.
__device__ __forceinline__ int a_slot_of_lane() { return 2 * (int)((threadIdx.x & 31u) / 8u) + (int)(((threadIdx.x & 31u) / 4u) & 1u); }
__device__ __forceinline__ int a_limb_of_lane() { return (int)(threadIdx.x & 3u); }

template <uint32_t FMT>
__device__ __forceinline__ uint32_t units_of(const vl_tiled_layout& L) {
    return FMT == VL_TYPE_Q8_0 ? L.groups : L.superblocks;
}

}  // namespace vl

#endif  // VL_QMV_CORE_H
