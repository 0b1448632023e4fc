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
    // All of a thread's table loads are issued before its stores.
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    if (FMT == VL_TYPE_IQ2_XXS) {
        constexpr uint32_t n = 256 + 128;
        uint64_t v[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t i = tid + j * nt;
            if (i < n) v[j] = i < 256 ? g_tables.iq2_codes[i] : g_tables.sign_sel[i - 256];
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t i = tid + j * nt;
            if (i < 256) lds.iq2.codes[i] = v[j];
            else if (i < n) lds.iq2.sign[i - 256] = v[j];
        }
    } else if (FMT == VL_TYPE_IQ3_XXS) {
        constexpr uint32_t n = 256 + 128;
        uint64_t v[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t i = tid + j * nt;
            if (i < n) v[j] = i < 256 ? g_tables.iq3_pm[i] : g_tables.iq3_sel[i - 256];
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t i = tid + j * nt;
            if (i < 256) lds.iq3.pm[i] = v[j];
            else if (i < n) lds.iq3.sel[i - 256] = v[j];
        }
    } else if (FMT == VL_TYPE_IQ1_S) {
        uint64_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t i = tid + j * nt;
            if (i < 2048) v[j] = g_tables.iq1_codes[i];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t i = tid + j * nt;
            if (i < 2048) lds.iq1.codes[i] = v[j];
        }
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

// A chunk is one lane's share of a tile over one IQ superblock (256 columns) or four Q8_0
// blocks (128 columns). Its weight bytes are loaded a few chunks ahead of use so that every
// wave keeps several HBM requests in flight while it decodes.
constexpr int kQ8ChunkBlocks = 4;

template <uint32_t FMT>
__host__ __device__ constexpr uint32_t chunk_cols() {
    return FMT == VL_TYPE_Q8_0 ? 32u * kQ8ChunkBlocks : 256u;
}

struct Chunk {
    uint4 p[4];      // IQ: payload quads; Q8_0: one quad per block
    uint4 a0, a1;    // IQ3_XXS sign/scale words
    uint16_t d[4];   // IQ: d[0]; Q8_0: one scale per block
};

template <uint32_t FMT>
__device__ __forceinline__ void load_chunk(const vl_tiled_layout& L, const uint8_t* __restrict__ w,
                                           uint32_t t, uint32_t n, int hh, uint32_t c,
                                           Chunk& ch) {
    if (FMT == VL_TYPE_Q8_0) {
        const uint32_t NG = L.groups;
        const uint4* Q = reinterpret_cast<const uint4*>(w);
        const uint16_t* S = reinterpret_cast<const uint16_t*>(w + L.plane1);
#pragma unroll
        for (int b = 0; b < kQ8ChunkBlocks; ++b) {
            const uint32_t G = kQ8ChunkBlocks * c + b;
            if (G < NG) {
                ch.p[b] = Q[(((uint64_t)t * NG + G) * 32u + n) * 2u + hh];
                ch.d[b] = S[((uint64_t)t * NG + G) * 32u + n];
            } else {
                ch.p[b] = make_uint4(0, 0, 0, 0);
                ch.d[b] = 0;
            }
        }
    } else {
        UnitPayload up;
        load_unit<FMT>(L, w, t, n, hh, c, up);
#pragma unroll
        for (int q = 0; q < 4; ++q) ch.p[q] = up.p[q];
        ch.d[0] = up.d;
        if (FMT == VL_TYPE_IQ3_XXS) load_iq3_aux(L, w, t, n, c, ch.a0, ch.a1);
    }
}

// Pipeline depth (chunks in flight per wave) by the register size of a chunk.
template <uint32_t FMT>
struct Depth {
    static constexpr int kValue = FMT == VL_TYPE_Q8_0 ? 2 : FMT == VL_TYPE_IQ3_XXS ? 2 : 3;
};

template <uint32_t FMT, int NT>
__device__ __forceinline__ void process_chunk(const Chunk& ch, uint32_t c, uint32_t ngroups,
                                              const int8_t* abase, uint32_t a_stride,
                                              const LdsTables& lds, float* accf) {
    constexpr int S = Acc<NT>::kSlots;
    const int hh = (threadIdx.x & 63) >> 5;
    const i32x16 zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const i32x4 zero4 = {0, 0, 0, 0};
    if (FMT == VL_TYPE_Q8_0) {
        // One block at a time (A fragment, MFMA, scaled accumulate): keeping all eight MFMA
        // results live at once would exhaust the registers.
#pragma unroll
        for (int b = 0; b < kQ8ChunkBlocks; ++b) {
            const uint32_t G = kQ8ChunkBlocks * c + b;
            const i32x4 afr = G < ngroups
                ? *reinterpret_cast<const i32x4*>(abase + (uint64_t)G * a_stride) : zero4;
            i32x4 bfr;
            bfr[0] = (int)ch.p[b].x; bfr[1] = (int)ch.p[b].y;
            bfr[2] = (int)ch.p[b].z; bfr[3] = (int)ch.p[b].w;
            const i32x16 acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr, bfr, zero16, 0, 0, 0);
            const float d = half_bits_to_float(ch.d[b]);
#pragma unroll
            for (int i = 0; i < S; ++i)
                accf[i] += d * limbs_to_float(acc[4 * i], acc[4 * i + 1], acc[4 * i + 2], acc[4 * i + 3]);
            __builtin_amdgcn_sched_barrier(0);
        }
        return;
    }
    i32x4 afr[8];
#pragma unroll
    for (int g = 0; g < 8; ++g)
        afr[g] = *reinterpret_cast<const i32x4*>(abase + (uint64_t)(8u * c + g) * a_stride);
    {
        UnitPayload up;
#pragma unroll
        for (int q = 0; q < 4; ++q) up.p[q] = ch.p[q];
        up.d = ch.d[0];
        int acc[S][4];
#pragma unroll
        for (int i = 0; i < S; ++i) acc[i][0] = acc[i][1] = acc[i][2] = acc[i][3] = 0;
        // Each group's MFMA result is consumed one group later, so the next group's decode
        // covers the MFMA latency. |r| < 2^23 and sc <= 31: the 24-bit multiply is exact.
        i32x16 r_prev = zero16;
        int sc_prev = 0;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            int sc;
            const i32x4 bfr = decode_group<FMT>(up, ch.a0, ch.a1, g, hh, lds, sc);
            const i32x16 r = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr[g], bfr, zero16, 0, 0, 0);
            if (g > 0) {
#pragma unroll
                for (int i = 0; i < S; ++i)
#pragma unroll
                    for (int l = 0; l < 4; ++l) acc[i][l] += __mul24(sc_prev, r_prev[4 * i + l]);
            }
            r_prev = r;
            sc_prev = sc;
        }
#pragma unroll
        for (int i = 0; i < S; ++i)
#pragma unroll
            for (int l = 0; l < 4; ++l) acc[i][l] += __mul24(sc_prev, r_prev[4 * i + l]);
        const float df = half_bits_to_float(up.d) * unit_factor<FMT>();
#pragma unroll
        for (int i = 0; i < S; ++i)
            accf[i] += df * limbs_to_float(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
    }
}

// Partial dot products of one wave over chunks [c0, c1) of tile t. On return accf[i] holds, for
// lane (n, hh), row n of the tile against token slot 2i + hh, in units of 2^-e of that token.
// abase: this lane's A-operand source (its token's limb row, K half hh; in LDS or global
// memory) or null when the lane's token slot is unused; a_stride: bytes between consecutive
// groups of that source.
// prologue(stride) runs after the first chunks' loads are issued and before any is consumed:
// the block stages its decode tables and activations there (and synchronizes) while the weight
// stream is already in flight. It returns this lane's A-operand source; a lane whose token slot
// is unused points at zeros and sets stride to 0.
template <uint32_t FMT, int NT, typename Prologue>
__device__ __forceinline__ void tile_partial(const vl_tiled_layout& L, const uint8_t* __restrict__ w,
                                             uint32_t t, uint32_t c0, uint32_t c1,
                                             uint32_t a_stride, const LdsTables& lds,
                                             float* accf, Prologue&& prologue) {
    constexpr int S = Acc<NT>::kSlots;
    constexpr int D = Depth<FMT>::kValue;
    const int lane = threadIdx.x & 63;
    const uint32_t n = lane & 31;
    const int hh = lane >> 5;
#pragma unroll
    for (int i = 0; i < S; ++i) accf[i] = 0.0f;
    if (c1 <= c0) {
        uint32_t unused = a_stride;
        prologue(unused);
        return;
    }
    // Buffer k always holds chunk c + k: every slot keeps its registers, so waiting for one
    // chunk's loads never waits for the chunks issued after it. Past the end, loads repeat the
    // last chunk (an L1/L2 hit) instead of branching.
    Chunk buf[D];
#pragma unroll
    for (int k = 0; k < D; ++k) load_chunk<FMT>(L, w, t, n, hh, min(c0 + k, c1 - 1u), buf[k]);
    uint32_t a_stride_lane = a_stride;
    const int8_t* abase = prologue(a_stride_lane);
    uint32_t c = c0;
    for (; c + D <= c1; c += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            process_chunk<FMT, NT>(buf[k], c + k, L.groups, abase, a_stride_lane, lds, accf);
            load_chunk<FMT>(L, w, t, n, hh, min(c + k + D, c1 - 1u), buf[k]);
        }
    }
#pragma unroll
    for (int k = 0; k < D; ++k)
        if (c + k < c1) process_chunk<FMT, NT>(buf[k], c + k, L.groups, abase, a_stride_lane, lds, accf);
}

// Copies activation limbs into LDS for the block: dst [group][NT slots][128 B] from the global
// limb buffer src [group][src_slots][128 B], slot s taking token tok(s). Slots >= ntok are left
// untouched (their lanes never read).
template <int NT, typename TokMap>
__device__ __forceinline__ void stage_limbs(int8_t* dst, const int8_t* __restrict__ src,
                                            uint32_t groups, uint32_t src_slots, uint32_t ntok,
                                            TokMap&& tok) {
    constexpr int kBatch = 4;  // loads in flight per thread before their stores
    const uint32_t per_group = ntok * 8u;  // 16-byte pieces
    const uint32_t total = groups * per_group;
    for (uint32_t base = 0; base < total; base += kBatch * blockDim.x) {
        uint4 v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const uint32_t i = base + threadIdx.x + j * blockDim.x;
            if (i < total) {
                const uint32_t G = i / per_group, r = i % per_group;
                v[j] = *reinterpret_cast<const uint4*>(
                    src + ((uint64_t)G * src_slots + tok(r / 8u)) * 128u + (r % 8u) * 16u);
            }
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const uint32_t i = base + threadIdx.x + j * blockDim.x;
            if (i < total) {
                const uint32_t G = i / per_group, r = i % per_group;
                *reinterpret_cast<uint4*>(dst + ((uint64_t)G * NT + r / 8u) * 128u + (r % 8u) * 16u) = v[j];
            }
        }
    }
}

// Largest activation staging, in bytes, that a block keeps in LDS.
constexpr uint32_t kMaxLdsLimbBytes = 32u * 1024u;

// Chunks of a tiled matrix row (the last one possibly partial for Q8_0).
template <uint32_t FMT>
__device__ __forceinline__ uint32_t chunks_of(const vl_tiled_layout& L) {
    return (L.cols + chunk_cols<FMT>() - 1u) / chunk_cols<FMT>();
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
