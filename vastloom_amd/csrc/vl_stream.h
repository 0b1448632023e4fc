// Shared device code of the quantized matvec kernels ("stream" kernels).
//
// Work model. A kernel's work is a list of jobs (one job = one 32-row tile of one matrix, or of
// a gate/up pair of matrices), each split into units (one unit = one IQ superblock, or four
// Q8_0 blocks, of the tile's columns). The units of all jobs form one sequence, and every
// wave of a persistent grid takes an equal contiguous range of it, so the whole grid finishes
// together whatever the job count. A wave accumulates its share of a job in registers and
// hands it over as a record; the last wave to finish a job sums the job's records in wave
// order (a fixed order: results are deterministic) and runs the job's epilogue.
//
// Record handoff between waves on different XCDs uses only agent-scope atomic stores and loads
// (which the gfx9 memory model makes coherent across the per-XCD L2s by themselves) and a
// relaxed counter; a wave waits for its record stores to complete (s_waitcnt vmcnt(0)) before
// it bumps the counter. This avoids the agent-scope fences, whose L2 write-back/invalidate
// costs tens of nanoseconds each and serializes.
//
// MFMA operands (v_mfma_i32_32x32x32_i8). Lane (m, kh) = (lane % 32, lane / 32).
//   B: weight row m of the tile, columns 16kh .. 16kh+15 of the group (vl_decode.h).
//   A: row m carries limb l of token slot s, m = 8(s/2) + 4(l/2) + 2(s%2) + (l%2), so that in
//      the result lane half kh holds limbs 2kh and 2kh+1 of slot s in registers 2s and 2s+1.
//      One token therefore needs two result registers per lane, eight tokens sixteen.
// Activations are int8 limbs of X = round(x * 2^e) (|X| <= 2^30) with one exponent per 256
// columns and token; group results are scaled by the integer group scale and summed exactly
// over a superblock, converted to float once per superblock, and scaled by the superblock's
// weight factor, 2^-e and 65536 for the high limbs.
#ifndef VL_STREAM_H
#define VL_STREAM_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vl_decode.h"
#include "vl_layout.h"
#include "vl_tables.h"

namespace vl {

static __device__ const DecodeTables g_tables = make_decode_tables();


typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Global-memory view of a pointer. Pointers that reach the kernels inside structures are
// generic (flat) to the compiler; flat accesses also count against the LDS counter and block
// LDS scheduling, so every global access in the stream kernels goes through this cast.
#define VL_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ VL_GLOBAL T* gp(T* p) { return (VL_GLOBAL T*)p; }

// 16-byte global load/store as ext-vector types (the HIP vector classes do not bind to
// address-space qualified references).
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_f4(const float* p) {
    const f32x4 v = *gp(reinterpret_cast<const f32x4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 ld_u4(const void* p) {
    const u32x4 v = *gp(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// A pointer every lane holds the same value of, moved to scalar registers.
template <typename T>
__device__ __forceinline__ T* uni_ptr(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint64_t lo = uni((uint32_t)v), hi = uni((uint32_t)(v >> 32));
    return reinterpret_cast<T*>((hi << 32) | lo);
}

// Waves per persistent block (one block per CU), at most. Kernels with four or more token
// slots per job run 8 waves per block, so that each wave has 256 registers for its slots'
// accumulators and MFMA results; the others run 16 waves of 128 registers.
constexpr uint32_t kStreamWaves = 16;
constexpr uint32_t kStreamThreads = kStreamWaves * 64;
template <int NT>
__host__ __device__ constexpr uint32_t stream_waves() {
    return NT >= 4 ? 8u : 16u;
}
template <int NT>
__host__ __device__ constexpr uint32_t stream_threads() {
    return stream_waves<NT>() * 64u;
}

template <uint32_t FMT>
__host__ __device__ constexpr uint32_t table_bytes() {
    return FMT == VL_TYPE_IQ2_XXS || FMT == VL_TYPE_IQ3_XXS ? kReplTableBytes
         : FMT == VL_TYPE_IQ1_S ? kIq1TableBytes : 0u;
}

// Columns of one unit.
template <uint32_t FMT>
__host__ __device__ constexpr uint32_t unit_cols() {
    return FMT == VL_TYPE_Q8_0 ? 128u : 256u;
}

__host__ __device__ inline uint32_t units_per_row(uint32_t type, uint32_t cols) {
    const uint32_t uc = type == VL_TYPE_Q8_0 ? 128u : 256u;
    return (cols + uc - 1u) / uc;
}

// Exponent blocks (256 columns) of a row of activations.
__host__ __device__ inline uint32_t exp_blocks(uint32_t cols) { return (cols + 255u) / 256u; }

// Decode tables into LDS in two halves, so that a prologue can issue its other global loads
// between them: load() fetches up to kB source words per thread (threads tid0, tid0 + nthr, ...,
// word i0 + j * nthr), store() writes them. IQ2_XXS / IQ3_XXS: word i < nB is copies 2(i % 8) and
// 2(i % 8) + 1 of selector entry i / 8 (16 bytes into the lower half of the entry's 256-byte
// row), the nA words after it the same for the grid entries. IQ1_S: word i is grid entry i.
template <uint32_t FMT>
struct TableFill {
    static constexpr int kB = 8;
    static constexpr uint32_t per = kTabCopies / 2u;  // 16-byte stores per IQ2/IQ3 entry
    static constexpr uint32_t nB = 128u * per, nA = 256u * per;
    static constexpr uint32_t words = FMT == VL_TYPE_IQ2_XXS || FMT == VL_TYPE_IQ3_XXS ? nB + nA
                                      : FMT == VL_TYPE_IQ1_S                             ? 2048u
                                                                                         : 0u;
    uint64_t v[kB];

    __device__ void load(uint32_t i0, uint32_t nthr) {
#pragma unroll
        for (int j = 0; j < kB; ++j) {
            const uint32_t i = i0 + j * nthr;
            v[j] = 0;
            if (FMT == VL_TYPE_IQ2_XXS || FMT == VL_TYPE_IQ3_XXS) {
                if (i < nB) v[j] = FMT == VL_TYPE_IQ2_XXS ? g_tables.sign_sel[i / per] : g_tables.iq3_sel[i / per];
                else if (i < nB + nA)
                    v[j] = FMT == VL_TYPE_IQ2_XXS ? g_tables.iq2_codes[(i - nB) / per] : g_tables.iq3_pm[(i - nB) / per];
            } else if (FMT == VL_TYPE_IQ1_S) {
                if (i < words) v[j] = g_tables.iq1_codes[i];
            }
        }
    }
    __device__ void store(uint8_t* lds, uint32_t i0, uint32_t nthr) const {
#pragma unroll
        for (int j = 0; j < kB; ++j) {
            const uint32_t i = i0 + j * nthr;
            if (i >= words) continue;
            if (FMT == VL_TYPE_IQ2_XXS || FMT == VL_TYPE_IQ3_XXS) {
                const uint32_t k = i < nB ? i : i - nB;
                const uint32_t off = (i < nB ? kTabB : kTabA) + (k / per) * 256u + (k % per) * 16u;
                *reinterpret_cast<uint4*>(lds + off) = make_uint4(lo32(v[j]), hi32(v[j]), lo32(v[j]), hi32(v[j]));
            } else {
                reinterpret_cast<uint64_t*>(lds)[i] = v[j];
            }
        }
    }
    // Whether one load/store pair covers every word.
    __device__ static bool single(uint32_t nthr) { return words <= kB * nthr; }
};

// The decode tables of FMT into LDS by threads tid0, tid0 + nthr, ... (the caller synchronizes);
// eight source loads per thread are issued before their stores, so a thread waits about one
// memory latency per eight stores rather than one per store.
template <uint32_t FMT>
__device__ __forceinline__ void fill_tables(uint8_t* lds, uint32_t tid0 = threadIdx.x,
                                            uint32_t nthr = blockDim.x) {
    using TF = TableFill<FMT>;
    for (uint32_t i0 = tid0; i0 < TF::words; i0 += TF::kB * nthr) {
        TF tf;
        tf.load(i0, nthr);
        tf.store(lds, i0, nthr);
    }
}

// dst[i] = src[i] for i < n (16-byte words, global to LDS) by threads tid0, tid0 + nthr, ...; four
// loads per thread are in flight before their stores.
__device__ __forceinline__ void copy_to_lds(uint4* dst, const uint4* src, uint32_t n, uint32_t tid0,
                                            uint32_t nthr) {
    constexpr int B = 4;
    for (uint32_t i0 = tid0; i0 < n; i0 += B * nthr) {
        uint4 v[B];
#pragma unroll
        for (int j = 0; j < B; ++j) {
            const uint32_t i = i0 + j * nthr;
            if (i < n) v[j] = ld_u4(src + i);
        }
#pragma unroll
        for (int j = 0; j < B; ++j) {
            const uint32_t i = i0 + j * nthr;
            if (i < n) dst[i] = v[j];
        }
    }
}

// ------------------------------------------------------------------------------------------
// Weight chunks (one unit of one tile, this lane's share).
// ------------------------------------------------------------------------------------------

struct TileRef {
    const uint8_t* p0;
    const uint8_t* p1;
    const uint8_t* p2;
};

// Target of the loads a wave issues past the end of its range (they keep every path through the
// stream loop the same; their data is never used). One small buffer that stays in L2, instead of
// re-reading the range's last unit from HBM. 4 KiB covers the widest unit read (four Q8_0 groups).
static __device__ __align__(4096) uint8_t g_idle_unit[4096];

__device__ __forceinline__ TileRef idle_tile() {
    const uint8_t* p = g_idle_unit;
    return TileRef{p, p, p};
}

template <uint32_t FMT>
__device__ __forceinline__ TileRef tile_ref(const vl_tiled_layout& L, const uint8_t* w, uint32_t t) {
    const uint64_t NB = L.superblocks, NG = L.groups;
    TileRef r;
    if (FMT == VL_TYPE_IQ2_XXS) {
        r.p0 = w + t * NB * 2048u;
        r.p1 = w + L.plane1 + t * NB * 64u;
        r.p2 = r.p1;
    } else if (FMT == VL_TYPE_IQ3_XXS) {
        r.p0 = w + t * NB * 2048u;
        r.p1 = w + L.plane1 + t * NB * 1024u;
        r.p2 = w + L.plane2 + t * NB * 64u;
    } else if (FMT == VL_TYPE_IQ1_S) {
        r.p0 = w + t * NB * 1024u;
        r.p1 = w + L.plane1 + t * NB * 512u;
        r.p2 = w + L.plane2 + t * NB * 64u;
    } else {
        r.p0 = w + t * NG * 1024u;
        r.p1 = w + L.plane1 + t * NG * 64u;
        r.p2 = r.p1;
    }
    return r;
}

struct Chunk {
    uint4 q0, q1, q2, q3;
    uint4 a0, a1;
    uint32_t d0, d1;
};

__device__ __forceinline__ uint4 ld_stream(const uint8_t* p) {
    const u32x4 v = __builtin_nontemporal_load(gp(reinterpret_cast<const u32x4*>(p)));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return *gp(reinterpret_cast<const uint16_t*>(p));
}

// ng: groups per row (bounds the last Q8_0 unit).
template <uint32_t FMT>
__device__ __forceinline__ void load_chunk(const TileRef& tr, uint32_t c, uint32_t ng, Chunk& ch) {
    const uint32_t lane = threadIdx.x & 63u, n = lane & 31u, hh = lane >> 5;
    if (FMT == VL_TYPE_IQ2_XXS) {
        const uint8_t* P = tr.p0 + (uint64_t)c * 2048u + lane * 32u;
        ch.q0 = ld_stream(P);
        ch.q1 = ld_stream(P + 16);
        ch.d0 = ld_u16(tr.p1 + (uint64_t)c * 64u + n * 2u);
    } else if (FMT == VL_TYPE_IQ3_XXS) {
        const uint8_t* Q = tr.p0 + (uint64_t)c * 2048u + n * 16u;
        ch.q0 = ld_stream(Q);
        ch.q1 = ld_stream(Q + 512);
        ch.q2 = ld_stream(Q + 1024);
        ch.q3 = ld_stream(Q + 1536);
        const uint8_t* A = tr.p1 + (uint64_t)c * 1024u + n * 16u;
        ch.a0 = ld_stream(A);
        ch.a1 = ld_stream(A + 512);
        ch.d0 = ld_u16(tr.p2 + (uint64_t)c * 64u + n * 2u);
    } else if (FMT == VL_TYPE_IQ1_S) {
        const uint8_t* Q = tr.p0 + (uint64_t)c * 1024u + n * 16u;
        ch.q0 = ld_stream(Q);
        ch.q1 = ld_stream(Q + 512);
        ch.q2 = ld_stream(tr.p1 + (uint64_t)c * 512u + n * 16u);
        ch.d0 = ld_u16(tr.p2 + (uint64_t)c * 64u + n * 2u);
    } else {
        uint4 q[4];
        uint32_t d[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t G = 4u * c + b;
            if (G < ng) {
                q[b] = ld_stream(tr.p0 + (uint64_t)G * 1024u + n * 32u + hh * 16u);
                d[b] = ld_u16(tr.p1 + (uint64_t)G * 64u + n * 2u);
            } else {
                q[b] = make_uint4(0, 0, 0, 0);
                d[b] = 0;
            }
        }
        ch.q0 = q[0]; ch.q1 = q[1]; ch.q2 = q[2]; ch.q3 = q[3];
        ch.d0 = d[0] | (d[1] << 16);
        ch.d1 = d[2] | (d[3] << 16);
    }
}

__device__ __forceinline__ uint32_t word(const uint4& q, int i) {
    return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
}

// Payload words of an IQ2_XXS chunk in the order of vl_layout.h.
__device__ __forceinline__ void iq2_words(const Chunk& ch, uint32_t (&w)[8]) {
    w[0] = ch.q0.x; w[1] = ch.q0.y; w[2] = ch.q0.z; w[3] = ch.q0.w;
    w[4] = ch.q1.x; w[5] = ch.q1.y; w[6] = ch.q1.z; w[7] = ch.q1.w;
}

template <uint32_t FMT>
__device__ __forceinline__ float unit_factor() {
    return FMT == VL_TYPE_IQ3_XXS ? 0.25f : FMT == VL_TYPE_Q8_0 ? 1.0f : 0.125f;
}

// Per-group B fragments and integer scales of one IQ chunk, in the order the MFMA loop uses
// them. For IQ2_XXS the two halves of a row exchange their scale bytes here.
template <uint32_t FMT>
struct ChunkDecoder {
    uint32_t w[8];
    uint32_t sc_lo, sc_hi;  // IQ2_XXS: 2s+1 of groups 0..3 and 4..7, one per byte
    __device__ __forceinline__ void init(const Chunk& ch) {
        if (FMT == VL_TYPE_IQ2_XXS) {
            iq2_words(ch, w);
            const uint32_t own = iq2_scale_bytes(w);
            const uint32_t other = (uint32_t)__shfl_xor((int)own, 32);
            const bool hi_half = (threadIdx.x & 32u) != 0;
            sc_lo = odd_scales4(hi_half ? other : own);
            sc_hi = odd_scales4(hi_half ? own : other);
        }
    }
    __device__ __forceinline__ i32x4 group(const Chunk& ch, int g, uint32_t lane_off, int hh,
                                           int& sc) const {
        if (FMT == VL_TYPE_IQ2_XXS) {
            sc = (int)bfe(g < 4 ? sc_lo : sc_hi, 8u * (uint32_t)(g & 3), 8);
            return decode_iq2_xxs(w, g, lane_off);
        } else if (FMT == VL_TYPE_IQ3_XXS) {
            const uint4& q = g < 2 ? ch.q0 : g < 4 ? ch.q1 : g < 6 ? ch.q2 : ch.q3;
            const uint32_t qs = word(q, 2 * (g & 1) + hh);
            const uint32_t aux = word(g < 4 ? ch.a0 : ch.a1, g & 3);
            sc = 2 * (int)(aux >> 28) + 1;
            return decode_iq3_xxs(qs, aux, hh, lane_off);
        } else {  // IQ1_S
            const uint32_t qs4 = word(g < 4 ? ch.q0 : ch.q1, g & 3);
            const uint32_t qh = (word(ch.q2, g >> 1) >> (16 * (g & 1))) & 0xffffu;
            sc = 2 * (int)((qh >> 12) & 7u) + 1;
            return decode_iq1_s(qs4, qh, hh);
        }
    }
};

// ------------------------------------------------------------------------------------------
// A operand: where a lane reads its limb row.
// ------------------------------------------------------------------------------------------

// Token slot and limb carried by A row m (inverse of m = 8(s/2) + 4(l/2) + 2(s%2) + l%2).
__device__ __forceinline__ uint32_t a_slot(uint32_t m) { return 2u * (m / 8u) + (m / 2u) % 2u; }
__device__ __forceinline__ uint32_t a_limb(uint32_t m) { return 2u * ((m / 4u) % 2u) + m % 2u; }

// Limb source of one lane: activation limbs are stored [group][slot][4 limbs][32 columns], so
// consecutive groups of one (slot, limb) row are STRIDE = slots * 128 bytes apart (STRIDE 0:
// the run-time `stride`, for token counts known only at launch). Lanes whose token slot is
// unused read slot 0's row: their products land in result registers of unused slots (scaled by
// 0) or in registers that are never read, so every lane has the same stride.
template <bool LDS, uint32_t STRIDE>
struct ASrc {
    const int8_t* ptr;  // global source (LDS == false)
    uint32_t off;       // LDS byte address (LDS == true)
    uint32_t stride;    // bytes between groups when STRIDE == 0
    __device__ __forceinline__ i32x4 load(uint32_t G) const {
        const uint32_t st = STRIDE ? STRIDE : stride;
        if (LDS) return lds_load<i32x4>(off + G * st);
        return *gp(reinterpret_cast<const i32x4*>(ptr + (uint64_t)G * st));
    }
};

// ------------------------------------------------------------------------------------------
// Chunk processing: accf[s] += this lane's partial of (row, slot s) over the unit.
// ------------------------------------------------------------------------------------------

// A unit's activation fragments and slot scales, for policies that prefetch them with the
// weights (their activations live in global memory, where a load per unit would wait a memory
// latency each time).
template <int NT>
struct Operands {
    i32x4 a[8];
    uint32_t ev;  // lane s < NT: slot s's activation exponent (policy-defined encoding)
};

// df: weight factor of the lane's row for the unit (d times the format factor, times 65536 in
// the high-limb half); fs[s]: 2^-e of slot s for the unit's exponent block. With PRE the A
// fragments come from pre[] instead of as.
template <uint32_t FMT, int NT, typename AS, bool PRE = false>
__device__ __forceinline__ void process_chunk(const Chunk& ch, uint32_t c, uint32_t ng, const AS& as,
                                              float hscale, const float (&fs)[NT], float (&accf)[NT],
                                              const i32x4* pre = nullptr) {
    const uint32_t lane = threadIdx.x & 63u;
    const int hh = (int)(lane >> 5);
    const uint32_t lane_off = (lane % kTabCopies) * 8u;
    const i32x16 zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    if (FMT == VL_TYPE_Q8_0) {
        // Block b + 1's A fragment is requested before block b's MFMA (the compiler still waits
        // for each fragment just before its MFMA; measured −0.1 µs per q8_moe layer).
        i32x4 anext = PRE ? pre[0] : as.load(4u * c);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t G = 4u * c + b;
            if (G >= ng) break;
            const i32x4 afr = anext;
            if (b + 1 < 4 && G + 1 < ng) anext = PRE ? pre[b + 1] : as.load(G + 1);
            const uint4& q = b == 0 ? ch.q0 : b == 1 ? ch.q1 : b == 2 ? ch.q2 : ch.q3;
            i32x4 bfr;
            bfr[0] = (int)q.x; bfr[1] = (int)q.y; bfr[2] = (int)q.z; bfr[3] = (int)q.w;
            const i32x16 r = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr, bfr, zero16, 0, 0, 0);
            const uint32_t dw = b < 2 ? ch.d0 : ch.d1;
            const float d = half_bits_to_float(dw >> (16 * (b & 1))) * hscale;
#pragma unroll
            for (int s = 0; s < NT; ++s)
                accf[s] += (d * fs[s]) * ((float)r[2 * s] + 256.0f * (float)r[2 * s + 1]);
        }
        return;
    }
    i32x4 afr[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) afr[g] = PRE ? pre[g] : as.load(8u * c + g);
    ChunkDecoder<FMT> dec;
    dec.init(ch);
    int acc[2 * NT];
#pragma unroll
    for (int i = 0; i < 2 * NT; ++i) acc[i] = 0;
    // The next group's table reads are issued before this group's fragment is formed, where the
    // registers allow: IQ2_XXS without prefetched operands, IQ1_S in the 4- and 8-slot kernels
    // (256 registers). IQ3_XXS (six reads a group) spills with it and decodes in place.
    constexpr bool kPipe2 = FMT == VL_TYPE_IQ2_XXS && !PRE;
    constexpr bool kPipe1 = FMT == VL_TYPE_IQ1_S && !PRE && NT >= 4;
    Iq2Fetch t2[2];
    Iq1Fetch t1[2];
    auto iq1_qs = [&](int g) { return word(g < 4 ? ch.q0 : ch.q1, g & 3); };
    auto iq1_qh = [&](int g) { return (word(ch.q2, g >> 1) >> (16 * (g & 1))) & 0xffffu; };
    if (kPipe2) t2[0] = fetch_iq2_xxs(dec.w, 0, lane_off);
    if (kPipe1) t1[0] = fetch_iq1_s(iq1_qs(0), iq1_qh(0), hh);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        int sc;
        i32x4 bfr;
        if (kPipe2) {
            if (g + 1 < 8) t2[(g + 1) & 1] = fetch_iq2_xxs(dec.w, g + 1, lane_off);
            sc = (int)bfe(g < 4 ? dec.sc_lo : dec.sc_hi, 8u * (uint32_t)(g & 3), 8);
            bfr = finish_iq2_xxs(t2[g & 1]);
        } else if (kPipe1) {
            if (g + 1 < 8) t1[(g + 1) & 1] = fetch_iq1_s(iq1_qs(g + 1), iq1_qh(g + 1), hh);
            sc = 2 * (int)((iq1_qh(g) >> 12) & 7u) + 1;
            bfr = finish_iq1_s(t1[g & 1]);
        } else {
            bfr = dec.group(ch, g, lane_off, hh, sc);
        }
        const i32x16 r = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr[g], bfr, zero16, 0, 0, 0);
        // |r| < 2^18 and sc <= 31: the 24-bit multiply is exact; the superblock sum stays
        // below 2^27.
#pragma unroll
        for (int i = 0; i < 2 * NT; ++i) acc[i] += __mul24(sc, r[i]);
    }
    const float df = half_bits_to_float(ch.d0) * (unit_factor<FMT>() * hscale);
#pragma unroll
    for (int s = 0; s < NT; ++s)
        accf[s] += (df * fs[s]) * ((float)acc[2 * s] + 256.0f * (float)acc[2 * s + 1]);
}

// Units in flight per wave. Sixteen waves per CU each with two 2 KiB IQ2_XXS units in flight keep
// enough bytes moving; deeper rings measured slower on MI355X (more registers, and the CU's
// oldest waves crowd out the rest), so depth is kept at two except for IQ1_S's small chunks.
template <uint32_t FMT>
struct StreamDepth {
    static constexpr int kValue = FMT == VL_TYPE_IQ1_S ? 3 : 2;
};

// ------------------------------------------------------------------------------------------
// Unit ranges and record handoff.
// ------------------------------------------------------------------------------------------

// Waves that take part: every one of them gets at least one unit, so the waves holding a
// job's units are exactly the consecutive waves from the first to the last of them.
__device__ __forceinline__ uint32_t active_waves(uint32_t nw, uint32_t total) {
    return total < nw ? total : nw;
}
// Wave w of nw active waves takes units [w*total/nw, (w+1)*total/nw); waves beyond nw none.
__device__ __forceinline__ uint32_t range_begin(uint32_t w, uint32_t nw, uint32_t total) {
    return w < nw ? (uint32_t)((uint64_t)w * total / nw) : total;
}
// The wave whose range holds unit u (a 32-bit division whenever the product fits in 32 bits).
__device__ __forceinline__ uint32_t wave_of_unit(uint32_t u, uint32_t nw, uint32_t total) {
    const uint64_t q = ((uint64_t)u + 1u) * nw - 1u;
    return (q >> 32) ? (uint32_t)(q / total) : (uint32_t)q / total;
}

__device__ __forceinline__ void store_shared(float* p, float v) {
    __hip_atomic_store(gp(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_shared(const float* p) {
    return __hip_atomic_load(gp(const_cast<float*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void or_bits(uint32_t* p, uint32_t bits) {
    __hip_atomic_fetch_or(gp(p), bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_shared_u32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(gp(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_shared_u32(const uint32_t* p) {
    return __hip_atomic_load(gp(const_cast<uint32_t*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sums of a job's records for (slot s, row n) of matrices 0..NM-1: records first..last in order,
// each record's two lane halves added first. The loads of eight records are issued before any of
// them is used, so a fixup waits about one memory latency per eight records (a job rarely has
// more contributors than that).
template <int NT, int NM>
__device__ __forceinline__ void sum_records(const float* rec, uint32_t rec_floats, uint32_t j,
                                            uint32_t first, uint32_t last, uint32_t s, uint32_t n,
                                            float (&out)[NM]) {
    constexpr int B = 8;
#pragma unroll
    for (int m = 0; m < NM; ++m) out[m] = 0.0f;
    for (uint32_t k0 = first; k0 <= last; k0 += B) {
        float v[B][NM][2];
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const uint32_t k = k0 + i <= last ? k0 + i : last;  // clamped loads are not added
            const float* r = rec + (uint64_t)(k + j) * rec_floats + s * 64u + n;
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                v[i][m][0] = load_shared(r + m * NT * 64u);
                v[i][m][1] = load_shared(r + m * NT * 64u + 32u);
            }
        }
#pragma unroll
        for (int i = 0; i < B; ++i)
            if (k0 + i <= last)
#pragma unroll
                for (int m = 0; m < NM; ++m) out[m] += v[i][m][0] + v[i][m][1];
    }
}

// OR of a predicate over the block, through one LDS word per wave (slots[kStreamWaves], no
// initialisation needed: every wave writes its own word). Contains a block barrier.
__device__ __forceinline__ bool block_any(bool v, uint32_t* slots) {
    const bool w = __any(v);
    if ((threadIdx.x & 63u) == 0) slots[threadIdx.x >> 6] = w ? 1u : 0u;
    __syncthreads();
    uint32_t r = 0;
    for (uint32_t i = 0; i < (blockDim.x >> 6); ++i) r |= slots[i];
    return r != 0;
}

// Publishes this wave's record stores and counts the wave in; returns true in every lane of
// the last wave of the job's kc contributors (which then owns the job's records and resets
// the counter for the next launch).
__device__ __forceinline__ bool arrive(uint32_t* counter, uint32_t kc) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's record stores have completed
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    uint32_t old = 0;
    if ((threadIdx.x & 63u) == 0)
        old = __hip_atomic_fetch_add(gp(counter), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = (uint32_t)__shfl((int)old, 0);
    const bool last = old == kc - 1u;
    if (last && (threadIdx.x & 63u) == 0)
        __hip_atomic_store(gp(counter), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return last;
}

// ------------------------------------------------------------------------------------------
// Activations -> limbs.
// ------------------------------------------------------------------------------------------

// Four limbs (signed base-256 digits, the top one carrying the sign) of round(v * 2^e) for
// four consecutive values, one 32-bit word per limb. Non-finite values encode as zero.
//
// For |X| < 2^30, Y = X + 0x808080 has bytes y0, y1, y2 in [0, 255] and a top byte y3 = Y >> 24 in
// [-64, 63], and X = (y0 - 128) + 2^8 (y1 - 128) + 2^16 (y2 - 128) + 2^24 y3: the digits in
// [-128, 127] are y_l ^ 0x80 as int8, the unique signed base-256 digits of X. So the bytes of
// Y ^ 0x808080 are the value's four limbs, and a 4x4 byte transpose groups them by limb.
__device__ __forceinline__ void limbs4(const float (&v)[4], int e, uint32_t (&packed)[4]) {
    uint32_t z[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int X = isfinite(v[k]) ? (int)rintf(ldexpf(v[k], e)) : 0;
        z[k] = ((uint32_t)X + 0x00808080u) ^ 0x00808080u;
    }
    // Bytes (value k, limb l) -> word l, byte k: first pair bytes of equal limb parity, then
    // interleave the pairs.
    const uint32_t e01 = __builtin_amdgcn_perm(z[1], z[0], 0x06020400u);  // z0b0 z1b0 z0b2 z1b2
    const uint32_t o01 = __builtin_amdgcn_perm(z[1], z[0], 0x07030501u);  // z0b1 z1b1 z0b3 z1b3
    const uint32_t e23 = __builtin_amdgcn_perm(z[3], z[2], 0x06020400u);
    const uint32_t o23 = __builtin_amdgcn_perm(z[3], z[2], 0x07030501u);
    packed[0] = __builtin_amdgcn_perm(e23, e01, 0x05040100u);
    packed[1] = __builtin_amdgcn_perm(o23, o01, 0x05040100u);
    packed[2] = __builtin_amdgcn_perm(e23, e01, 0x07060302u);
    packed[3] = __builtin_amdgcn_perm(o23, o01, 0x07060302u);
}

// Exponent that brings m = max |v| (finite, >= 0) to just below 2^30.
__device__ __forceinline__ int limb_exponent(float m) {
    int q = 0;
    frexpf(m, &q);
    return m > 0.0f ? 30 - q : 0;
}

// One wave: limbs of columns [256 xb, 256 xb + 256) of token t of x ([tokens][cols], token
// stride x_stride) into xl ([cols/32][slots][4][32]), the block's exponent into xe[estride xb + t]
// and a non-finite flag into flags[estride xb + t] (written whatever its value). cols is a
// multiple of 32. The stores are agent-scope (written through to memory), so that blocks of the
// same launch on other XCDs can read them after a grid barrier.
__device__ __forceinline__ void prep_x_token(const float* __restrict__ x, uint64_t x_stride,
                                             uint32_t cols, uint32_t t, uint32_t slots,
                                             uint32_t estride, uint32_t xb, int8_t* __restrict__ xl,
                                             int* __restrict__ xe, uint32_t* __restrict__ flags) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t col = xb * 256u + lane * 4u;
    {
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (col < cols) {
            const float4 f = ld_f4(x + (uint64_t)t * x_stride + col);
            v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
        }
        bool finite = true;
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            finite &= isfinite(v[k]);
            if (isfinite(v[k])) m = fmaxf(m, fabsf(v[k]));
        }
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        const bool all_finite = __all(finite);
        const int e = limb_exponent(m);
        if (lane == 0) {
            store_shared_u32(reinterpret_cast<uint32_t*>(xe + estride * xb + t), (uint32_t)e);
            store_shared_u32(flags + estride * xb + t, all_finite ? 0u : 1u);
        }
        if (col < cols) {
            uint32_t packed[4];
            limbs4(v, e, packed);
            const uint64_t base = ((uint64_t)(col / 32u) * slots + t) * 128u + (col % 32u);
#pragma unroll
            for (int l = 0; l < 4; ++l) store_shared_u32(reinterpret_cast<uint32_t*>(xl + base + 32u * l), packed[l]);
        }
    }
}

// One wave per token t in [t0, t1) of the block: prep_x_token.
__device__ __forceinline__ void prep_x_block(const float* __restrict__ x, uint64_t x_stride,
                                             uint32_t cols, uint32_t t0, uint32_t t1, uint32_t slots,
                                             uint32_t estride, uint32_t xb, int8_t* __restrict__ xl,
                                             int* __restrict__ xe, uint32_t* __restrict__ flags) {
    const uint32_t wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    for (uint32_t t = t0 + wave; t < t1; t += nwaves)
        prep_x_token(x, x_stride, cols, t, slots, estride, xb, xl, xe, flags);
}

// ------------------------------------------------------------------------------------------
// The wave loop.
//
// Policy interface (all values wave-uniform):
//   uint32_t chunks, nmat, ng;            units per matrix row, matrices per job, groups/row
//   TileRef tref(uint32_t j, uint32_t mat)
//   void job_begin(uint32_t j)            prepares as, hscale for job j
//   ASrc<LDS> as; float hscale;
//   void scales(uint32_t j, uint32_t c, float (&fs)[NT])
//   uint32_t* store(uint32_t j, const float (&m0)[NT], const float (&m1)[NT], uint32_t& kc)
//       stores the wave's record of job j; returns the job's counter and its contributor count
//   void fixup(uint32_t j)   the job's epilogue, by the last contributor
//   static constexpr bool kPrefetch; with it set,
//   void load_ops(uint32_t j, uint32_t c, Operands<NT>& o)
//       issues unit (j, c)'s A fragment and exponent loads one unit ahead, waiting for nothing
//       (issued before that iteration's weight prefetch, so waiting for them never waits for
//       newer weights); as is not used
//   void ops_scales(const Operands<NT>& o, uint32_t j, uint32_t c, float (&fs)[NT])
//       the unit's slot scales, when it is processed
// ------------------------------------------------------------------------------------------

// Issue priority by remaining work. Among ready waves of equal priority a SIMD serves the oldest
// first, so a block's younger waves fall behind and finish alone with the SIMD under-occupied
// (measured: finish times 9 us apart within a CU). A wave with more of its range left takes a
// higher priority (four levels over its range), which keeps a SIMD's waves advancing together.
__device__ __forceinline__ void progress_priority(uint32_t rem, uint32_t len) {
    const uint32_t lvl = rem ? ((rem - 1u) * 4u) / len : 0u;
    if (lvl >= 3u) __builtin_amdgcn_s_setprio(3);
    else if (lvl == 2u) __builtin_amdgcn_s_setprio(2);
    else if (lvl == 1u) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}

template <uint32_t FMT, int NT, bool LDS, typename Pol>
__device__ __forceinline__ void stream_range(Pol& pol, uint32_t u0, uint32_t u1) {
    constexpr int D = StreamDepth<FMT>::kValue;
    if (u0 >= u1) return;
    const uint32_t C = pol.chunks, NM = pol.nmat, UJ = C * NM;
    // Load head: D units ahead of the processing position. Loads are issued unconditionally
    // (past the end of the range the head moves to the idle unit, an L2 hit) so that every
    // path through the loop has the same loads outstanding and the waits before each chunk
    // stay partial.
    uint32_t hj = u0 / UJ, hm = (u0 - hj * UJ) / C, hc = u0 - hj * UJ - hm * C;
    uint32_t hu = u0;
    TileRef htr = pol.tref(hj, hm);
    auto head_next = [&]() {
        if (hu + 1u >= u1) {
            htr = idle_tile();
            hc = 0;
            return;
        }
        ++hu;
        if (++hc == C) {
            hc = 0;
            if (++hm == NM) {
                hm = 0;
                ++hj;
            }
            htr = pol.tref(hj, hm);
        }
    };
    constexpr bool PF = Pol::kPrefetch;
    uint32_t pj = u0 / UJ, pm = (u0 - pj * UJ) / C, pc = u0 - pj * UJ - pm * C;
    Operands<NT> ob;
    if constexpr (PF) {
        pol.load_ops(pj, pc, ob);
        __builtin_amdgcn_sched_barrier(0);
    }
    Chunk buf[D];
#pragma unroll
    for (int k = 0; k < D; ++k) {
        load_chunk<FMT>(htr, hc, pol.ng, buf[k]);
        head_next();
    }
    pol.job_begin(pj);
    auto flush = [&](uint32_t j, const float (&m0)[NT], const float (&m1)[NT]) {
        uint32_t kc;
        uint32_t* ctr = pol.store(j, m0, m1, kc);
        if (arrive(ctr, kc)) pol.fixup(j);
    };
    float acc[NT], keep[NT], fs[NT];
#pragma unroll
    for (int s = 0; s < NT; ++s) acc[s] = keep[s] = 0.0f;
    for (uint32_t u = u0; u < u1; u += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            const uint32_t uu = u + k;
            progress_priority(uu < u1 ? u1 - uu : 0u, u1 - u0);
            if (uu < u1) {
                if constexpr (PF) {
                    pol.ops_scales(ob, pj, pc, fs);
                    process_chunk<FMT, NT, decltype(pol.as), true>(buf[k], pc, pol.ng, pol.as, pol.hscale,
                                                                   fs, acc, ob.a);
                } else {
                    pol.scales(pj, pc, fs);
                    process_chunk<FMT, NT>(buf[k], pc, pol.ng, pol.as, pol.hscale, fs, acc);
                }
            }
            if constexpr (!PF) {
                load_chunk<FMT>(htr, hc, pol.ng, buf[k]);
                head_next();
            }
            if (uu < u1) {
                bool job_end = false;
                if (++pc == C) {
                    pc = 0;
                    if (pm + 1 < NM) {
#pragma unroll
                        for (int s = 0; s < NT; ++s) {
                            keep[s] = acc[s];
                            acc[s] = 0.0f;
                        }
                        ++pm;
                    } else {
                        job_end = true;
                    }
                }
                if (job_end || uu + 1 == u1) {
                    if (NM == 2 && pm == 1) flush(pj, keep, acc);
                    else flush(pj, acc, keep);  // keep is zero here
#pragma unroll
                    for (int s = 0; s < NT; ++s) acc[s] = keep[s] = 0.0f;
                    if (job_end) {
                        ++pj;
                        pm = 0;
                        if (uu + 1 < u1) pol.job_begin(pj);
                    }
                }
            }
            if constexpr (PF) {
                if (uu + 1 < u1) pol.load_ops(pj, pc, ob);  // (pj, pc) is now the next unit
                __builtin_amdgcn_sched_barrier(0);  // the operand loads stay ahead of the weights'
                load_chunk<FMT>(htr, hc, pol.ng, buf[k]);
                head_next();
            }
        }
    }
}

}  // namespace vl

#endif  // VL_STREAM_H
