// The grouped MoE layer's expert projections on fp16 MFMA, for IQ2_XXS gate/up and down
// matrices: every weight is (d/8) * (2s+1) * m * sign with m in {8, 25, 43} and 2s+1 <= 31, so
// the integer part (2s+1) * m * sign (at most 1333 in magnitude) is exact in fp16, and one
// v_mfma_f32_32x32x16_f16 takes sixteen tokens at once with each activation split into an fp16
// high and low part. The superblock factor d/8 and the activation's block scale are applied once
// per 256 columns, in float, to the MFMA's float results.
//
//   k_wide_prep    activations -> hi/lo fp16 of x * 2^e with max |x * 2^e| in [2^14, 2^15) over
//                  the token's row, the scale 2^-e, a non-finite flag per 256-column block;
//                  zeroes the layer's status word
//   k_wide_gateup  one block per (item, 256 rows of gate and up): the item's tokens (up to two
//                  groups of sixteen) against every column, SwiGLU of the semantics, then h of
//                  the block's 256 rows as hi/lo fp16 with one scale per token
//   k_wide_down    one block per (item, run of 512-row slabs of the output): the item's h against
//                  the down rows, each (entry, slot)'s output rows into the partial-output array
//                  that k_moe_combine adds in the reference's combine order
//
// An item is a run of up to 2 * kWideGroups consecutive entries of the group list of one expert
// (k_moe_plan's 8-token entries, ascending tokens): entry pair 2g, 2g+1 of the item is MFMA
// group g, slot t of the group is entry 2g + t/8, slot t%8. Rows of the group's A operand carry
// (slot, hi/lo): row m = 8(t/4) + 4((t/2)%2) + 2(t%2) + limb, which puts a token's high and low
// results in adjacent result registers of one lane.
//
// Precision: x (or h) equals hi + lo to 2^-22 of its own magnitude; the products of the fp16
// operands are exact in float; each superblock's sum is rounded in float at every 16-column step
// and again when scaled and added. The error stays below about 3e-6 * sum |w| |x|, well inside
// the 1e-5 * |w_row| |x| bound of the layer tests.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iq_codebooks.h"
#include "vl_kernels.h"
#include "vl_moe.h"
#include "vl_moe_dev.h"
#include "vl_moe_wide.h"
#include "vl_stream.h"

namespace vl {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// LDS of the projection kernels, from byte 0:
//   grid    the 256 IQ2_XXS grid entries as eight fp16 magnitudes (16 bytes), in kWideGridCopies
//           copies: entry e, copy c at byte (e * kWideGridCopies + c) * 16; lane l reads copy
//           l % kWideGridCopies, which spreads the random lookups of one LDS cycle over more banks
//   signs   for each 4-bit scale s and 7-bit sign field f, the eight fp16 factors +-(2s+1) with
//           the signs of f and its parity bit, at byte kWideSigns + (s * 128 + f) * 16 (32 KiB)
//   A       two buffers (superblock parity) of kWideGroups groups x 32 rows x 256 fp16 columns,
//           rows kWideRowBytes apart (16 bytes of padding keep the 16 lanes of one LDS cycle on
//           distinct banks)
//   scale   per buffer and group, the 16 slots' block scales
//   red     per wave and group, the slots' maxima of |h| (gate/up)
// A weight's fp16 B value is grid * factor: both are exact small integers and their product
// (at most 43 * 31 = 1333) is exact in fp16.
constexpr uint32_t kWideGridCopies = 8;
constexpr uint32_t kWideGridBytes = 256u * kWideGridCopies * 16u;
constexpr uint32_t kWideSigns = kWideGridBytes;
constexpr uint32_t kWideTabBytes = kWideSigns + 16u * 128u * 16u;
constexpr uint32_t kWideRowBytes = 528u;
constexpr uint32_t kWideGroupBytes = 32u * kWideRowBytes;
constexpr uint32_t kWideA = kWideTabBytes;
constexpr uint32_t kWideScale = kWideA + 2u * kWideGroups * kWideGroupBytes;
constexpr uint32_t kWideRed = kWideScale + 2u * kWideGroups * 16u * 4u;
constexpr uint32_t kWideLdsBytes = kWideRed + kWideWaves * kWideGroups * 16u * 4u;
static_assert(kWideLdsBytes <= 160u * 1024u, "LDS of one workgroup");
static_assert(kWideWaves * 32u == 256u, "a block covers one 256-row block of h");

static __device__ const uint16_t g_iq2_codes16[256] = VL_IQ2XXS_CODES;

// Row m of a group's A operand: its slot and limb (0 high, 1 low).
__device__ __forceinline__ uint32_t wide_slot(uint32_t m) { return 4u * (m / 8u) + 2u * ((m / 4u) % 2u) + (m % 4u) / 2u; }
__device__ __forceinline__ uint32_t wide_limb(uint32_t m) { return m % 2u; }
// Slot of result pair q (registers 2q, 2q+1) of a lane in half hh.
__device__ __forceinline__ uint32_t wide_pair_slot(uint32_t q, uint32_t hh) { return 4u * (q / 2u) + 2u * hh + q % 2u; }

// Exponent e with max |v * 2^e| in [2^14, 2^15) for m = max |v| > 0 (0 for m == 0).
__device__ __forceinline__ int wide_exponent(float m) {
    int q = 0;
    frexpf(m, &q);
    return m > 0.0f ? 15 - q : 0;
}

// hi/lo fp16 of v * 2^e.
__device__ __forceinline__ void split16(float v, int e, _Float16& hi, _Float16& lo) {
    const float s = __builtin_amdgcn_ldexpf(v, e);
    hi = (_Float16)s;
    lo = (_Float16)(s - (float)hi);
}

// ------------------------------------------------------------------------------------------
// Activations.
// ------------------------------------------------------------------------------------------

// Block t: token t, one exponent for the whole row (fp16's exponent range keeps the hi/lo split of
// the smallest values within 2^-39 of the row's largest); wave v takes the 256-column blocks
// v, v + 4, ... and flags each block's non-finite values.
__global__ void __launch_bounds__(256) k_wide_prep(const MoeShape s, const MoeInputs in, const MoeWorkspace w) {
    __shared__ float red[4];
    const uint32_t t = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63u, H = s.width;
    if (t == 0 && threadIdx.x < 2) {
        MoeHeader* hdr = ws_ptr<MoeHeader>(w, w.off_header);
        (&hdr->status)[threadIdx.x] = 0;
    }
    const float* xr = in.x + (uint64_t)t * H;
    float m = 0.0f;
    for (uint32_t b = wave; b < w.xblocks; b += 4u) {
        const float4 f = ld_f4(xr + b * 256u + lane * 4u);
        const float v[4] = {f.x, f.y, f.z, f.w};
        bool finite = true;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            finite &= isfinite(v[k]);
            if (isfinite(v[k])) m = fmaxf(m, fabsf(v[k]));
        }
        const bool all_finite = __all(finite);
        if (lane == 0) *gp(ws_ptr<uint32_t>(w, w.off_xflags) + (uint64_t)w.estride * b + t) = all_finite ? 0u : 1u;
    }
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    const int e = wide_exponent(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
    _Float16* row = ws_ptr<_Float16>(w, w.off_x16) + (uint64_t)t * 2u * H;
    for (uint32_t b = wave; b < w.xblocks; b += 4u) {
        const uint32_t col = b * 256u + lane * 4u;
        const float4 f = ld_f4(xr + col);
        const float v[4] = {f.x, f.y, f.z, f.w};
        uint32_t hb[4], lb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            _Float16 hi, lo;
            split16(isfinite(v[k]) ? v[k] : 0.0f, e, hi, lo);
            hb[k] = __builtin_bit_cast(uint16_t, hi);
            lb[k] = __builtin_bit_cast(uint16_t, lo);
        }
        *reinterpret_cast<uint2*>(row + col) = make_uint2(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16));
        *reinterpret_cast<uint2*>(row + H + col) = make_uint2(lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16));
    }
    if (threadIdx.x == 0) *gp(ws_ptr<float>(w, w.off_xsc) + t) = __builtin_amdgcn_ldexpf(1.0f, -e);
}

// ------------------------------------------------------------------------------------------
// Shared pieces of the projection kernels.
// ------------------------------------------------------------------------------------------

// The grid and sign/scale tables into LDS (512 threads).
__device__ __forceinline__ void wide_fill_table(uint8_t* lds) {
    const uint32_t i = threadIdx.x;
    if (i >= 512u) return;
    {
        // Grid entry i / 2, copies 4 (i % 2) .. 4 (i % 2) + 3.
        const uint32_t e = i >> 1, codes = g_iq2_codes16[e];
        uint32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t h2v[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t c = (codes >> (2 * (2 * k + j))) & 3u;
                h2v[j] = c == 0u ? 0x4800u : c == 1u ? 0x4e40u : 0x5160u;  // fp16 8, 25, 43
            }
            v[k] = h2v[0] | (h2v[1] << 16);
        }
#pragma unroll
        for (uint32_t c = 0; c < kWideGridCopies / 2u; ++c)
            *reinterpret_cast<uint4*>(lds + (e * kWideGridCopies + (i & 1u) * (kWideGridCopies / 2u) + c) * 16u) =
                make_uint4(v[0], v[1], v[2], v[3]);
    }
#pragma unroll
    for (uint32_t j = 0; j < 4u; ++j) {
        // Sign/scale entry i * 4 + j = (scale s, sign field f).
        const uint32_t idx = i * 4u + j, sc = idx >> 7, f = idx & 127u;
        const uint32_t s8 = f | ((__builtin_popcount(f) & 1u) << 7);
        const uint32_t mag = __builtin_bit_cast(uint16_t, (_Float16)(float)(2u * sc + 1u));
        uint32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            v[k] = (mag | (((s8 >> (2 * k)) & 1u) << 15)) | ((mag | (((s8 >> (2 * k + 1)) & 1u) << 15)) << 16);
        *reinterpret_cast<uint4*>(lds + kWideSigns + idx * 16u) = make_uint4(v[0], v[1], v[2], v[3]);
    }
}

// One lane's B fragment of K step k = 2G + p of its superblock row half: the grid index and sign
// field of sub-block 2(G % 2) + p of w[G / 2], w[4 + G / 2], and sbase = the group's scale
// times 2048 (its row of the sign/scale table). fetch reads the two table entries, finish
// multiplies them.
struct WideFetch {
    u32x4 g, f;
};
__device__ __forceinline__ WideFetch wide_fetch(const uint32_t (&w)[8], uint32_t k, uint32_t sbase, uint32_t lane_off) {
    const uint32_t G = k >> 1, sub = 2u * (G & 1u) + (k & 1u);
    const uint32_t gi = bfe(w[G >> 1], 8u * sub, 8u);
    const uint32_t f = bfe(w[4u + (G >> 1)], 7u * sub, 7u);
    return WideFetch{lds_load<u32x4>((gi << 7) | lane_off), lds_load<u32x4>(kWideSigns + (sbase | (f << 4)))};
}
__device__ __forceinline__ h8 wide_finish(const WideFetch& t) {
    const uint32_t g[4] = {t.g.x, t.g.y, t.g.z, t.g.w}, f[4] = {t.f.x, t.f.y, t.f.z, t.f.w};
    h8 r;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const h2 x = __builtin_bit_cast(h2, g[k]) * __builtin_bit_cast(h2, f[k]);
        r[2 * k] = x[0];
        r[2 * k + 1] = x[1];
    }
    return r;
}

// A superblock's activation rows for the block, from global to a register stage and from there
// to LDS, with (PB) the slots' scales of the superblock's 256-column block. Each of the 512
// threads moves two 16-byte pieces per group in use: piece c = tid + 512 j is group c / 1024,
// row (c / 32) % 32, 16-byte column chunk c % 32. Rows of empty slots read the item's first row
// instead (every load is unconditional, so waits stay partial); their results are never used.
template <bool PB>
struct WideStage {
    uint4 v[2 * kWideGroups];
    const _Float16* src[2 * kWideGroups];  // the piece's row
    uint32_t dst[2 * kWideGroups];         // LDS offset within a buffer
    float sc;                              // thread tid < 16 * kWideGroups: slot tid's scale
    const float* scsrc;                    // that slot's scale row

    // rowid(g, t): the activation row (into the hi/lo array) of group g's slot t, or ~0u;
    // row0: a row that exists.
    template <typename RowOf>
    __device__ void init(RowOf rowid, uint32_t row0, uint32_t cols, const _Float16* base, const float* scales,
                         uint32_t nblocks) {
        const uint32_t tid = threadIdx.x;
#pragma unroll
        for (uint32_t j = 0; j < 2u * kWideGroups; ++j) {
            const uint32_t c = tid + 512u * j;
            const uint32_t g = c / 1024u, m = (c / 32u) % 32u, ch = c % 32u;
            uint32_t r = rowid(g, wide_slot(m));
            r = r == ~0u ? row0 : r;
            src[j] = base + ((uint64_t)r * 2u + wide_limb(m)) * cols + ch * 8u;
            dst[j] = g * kWideGroupBytes + m * kWideRowBytes + ch * 16u;
        }
        uint32_t r = tid < 16u * kWideGroups ? rowid(tid / 16u, tid % 16u) : ~0u;
        r = r == ~0u ? row0 : r;
        scsrc = scales + (uint64_t)r * nblocks;
    }
    // NG: groups in use (pieces j < 2 * NG).
    template <uint32_t NG>
    __device__ void load(uint32_t sb) {
#pragma unroll
        for (uint32_t j = 0; j < 2u * NG; ++j) v[j] = ld_u4(reinterpret_cast<const uint4*>(src[j] + 256u * sb));
        if (PB) sc = *gp(scsrc + sb);
    }
    template <uint32_t NG>
    __device__ void store(uint8_t* lds, uint32_t buf) const {
        const uint32_t base = kWideA + buf * kWideGroups * kWideGroupBytes;
#pragma unroll
        for (uint32_t j = 0; j < 2u * NG; ++j) *reinterpret_cast<uint4*>(lds + base + dst[j]) = v[j];
        if (PB && threadIdx.x < 16u * kWideGroups)
            *reinterpret_cast<float*>(lds + kWideScale + (buf * kWideGroups * 16u + threadIdx.x) * 4u) = sc;
    }
};

// One lane's IQ2_XXS words of a superblock of one matrix row (tiled layout: 32 contiguous bytes
// per lane, the fp16 d in a separate plane).
struct WideRow {
    uint4 q0, q1;
    uint32_t d;
    __device__ void load(const uint8_t* p0, const uint8_t* p1, uint32_t sb) {
        const uint32_t lane = threadIdx.x & 63u;
        const uint8_t* P = p0 + (uint64_t)sb * 2048u + lane * 32u;
        q0 = ld_stream(P);
        q1 = ld_stream(P + 16);
        d = ld_u16(p1 + (uint64_t)sb * 64u + (lane & 31u) * 2u);
    }
};

// acc[m][g][q] += the superblock's products of matrix m (rows of the lane's tile) with group g's
// slot pair q, scaled by d/8 and the slots' block scales. NM matrices (gate and up, or down).
template <int NM, uint32_t NG, bool PB>
__device__ __forceinline__ void wide_superblock(const uint8_t* lds, uint32_t buf, const WideRow (&wr)[NM],
                                                float (&acc)[NM][kWideGroups][8]) {
    const uint32_t lane = threadIdx.x & 63u, n = lane & 31u, hh = lane >> 5;
    uint32_t w[NM][8];
    uint32_t sc_lo[NM], sc_hi[NM];  // scale bytes (scale in bits 4..7) of groups 0..3 / 4..7
#pragma unroll
    for (int mt = 0; mt < NM; ++mt) {
        w[mt][0] = wr[mt].q0.x; w[mt][1] = wr[mt].q0.y; w[mt][2] = wr[mt].q0.z; w[mt][3] = wr[mt].q0.w;
        w[mt][4] = wr[mt].q1.x; w[mt][5] = wr[mt].q1.y; w[mt][6] = wr[mt].q1.z; w[mt][7] = wr[mt].q1.w;
        const uint32_t own = iq2_scale_bytes(w[mt]);
        const uint32_t other = (uint32_t)__shfl_xor((int)own, 32);
        sc_lo[mt] = hh ? other : own;
        sc_hi[mt] = hh ? own : other;
    }
    const uint32_t lane_off = (lane % kWideGridCopies) * 16u;
    auto sbase = [&](int mt, uint32_t G) { return bfe(G < 4u ? sc_lo[mt] : sc_hi[mt], 8u * (G & 3u) + 4u, 4u) << 11; };
    const uint32_t abase = kWideA + buf * kWideGroups * kWideGroupBytes + n * kWideRowBytes + 32u * hh;
    // K step k + 1's table and A reads are issued before step k's fragments are finished.
    f32x16 C[NM][NG];
    const f32x16 zero = {};
    WideFetch tf[NM][2];
    h8 A[NG][2];
#pragma unroll
    for (int mt = 0; mt < NM; ++mt) tf[mt][0] = wide_fetch(w[mt], 0u, sbase(mt, 0u), lane_off);
#pragma unroll
    for (uint32_t g = 0; g < NG; ++g) A[g][0] = lds_load<h8>(abase + g * kWideGroupBytes);
#pragma unroll
    for (uint32_t k = 0; k < 16u; ++k) {
        const uint32_t cur = k & 1u, nx = cur ^ 1u;
        if (k + 1u < 16u) {
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) tf[mt][nx] = wide_fetch(w[mt], k + 1u, sbase(mt, (k + 1u) >> 1), lane_off);
#pragma unroll
            for (uint32_t g = 0; g < NG; ++g)
                A[g][nx] = lds_load<h8>(abase + g * kWideGroupBytes + 64u * ((k + 1u) >> 1) + 16u * ((k + 1u) & 1u));
        }
        h8 B[NM];
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) B[mt] = wide_finish(tf[mt][cur]);
#pragma unroll
        for (uint32_t g = 0; g < NG; ++g)
#pragma unroll
            for (int mt = 0; mt < NM; ++mt)
                C[mt][g] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[g][cur], B[mt], k ? C[mt][g] : zero, 0, 0, 0);
    }
    float df[NM];
#pragma unroll
    for (int mt = 0; mt < NM; ++mt) df[mt] = half_bits_to_float(wr[mt].d) * 0.125f;
#pragma unroll
    for (uint32_t g = 0; g < NG; ++g) {
        const uint32_t sbase = kWideScale + (buf * kWideGroups + g) * 64u;
#pragma unroll
        for (uint32_t q = 0; q < 8u; ++q) {
            const float xs = PB ? lds_load<float>(sbase + 4u * wide_pair_slot(q, hh)) : 1.0f;
#pragma unroll
            for (int mt = 0; mt < NM; ++mt)
                acc[mt][g][q] += (C[mt][g][2 * q] + C[mt][g][2 * q + 1]) * (PB ? df[mt] * xs : df[mt]);
        }
    }
}

// The stream over a row's superblocks: activations staged one superblock ahead (registers, then
// LDS behind a barrier), weights loaded one superblock ahead.
template <int NM, uint32_t NG, bool PB>
__device__ __forceinline__ void wide_rows_ng(uint8_t* lds, WideStage<PB>& st, uint32_t nsb,
                                             const uint8_t* const (&p0)[NM], const uint8_t* const (&p1)[NM],
                                             float (&acc)[NM][kWideGroups][8]) {
    WideRow cur[NM], nxt[NM];
#pragma unroll
    for (int mt = 0; mt < NM; ++mt) cur[mt].load(p0[mt], p1[mt], 0u);
    st.template load<NG>(0u);
    st.template store<NG>(lds, 0u);
    __syncthreads();
    for (uint32_t sb = 0; sb < nsb; ++sb) {
        const bool more = sb + 1u < nsb;
        const uint32_t nb = more ? sb + 1u : sb;
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) nxt[mt].load(p0[mt], p1[mt], nb);
        st.template load<NG>(nb);
        // The loads stay here, a superblock ahead of their use (the compiler would otherwise
        // sink them to it).
        asm volatile("" ::: "memory");
        wide_superblock<NM, NG, PB>(lds, sb & 1u, cur, acc);
        if (more) st.template store<NG>(lds, (sb + 1u) & 1u);
        __syncthreads();
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) cur[mt] = nxt[mt];
    }
}

// wide_rows_ng for the item's group count (block-uniform).
template <int NM, bool PB>
__device__ __forceinline__ void wide_rows(uint8_t* lds, WideStage<PB>& st, uint32_t nsb, uint32_t groups,
                                          const uint8_t* const (&p0)[NM], const uint8_t* const (&p1)[NM],
                                          float (&acc)[NM][kWideGroups][8]) {
    static_assert(kWideGroups == 2, "one or two groups");
    if (groups > 1u) wide_rows_ng<NM, 2, PB>(lds, st, nsb, p0, p1, acc);
    else wide_rows_ng<NM, 1, PB>(lds, st, nsb, p0, p1, acc);
}

// Entry a's fields through the plan's group list.
__device__ __forceinline__ const ActiveExpert& wide_entry(const MoeWorkspace& w, uint32_t a) {
    return ws_ptr<const ActiveExpert>(w, w.off_active)[a];
}

// ------------------------------------------------------------------------------------------
// Gate/up.
// ------------------------------------------------------------------------------------------

__global__ void __launch_bounds__(kWideWaves * 64u) k_wide_gateup(const MoeShape s, const MoeInputs in,
                                                                 const MoeWorkspace w) {
    extern __shared__ __align__(16) uint8_t lds[];
    const MoeHeader* hdr = ws_ptr<const MoeHeader>(w, w.off_header);
    const uint32_t nitems = uni(*gp(&hdr->reserved[0]));
    const uint32_t slabs = s.inter / 256u;
    const uint32_t item = blockIdx.x / slabs, slab = blockIdx.x - item * slabs;
    if (item >= nitems) return;
    const WideItem it = ws_ptr<const WideItem>(w, w.off_items)[item];
    const uint32_t a0 = uni(it.first), ne = uni(it.entries), groups = (ne + 1u) / 2u;
    wide_fill_table(lds);
    // Slot t of group g: entry a0 + 2g + t/8, slot t%8, its token's activation row.
    uint32_t ntok[2 * kWideGroups];
#pragma unroll
    for (uint32_t k = 0; k < 2u * kWideGroups; ++k) ntok[k] = k < ne ? uni(*gp(&wide_entry(w, a0 + k).ntok)) : 0u;
    auto rowid = [&](uint32_t g, uint32_t t) -> uint32_t {
        const uint32_t k = 2u * g + t / 8u, sl = t % 8u;
        uint32_t nt = 0;
#pragma unroll
        for (uint32_t kk = 0; kk < 2u * kWideGroups; ++kk) nt = kk == k ? ntok[kk] : nt;
        return sl < nt ? *gp(&wide_entry(w, a0 + k).tok[sl]) : ~0u;
    };
    WideStage<false> st;
    st.init(rowid, uni(*gp(&wide_entry(w, a0).tok[0])), s.width, ws_ptr<const _Float16>(w, w.off_x16),
            ws_ptr<const float>(w, w.off_xsc), 1u);
    const MoeExpert ex = ws_ptr<const MoeExpert>(w, w.off_gweights)[a0];
    vl_tiled_layout L;
    vl_make_layout(VL_TYPE_IQ2_XXS, s.inter, s.width, &L);
    const uint32_t wave = threadIdx.x >> 6, tile = slab * kWideWaves + wave;
    const uint8_t* g0 = uni_ptr(ex.gate);
    const uint8_t* u0 = uni_ptr(ex.up);
    const uint8_t* const p0[2] = {g0 + (uint64_t)tile * L.superblocks * 2048u, u0 + (uint64_t)tile * L.superblocks * 2048u};
    const uint8_t* const p1[2] = {g0 + L.plane1 + (uint64_t)tile * L.superblocks * 64u,
                                  u0 + L.plane1 + (uint64_t)tile * L.superblocks * 64u};
    float acc[2][kWideGroups][8];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (uint32_t g = 0; g < kWideGroups; ++g)
#pragma unroll
            for (int q = 0; q < 8; ++q) acc[mt][g][q] = 0.0f;
    __syncthreads();  // the table
    wide_rows<2, false>(lds, st, L.superblocks, groups, p0, p1, acc);

    // SwiGLU per (slot, row), then h of the block's 256 rows as hi/lo with one scale per slot.
    const uint32_t lane = threadIdx.x & 63u, n = lane & 31u, hh = lane >> 5;
    const uint32_t row = tile * 32u + n, F = s.inter;
    float h[kWideGroups][8];
    bool bad = false;
#pragma unroll
    for (uint32_t g = 0; g < kWideGroups; ++g) {
#pragma unroll
        for (uint32_t q = 0; q < 8u; ++q) {
            h[g][q] = 0.0f;
            const uint32_t t = wide_pair_slot(q, hh), k = 2u * g + t / 8u, sl = t % 8u;
            if (g < groups && k < ne) {
                const ActiveExpert& ae = wide_entry(w, a0 + k);
                if (sl < *gp(&ae.ntok)) {
                    // The token's activation scale, a power of two: exact.
                    const float xs = *gp(ws_ptr<const float>(w, w.off_xsc) + *gp(&ae.tok[sl]));
                    const float gv = acc[0][g][q] * xs, uv = acc[1][g][q] * xs;
                    const float v = swiglu(s.semantics, gv, uv, *gp(&ae.limit), *gp(&ae.apply_w) != 0u,
                                           *gp(&ae.route_w[sl]));
                    bad |= !isfinite(gv) || !isfinite(uv) || !isfinite(v);
                    h[g][q] = isfinite(v) ? v : 0.0f;
                }
            }
        }
    }
    if (__any(bad) && lane == 0) or_bits(&ws_ptr<MoeHeader>(w, w.off_header)->status, kStatusNonFiniteOutput);
    // Slot maxima over the block's rows: the 32 lanes of a half share their slots, the waves
    // meet in LDS.
    float* red = reinterpret_cast<float*>(lds + kWideRed);
#pragma unroll
    for (uint32_t g = 0; g < kWideGroups; ++g)
#pragma unroll
        for (uint32_t q = 0; q < 8u; ++q) {
            float m = fabsf(h[g][q]);
            for (int o = 16; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
            if (n == 0) red[(wave * kWideGroups + g) * 16u + wide_pair_slot(q, hh)] = m;
        }
    __syncthreads();
    _Float16* h16 = ws_ptr<_Float16>(w, w.off_h16);
    float* hsc = ws_ptr<float>(w, w.off_hsc);
#pragma unroll
    for (uint32_t g = 0; g < kWideGroups; ++g) {
        if (g >= groups) break;
#pragma unroll
        for (uint32_t q = 0; q < 8u; ++q) {
            const uint32_t t = wide_pair_slot(q, hh), k = 2u * g + t / 8u, sl = t % 8u;
            float m = 0.0f;
            for (uint32_t v = 0; v < kWideWaves; ++v) m = fmaxf(m, red[(v * kWideGroups + g) * 16u + t]);
            const int e = wide_exponent(m);
            if (k < ne && sl < ntok[k]) {
                const uint64_t r = (uint64_t)(a0 + k) * kMoeMaxTokens + sl;
                _Float16 hi, lo;
                split16(h[g][q], e, hi, lo);
                h16[(r * 2u) * F + row] = hi;
                h16[(r * 2u + 1u) * F + row] = lo;
                if (wave == 0 && n == 0) hsc[r * w.hblocks + slab] = __builtin_amdgcn_ldexpf(1.0f, -e);
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// Down.
// ------------------------------------------------------------------------------------------

__global__ void __launch_bounds__(kWideWaves * 64u) k_wide_down(const MoeShape s, const MoeInputs in,
                                                               const MoeWorkspace w) {
    extern __shared__ __align__(16) uint8_t lds[];
    const MoeHeader* hdr = ws_ptr<const MoeHeader>(w, w.off_header);
    const uint32_t nitems = uni(*gp(&hdr->reserved[0]));
    const uint32_t slabs = (s.width + 511u) / 512u, runs = (slabs + kWideDownSlabs - 1u) / kWideDownSlabs;
    const uint32_t item = blockIdx.x / runs, run = blockIdx.x - item * runs;
    if (item >= nitems) return;
    const WideItem it = ws_ptr<const WideItem>(w, w.off_items)[item];
    const uint32_t a0 = uni(it.first), ne = uni(it.entries), groups = (ne + 1u) / 2u;
    wide_fill_table(lds);
    uint32_t ntok[2 * kWideGroups];
#pragma unroll
    for (uint32_t k = 0; k < 2u * kWideGroups; ++k) ntok[k] = k < ne ? uni(*gp(&wide_entry(w, a0 + k).ntok)) : 0u;
    auto rowid = [&](uint32_t g, uint32_t t) -> uint32_t {
        const uint32_t k = 2u * g + t / 8u, sl = t % 8u;
        uint32_t nt = 0;
#pragma unroll
        for (uint32_t kk = 0; kk < 2u * kWideGroups; ++kk) nt = kk == k ? ntok[kk] : nt;
        return sl < nt ? (a0 + k) * kMoeMaxTokens + sl : ~0u;
    };
    WideStage<true> st;
    st.init(rowid, a0 * kMoeMaxTokens, s.inter, ws_ptr<const _Float16>(w, w.off_h16),
            ws_ptr<const float>(w, w.off_hsc), w.hblocks);
    const MoeExpert ex = ws_ptr<const MoeExpert>(w, w.off_gweights)[a0];
    vl_tiled_layout L;
    vl_make_layout(VL_TYPE_IQ2_XXS, s.width, s.inter, &L);
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u, n = lane & 31u, hh = lane >> 5;
    const uint8_t* d0 = uni_ptr(ex.down);
    float* ypart = ws_ptr<float>(w, w.off_ypart);
    const uint32_t H = s.width;
    __syncthreads();  // the table
    // Each wave takes two tiles of a 512-row slab (rows 32 (16 slab + wave) and 256 rows further),
    // so that every A fragment read from LDS feeds two MFMAs. A slab past the last full 256 rows
    // computes its first tile twice and stores it once.
    const uint32_t tiles = L.tiles;
    for (uint32_t sl0 = run * kWideDownSlabs; sl0 < slabs && sl0 < (run + 1u) * kWideDownSlabs; ++sl0) {
        const uint32_t t0 = sl0 * 2u * kWideWaves + wave, t1r = t0 + kWideWaves;
        const uint32_t t1 = t1r < tiles ? t1r : t0;
        const uint8_t* const p0[2] = {d0 + (uint64_t)t0 * L.superblocks * 2048u, d0 + (uint64_t)t1 * L.superblocks * 2048u};
        const uint8_t* const p1[2] = {d0 + L.plane1 + (uint64_t)t0 * L.superblocks * 64u,
                                      d0 + L.plane1 + (uint64_t)t1 * L.superblocks * 64u};
        float acc[2][kWideGroups][8];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (uint32_t g = 0; g < kWideGroups; ++g)
#pragma unroll
                for (int q = 0; q < 8; ++q) acc[mt][g][q] = 0.0f;
        wide_rows<2, true>(lds, st, L.superblocks, groups, p0, p1, acc);
#pragma unroll
        for (uint32_t g = 0; g < kWideGroups; ++g) {
            if (g >= groups) break;
#pragma unroll
            for (uint32_t q = 0; q < 8u; ++q) {
                const uint32_t t = wide_pair_slot(q, hh), k = 2u * g + t / 8u, sl = t % 8u;
                if (k < ne && sl < ntok[k]) {
                    float* y = ypart + ((uint64_t)(a0 + k) * kMoeMaxTokens + sl) * H;
                    y[t0 * 32u + n] = acc[0][g][q];
                    if (t1r < tiles) y[t1r * 32u + n] = acc[1][g][q];
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// Host side.
// ------------------------------------------------------------------------------------------

bool wide_shape_ok(const MoeShape& s) {
    return s.tokens > kMoeMaxTokens && s.gate_type == VL_TYPE_IQ2_XXS && s.down_type == VL_TYPE_IQ2_XXS &&
           s.width % 256u == 0 && s.inter % 256u == 0;
}

uint32_t wide_lds_bytes() { return kWideLdsBytes; }

hipError_t launch_wide_prep(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w, hipStream_t st) {
    hipLaunchKernelGGL(k_wide_prep, dim3(s.tokens), dim3(256), 0, st, s, in, w);
    return hipGetLastError();
}

hipError_t launch_wide_gateup(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w, hipStream_t st) {
    hipError_t e = ensure_dynamic_lds((const void*)k_wide_gateup, kWideLdsBytes);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_wide_gateup, dim3(w.max_items * (s.inter / 256u)), dim3(kWideWaves * 64u), kWideLdsBytes,
                       st, s, in, w);
    return hipGetLastError();
}

hipError_t launch_wide_down(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w, hipStream_t st) {
    hipError_t e = ensure_dynamic_lds((const void*)k_wide_down, kWideLdsBytes);
    if (e != hipSuccess) return e;
    const uint32_t runs = ((s.width + 511u) / 512u + kWideDownSlabs - 1u) / kWideDownSlabs;
    hipLaunchKernelGGL(k_wide_down, dim3(w.max_items * runs), dim3(kWideWaves * 64u), kWideLdsBytes, st, s, in, w);
    return hipGetLastError();
}

}  // namespace vl
