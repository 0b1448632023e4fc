// Single-token MoE layers (vl_moe_token.h): the gate/up kernel, which also routes the token, and
// the down kernel, which also combines the experts' outputs. The router kernel of vl_moe.hip runs
// first (router logits, selection keys, the token's activation limbs, zeroed counters).
//
// Routing, one token. Every wave of a gate/up block holds all E selection keys (PER per lane)
// and ranks a share of the candidates: the rank of expert c is the number of experts whose key
// is larger, or equal with a lower id, counted with one 64-bit compare and a ballot per register.
// The K experts of rank < K are the reference's top-k in its rank order
// (deepseek_v4_reference.cpp:243-247, qwen3_8_flash_next_reference.cpp:1217-1221); one wave then
// forms their weights with the reference's float64 arithmetic, adding in rank order.
//
// Gate/up. A block streams its share of the shared expert while the routing is formed, then its
// routed jobs. A job's h rows are SwiGLU(gate, up) of the semantics (execute_expert,
// deepseek_v4_graph.cpp:1826-1894; qwen38_expert_mlp_q8, qwen3_8_flash_next_reference.cpp:
// 1317-1342; routed_expert_iq1_s_iq3_xxs_f32, ggml_quantization.cpp:1678-1745), stored as floats
// with the maximum |h| of each 256-row block, from which the down kernel takes its limb exponents.
//
// Down. A block owns output tiles and every active expert's rows of them: it turns the experts'
// h into limbs in LDS, streams the down matrices and adds the experts' rows in the combine order
// (moe_forward, deepseek_v4_graph.cpp:2129-2266; qwen38_moe_block, qwen3_8_flash_next_reference.cpp:
// 1377-1421) without leaving the block, except for tiles of the stream-K region.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>

#include "vl_kernels.h"
#include "vl_moe_dev.h"
#include "vl_moe_token.h"
#include "vl_stream.h"

namespace vl {

// ------------------------------------------------------------------------------------------
// Partition (host and device).
// ------------------------------------------------------------------------------------------

// Piece of region X for block b: units [lo, hi); n chunks of cu units, the first starting at
// unit c0 * cu (the first and last chunks may be partial).
struct TokPiece {
    uint32_t lo, hi, n, c0;
};

// First unit of block b's piece of region X (a 32-bit division whenever the product fits).
__host__ __device__ inline uint32_t tok_piece_lo(const TokRegion& X, uint32_t b) {
    const uint64_t q = (uint64_t)b * X.total;
    return (q >> 32) ? (uint32_t)(q / X.blocks) : (uint32_t)q / X.blocks;
}

__host__ __device__ inline TokPiece tok_piece(const TokRegion& X, uint32_t b, uint32_t cu) {
    TokPiece p{0, 0, 0, 0};
    if (b >= X.blocks) return p;
    p.lo = tok_piece_lo(X, b);
    p.hi = tok_piece_lo(X, b + 1u);
    p.c0 = p.lo / cu;
    p.n = p.hi > p.lo ? (p.hi + cu - 1u) / cu - p.c0 : 0u;
    return p;
}

// The block of region X whose piece holds unit u (pieces are non-empty: blocks <= total).
__host__ __device__ inline uint32_t tok_block_of(const TokRegion& X, uint32_t u) {
    const uint64_t q = ((uint64_t)u + 1u) * X.blocks - 1u;
    return (q >> 32) ? (uint32_t)(q / X.total) : (uint32_t)q / X.total;
}

static TokRegion make_region(uint32_t total, uint32_t grid, uint32_t job0) {
    TokRegion r{total, total < grid ? total : grid, job0};
    if (total == 0) r.blocks = 0;
    return r;
}

static uint32_t tok_max_chunks(const TokPlan& p) {
    uint32_t m = 0;
    for (uint32_t b = 0; b < p.grid; ++b) {
        const uint32_t n = tok_piece(p.S, b, p.CU).n + tok_piece(p.R, b, p.CU).n + p.q * p.UJ / p.CU;
        m = n > m ? n : m;
    }
    return m;
}

// Jobs (a, t) = a * tiles + t over A active experts; the shared expert is the last one and forms
// region S; routed jobs are data-parallel except the remainder, region R.
TokPlan tok_plan_gateup(const MoeShape& s, uint32_t blocks) {
    TokPlan p{};
    p.grid = blocks;
    p.A = s.top_k + (s.has_shared ? 1u : 0u);
    p.tiles = (s.inter + 31u) / 32u;
    p.C = units_per_row(s.gate_type, s.width);
    p.CU = tok_chunk_units(s.gate_type);
    p.UJ = 2u * p.C;
    const uint32_t Jr = s.top_k * p.tiles;
    p.q = Jr / blocks;
    p.S = make_region(s.has_shared ? p.tiles * p.UJ : 0u, blocks, s.top_k * p.tiles);
    p.R = make_region((Jr - p.q * blocks) * p.UJ, blocks, p.q * blocks);
    p.max_chunks = tok_max_chunks(p);
    return p;
}

// Jobs are output tiles. With at least as many tiles as blocks, blocks own q tiles each and split
// the remainder; with fewer, either one tile per block (when that leaves less than a third of the
// blocks idle) or every tile split over all blocks.
TokPlan tok_plan_down(const MoeShape& s, uint32_t blocks) {
    TokPlan p{};
    p.A = s.top_k + (s.has_shared ? 1u : 0u);
    p.tiles = (s.width + 31u) / 32u;
    p.C = units_per_row(s.down_type, s.inter);
    p.CU = tok_chunk_units(s.down_type);
    p.UJ = p.A * p.C;
    p.S = make_region(0, blocks, 0);
    if (p.tiles >= blocks) {
        p.grid = blocks;
        p.q = p.tiles / blocks;
        p.R = make_region((p.tiles - p.q * blocks) * p.UJ, blocks, p.q * blocks);
    } else if (3u * p.tiles >= 2u * blocks) {
        p.grid = p.tiles;
        p.q = 1;
        p.R = make_region(0, p.grid, 0);
    } else {
        p.grid = blocks;
        p.q = 0;
        p.R = make_region(p.tiles * p.UJ, blocks, 0);
    }
    p.max_chunks = tok_max_chunks(p);
    return p;
}

// LDS of the gate/up kernel, from byte 0: decode tables, the token's limbs, its 2^-e per 256
// columns, chunk partials, counters and flags, the active list, combine entries, weight pointers
// of the active experts, the rare-path record, then the routing area: every expert's gate and up
// pointers (pools of up to kTokPtrTab experts), every expert's value, group maxima, the candidate
// list and the top-k by rank.
constexpr uint32_t kTokPtrTab = 256;
constexpr uint32_t kTokRareBytes = 256;  // TokRare, rounded up
constexpr uint32_t kTokMaxGroups = 64;   // group maxima of the routing threshold
struct TokGuLds {
    uint32_t xstage, xscale, part, desc, misc, act, comb, wptr, rare, ptab, val, gmax, cand, sel, bytes;
};
// misc words: the chunk counter, chunks done per segment of the S and R pieces, the chunks each
// such segment has, the refusal flag, one x-flag word per wave, the candidate count, one
// non-finite-key flag word per wave.
constexpr uint32_t kMiscGrab = 0, kMiscSeg = 1, kMiscSegN = kMiscSeg + 2 * kTokMaxSeg,
                   kMiscBad = kMiscSegN + 2 * kTokMaxSeg, kMiscWaveFlags = kMiscBad + 1,
                   kMiscCand = kMiscWaveFlags + kTokWaves, kMiscKeyFlags = kMiscCand + 1,
                   kMiscWords = kMiscKeyFlags + kTokWaves;

__host__ __device__ inline bool tok_has_ptab(uint32_t experts) { return experts + 1u <= kTokPtrTab + 1u; }

__host__ __device__ inline TokGuLds tok_lds_gu(uint32_t table_bytes, uint32_t width, uint32_t max_chunks,
                                               uint32_t experts) {
    TokGuLds l;
    l.xstage = table_bytes;
    l.xscale = l.xstage + (width / 32u) * 128u;
    l.part = (l.xscale + ((width + 255u) / 256u) * 4u + 15u) & ~15u;
    l.desc = l.part + max_chunks * 256u;
    l.misc = l.desc + max_chunks * 8u;
    l.act = (l.misc + kMiscWords * 4u + 15u) & ~15u;
    l.comb = l.act + kTokMaxActive * (uint32_t)sizeof(ActiveExpert);
    l.wptr = (l.comb + (kMoeMaxTopK + 1u) * (uint32_t)sizeof(CombineEntry) + 15u) & ~15u;
    l.rare = l.wptr + kTokMaxActive * 16u;
    l.ptab = l.rare + kTokRareBytes;
    l.val = l.ptab + (tok_has_ptab(experts) ? (experts + 1u) * 16u : 0u);
    l.gmax = (l.val + experts * 4u + 15u) & ~15u;
    l.cand = l.gmax + kTokMaxGroups * 4u;
    l.sel = l.cand + experts * 16u;
    l.bytes = l.sel + kMoeMaxTopK * 8u;
    return l;
}

// LDS of the down kernel: decode tables, the active experts' h limbs and 2^-e per 256 rows, chunk
// partials, counters, combine entries, down pointers of the active experts, every expert's down
// pointer (pools of up to kTokPtrTab experts).
struct TokDnLds {
    uint32_t hstage, hscale, part, desc, misc, comb, dptr, rare, ptab, eid, bytes;
};
__host__ __device__ inline TokDnLds tok_lds_dn(uint32_t table_bytes, uint32_t A, uint32_t inter,
                                               uint32_t max_chunks) {
    TokDnLds l;
    l.hstage = table_bytes;
    l.hscale = l.hstage + A * (inter / 32u) * 128u;
    l.part = (l.hscale + A * ((inter + 255u) / 256u) * 4u + 15u) & ~15u;
    l.desc = l.part + max_chunks * 256u;
    l.misc = l.desc + max_chunks * 8u;
    l.comb = (l.misc + kMiscWords * 4u + 15u) & ~15u;
    l.dptr = (l.comb + (kMoeMaxTopK + 1u) * (uint32_t)sizeof(CombineEntry) + 15u) & ~15u;
    l.rare = l.dptr + kTokMaxActive * 8u;
    l.ptab = l.rare + kTokRareBytes;
    l.eid = l.ptab + (kTokPtrTab + 1u) * 8u;
    l.bytes = l.eid + kTokMaxActive * 4u;
    return l;
}

constexpr uint32_t kLdsLimit = 160u * 1024u;

static uint32_t tab_bytes(uint32_t type) {
    return type == VL_TYPE_IQ2_XXS || type == VL_TYPE_IQ3_XXS ? kReplTableBytes
         : type == VL_TYPE_IQ1_S ? kIq1TableBytes : 0u;
}

// Keeps the compiler from moving the loads issued before it to after it (it would otherwise
// sink each load to its first use, and a prologue would wait one memory latency per load).
__device__ __forceinline__ void issue_fence() { asm volatile("" ::: "memory"); }
// A load from a constant table that stays where it is written: the pointer passes through an
// empty asm, so the compiler no longer knows it addresses constant memory (loads from which it may
// move past issue_fence).
__device__ __forceinline__ uint64_t ld_pinned(const uint64_t* p) {
    asm volatile("" : "+v"(p));
    return *gp(p);
}

// Decode tables of FMT for the token kernels, filled by nt threads (thread t of them): 8-byte
// source entries loaded unconditionally (clamped indices; entries past the last are not stored),
// then replicated into LDS. IQ2_XXS and IQ3_XXS: 128 sign entries (rows 0..127, upper halves) and
// 256 grid entries (rows 0..255, lower halves), 16 copies each (vl_decode.h), one entry per thread
// (nt >= 384); IQ1_S: 2048 entries, one copy, entries t, t + nt and t + 2 nt (nt >= 683).
template <uint32_t FMT>
struct TokTables {
    static constexpr bool kRepl = FMT == VL_TYPE_IQ2_XXS || FMT == VL_TYPE_IQ3_XXS;
    static constexpr uint32_t kEntries = kRepl ? 384u : FMT == VL_TYPE_IQ1_S ? 2048u : 0u;
    uint64_t v[3];
    __device__ __forceinline__ void load(uint32_t t, uint32_t nt) {
        if (kRepl) {
            const uint32_t i = t < kEntries ? t : kEntries - 1u;
            const uint64_t* src = FMT == VL_TYPE_IQ2_XXS ? (i < 128u ? g_tables.sign_sel + i : g_tables.iq2_codes + (i - 128u))
                                                         : (i < 128u ? g_tables.iq3_sel + i : g_tables.iq3_pm + (i - 128u));
            v[0] = ld_pinned(src);
        } else if (FMT == VL_TYPE_IQ1_S) {
#pragma unroll
            for (uint32_t j = 0; j < 3u; ++j) {
                const uint32_t i = t + j * nt;
                v[j] = ld_pinned(g_tables.iq1_codes + (i < kEntries ? i : kEntries - 1u));
            }
        }
    }
    __device__ __forceinline__ void store(uint8_t* lds, uint32_t t, uint32_t nt) const {
        if (kRepl) {
            if (t >= kEntries) return;
            const uint32_t row = t < 128u ? t * 256u + kTabB : (t - 128u) * 256u + kTabA;
            const uint4 q = make_uint4(lo32(v[0]), hi32(v[0]), lo32(v[0]), hi32(v[0]));
#pragma unroll
            for (uint32_t c = 0; c < kTabCopies / 2u; ++c) *reinterpret_cast<uint4*>(lds + row + 16u * c) = q;
        } else if (FMT == VL_TYPE_IQ1_S) {
#pragma unroll
            for (uint32_t j = 0; j < 3u; ++j)
                if (t + j * nt < kEntries) reinterpret_cast<uint64_t*>(lds)[t + j * nt] = v[j];
        }
    }
};

// Whether every block's piece of each stream-K region touches at most kTokMaxSeg jobs.
static bool segments_fit(const TokRegion& X, uint32_t UJ) {
    if (!X.total) return true;
    const uint32_t piece = (X.total + X.blocks - 1u) / X.blocks;
    return (piece + UJ - 1u) / UJ + 1u <= kTokMaxSeg;
}

bool tok_applies(const MoeShape& s, uint32_t blocks) {
    if (s.tokens != 1 || blocks == 0 || s.routing > kRouteGiven) return false;
    // IQ3_XXS units (six table reads a group) do not fit these kernels' registers without spills.
    if (s.gate_type == VL_TYPE_IQ3_XXS || s.down_type == VL_TYPE_IQ3_XXS) return false;
    const uint32_t A = s.top_k + (s.has_shared ? 1u : 0u);
    if (A > kTokMaxActive || s.experts > kTokMaxExperts) return false;
    const uint32_t cg = units_per_row(s.gate_type, s.width), cd = units_per_row(s.down_type, s.inter);
    if (cg % tok_chunk_units(s.gate_type) || cd % tok_chunk_units(s.down_type)) return false;
    const TokPlan g = tok_plan_gateup(s, blocks), d = tok_plan_down(s, blocks);
    if (!segments_fit(g.S, g.UJ) || !segments_fit(g.R, g.UJ) || !segments_fit(d.R, d.UJ)) return false;
    // The data-parallel finishes keep their sums where the activations were staged.
    if (2ull * g.q * 256u > 4ull * s.width || (uint64_t)d.q * A * 256u > 4ull * A * s.inter) return false;
    if (tok_lds_gu(tab_bytes(s.gate_type), s.width, g.max_chunks, s.experts).bytes > kLdsLimit) return false;
    if (tok_lds_dn(tab_bytes(s.down_type), A, s.inter, d.max_chunks).bytes > kLdsLimit) return false;
    return true;
}

// Records: gate/up [2 regions][grid][kTokMaxSeg][2 matrices][64]; down [grid][kTokMaxSeg][A][64].
__host__ __device__ inline uint64_t gu_record_bytes(uint32_t blocks) { return 2ull * blocks * kTokMaxSeg * 2u * 64u * 4u; }

uint64_t tok_record_bytes(const MoeShape& s, uint32_t blocks) {
    if (!tok_applies(s, blocks)) return 0;
    const uint32_t A = s.top_k + (s.has_shared ? 1u : 0u);
    return gu_record_bytes(blocks) + (uint64_t)blocks * kTokMaxSeg * A * 64u * 4u;
}

// ------------------------------------------------------------------------------------------
// Chunks.
// ------------------------------------------------------------------------------------------

// A chunk as the partition defines it: count units from unit v of job `job`.
struct TokChunk {
    uint32_t count;   // units (0: no chunk)
    uint32_t job;     // job index (gate/up: a * tiles + t; down: output tile)
    uint32_t v;       // first unit within the job
    uint32_t region;  // 0 S, 1 R, 2 D
    uint32_t seg;     // S/R: job index within the block's piece
};

// Chunk k of a block: its S chunks, then its R chunks, then its D chunks.
template <uint32_t CU>
__host__ __device__ inline TokChunk tok_chunk(const TokPlan p, uint32_t b, const TokPiece ps, const TokPiece pr,
                                              uint32_t k) {
    TokChunk c{0, 0, 0, 2, 0};
    const uint32_t nd = p.q * p.UJ / CU;
    uint32_t lo, hi, c0, job0;
    if (k < ps.n) {
        lo = ps.lo, hi = ps.hi, c0 = ps.c0, job0 = p.S.job0;
        c.region = 0;
    } else if (k < ps.n + pr.n) {
        k -= ps.n;
        lo = pr.lo, hi = pr.hi, c0 = pr.c0, job0 = p.R.job0;
        c.region = 1;
    } else if (k < ps.n + pr.n + nd) {
        const uint32_t u = (k - ps.n - pr.n) * CU;
        c.count = CU;
        c.job = b * p.q + u / p.UJ;
        c.v = u % p.UJ;
        return c;
    } else {
        return c;
    }
    const uint32_t s0 = (c0 + k) * CU;
    const uint32_t u0 = s0 > lo ? s0 : lo;
    const uint32_t u1 = s0 + CU < hi ? s0 + CU : hi;
    c.count = u1 - u0;
    c.job = job0 + u0 / p.UJ;
    c.v = u0 % p.UJ;
    c.seg = u0 / p.UJ - lo / p.UJ;
    return c;
}

// A chunk as the wave loop uses it, decoded from the block's LDS table (no division on the way):
// unit `col` of a matrix row and `count` units, of tile t of active expert a (gate/up: matrix m of
// job a * tiles + t; down: output tile t, expert a).
struct TokWork {
    uint32_t count, t, a, m, col, region, seg;
};

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

__host__ __device__ inline u32x2 encode_work(const TokChunk& c, uint32_t tiles, uint32_t C, bool gate_up) {
    uint32_t t, a, m;
    if (gate_up) {
        a = c.job / tiles;
        t = c.job - a * tiles;
        m = c.v / C;
    } else {
        t = c.job;
        a = c.v / C;
        m = 0;
    }
    const u32x2 r = {t | (a << 16) | (m << 21) | (c.region << 22) | (c.seg << 24), (c.v % C) | (c.count << 16)};
    return r;
}

__host__ __device__ inline TokWork decode_work(u32x2 d) {
    TokWork w;
    w.t = d.x & 0xffffu;
    w.a = (d.x >> 16) & 31u;
    w.m = (d.x >> 21) & 1u;
    w.region = (d.x >> 22) & 3u;
    w.seg = (d.x >> 24) & 7u;
    w.col = d.y & 0xffffu;
    w.count = d.y >> 16;
    return w;
}

// Chunks [first, first + n) (indices within the region's chunks of the block) of segment `seg` of a
// piece.
template <uint32_t CU>
__host__ __device__ inline void seg_chunks(const TokPlan& p, const TokPiece P, uint32_t seg, uint32_t& first,
                                           uint32_t& n) {
    const uint32_t j = P.lo / p.UJ + seg;
    const uint32_t lo = j * p.UJ > P.lo ? j * p.UJ : P.lo;
    const uint32_t hi = (j + 1u) * p.UJ < P.hi ? (j + 1u) * p.UJ : P.hi;
    first = lo / CU - P.c0;
    n = (hi + CU - 1u) / CU - lo / CU;
}

// Contributing blocks [first, last] of job j of region X.
__device__ __forceinline__ void job_blocks(const TokPlan& p, const TokRegion& X, uint32_t j,
                                           uint32_t& first, uint32_t& last) {
    const uint32_t lo = (j - X.job0) * p.UJ;
    first = tok_block_of(X, lo);
    last = tok_block_of(X, lo + p.UJ - 1u);
}

// The kernels declare no static LDS, so dynamic LDS starts at address 0 and LDS data is named by
// byte address.
__device__ __forceinline__ uint8_t* lds_base() {
    extern __shared__ __align__(16) uint8_t tok_lds[];
    return tok_lds;
}
template <typename T>
__device__ __forceinline__ VL_LDS T* lptr(uint32_t addr) {
    return reinterpret_cast<VL_LDS T*>((uintptr_t)addr);
}
__device__ __forceinline__ uint32_t lds_u32(uint32_t addr) { return lds_load<uint32_t>(addr); }
__device__ __forceinline__ float lds_f32(uint32_t addr) { return lds_load<float>(addr); }
__device__ __forceinline__ void lds_st_u32(uint32_t addr, uint32_t v) { *lptr<uint32_t>(addr) = v; }
__device__ __forceinline__ void lds_st_f32(uint32_t addr, float v) { *lptr<float>(addr) = v; }
__device__ __forceinline__ uint32_t lds_add(uint32_t addr, uint32_t v) {
    return __hip_atomic_fetch_add(lptr<uint32_t>(addr), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// A struct to and from LDS word by word (a copy constructor cannot take an LDS reference).
template <typename T>
__device__ __forceinline__ T lds_get(uint32_t addr) {
    static_assert(sizeof(T) % 4 == 0, "word-sized struct");
    T v;
    uint32_t* d = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
    for (uint32_t i = 0; i < sizeof(T) / 4; ++i) d[i] = lds_load<uint32_t>(addr + 4u * i);
    return v;
}
template <typename T>
__device__ __forceinline__ void lds_put(uint32_t addr, const T& v) {
    static_assert(sizeof(T) % 4 == 0, "word-sized struct");
    const uint32_t* s = reinterpret_cast<const uint32_t*>(&v);
#pragma unroll
    for (uint32_t i = 0; i < sizeof(T) / 4; ++i) *lptr<uint32_t>(addr + 4u * i) = s[i];
}
// This wave's LDS stores have been performed (LDS serves a block's requests in order, so a later
// LDS atomic of this wave is seen after them).
__device__ __forceinline__ void lds_settle() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// This lane's sum of the LDS partials of chunks k0 .. k0 + n - 1 (256-byte slots from part), added
// in chunk order with eight reads in flight.
__device__ __forceinline__ float sum_parts(uint32_t part, uint32_t k0, uint32_t n) {
    const uint32_t base = part + k0 * 256u + (threadIdx.x & 63u) * 4u;
    float v = 0.0f;
    for (uint32_t i0 = 0; i0 < n; i0 += 8u) {
        float t[8];
#pragma unroll
        for (uint32_t j = 0; j < 8u; ++j) t[j] = i0 + j < n ? lds_f32(base + (i0 + j) * 256u) : 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < 8u; ++j)
            if (i0 + j < n) v += t[j];
    }
    return v;
}
__device__ __forceinline__ double readlane_f64(double v, uint32_t k) {
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, k);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), k);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ float readlane_f32(float v, uint32_t k) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), k));
}

// Next chunk index for this wave (one LDS atomic, result uniform).
__device__ __forceinline__ uint32_t grab(uint32_t misc) {
    uint32_t k = 0;
    if ((threadIdx.x & 63u) == 0) k = lds_add(misc + 4u * kMiscGrab, 1u);
    return uni(k);
}

// OR of a predicate over the block through one LDS word per wave (flags, no initialisation
// needed: every wave writes its own word); contains a block barrier.
__device__ __forceinline__ bool block_or(bool v, uint32_t flags) {
    const bool wv = __any(v);
    if ((threadIdx.x & 63u) == 0) lds_st_u32(flags + 4u * (threadIdx.x >> 6), wv ? 1u : 0u);
    __syncthreads();
    uint32_t r = 0;
    for (uint32_t i = 0; i < (blockDim.x >> 6); ++i) r |= lds_u32(flags + 4u * i);
    return r != 0;
}

// ------------------------------------------------------------------------------------------
// The wave loop: a chunk's units are loaded one chunk ahead of the processing position.
//
// Ctx interface (values wave-uniform):
//   TokWork chunk(uint32_t k)                 the block's chunk k (count 0 past the last)
//   TileRef tref(const TokWork&)              weight planes of the chunk's matrix tile
//   ASrc<true, 128> asrc(const TokWork&)      the chunk's activation limbs (LDS)
//   float scale(const TokWork&, uint32_t c)   2^-e of the activations of unit c of the row
//   bool done(const TokWork&)                 counts a stream-K chunk; true when it ended its segment
//   void segment(const TokWork&)              the hand-off of a completed segment
//   uint32_t part, misc, ng;                  LDS partials, LDS counters, groups per row
// ------------------------------------------------------------------------------------------

// This lane's index, opaque to loop-invariant code motion: the per-lane load offsets derived from it
// are then formed next to each load (two VALU) instead of being hoisted out of the wave loop as
// 64-bit values that crowd out the chunk buffers.
__device__ __forceinline__ uint32_t lane_here() {
    uint32_t l = threadIdx.x & 63u;
    asm volatile("" : "+v"(l));
    return l;
}

// load_chunk for the wave loop of this file, with the per-lane offsets formed at each load.
template <uint32_t FMT>
__device__ __forceinline__ void tok_load(const TileRef& tr, uint32_t c, uint32_t ng, Chunk& ch) {
    const uint32_t lane = lane_here(), n = lane & 31u, hh = lane >> 5;
    if (FMT == VL_TYPE_IQ2_XXS) {
        const uint8_t* P = tr.p0 + (uint64_t)c * 2048u;
        ch.q0 = ld_stream(P + lane * 32u);
        ch.q1 = ld_stream(P + lane * 32u + 16u);
        ch.d0 = ld_u16(tr.p1 + (uint64_t)c * 64u + n * 2u);
    } else if (FMT == VL_TYPE_IQ1_S) {
        const uint8_t* Q = tr.p0 + (uint64_t)c * 1024u;
        ch.q0 = ld_stream(Q + n * 16u);
        ch.q1 = ld_stream(Q + 512u + n * 16u);
        ch.q2 = ld_stream(tr.p1 + (uint64_t)c * 512u + n * 16u);
        ch.d0 = ld_u16(tr.p2 + (uint64_t)c * 64u + n * 2u);
    } else if (FMT == VL_TYPE_Q8_0) {
        uint4 q[4];
        uint32_t d[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t G = 4u * c + b;
            if (G < ng) {
                q[b] = ld_stream(tr.p0 + (uint64_t)G * 1024u + (n * 32u + hh * 16u));
                d[b] = ld_u16(tr.p1 + (uint64_t)G * 64u + n * 2u);
            } else {
                q[b] = make_uint4(0, 0, 0, 0);
                d[b] = 0;
            }
        }
        ch.q0 = q[0]; ch.q1 = q[1]; ch.q2 = q[2]; ch.q3 = q[3];
        ch.d0 = d[0] | (d[1] << 16);
        ch.d1 = d[2] | (d[3] << 16);
    } else {
        load_chunk<FMT>(tr, c, ng, ch);
    }
}

template <uint32_t FMT, uint32_t CU, typename Ctx>
__device__ __forceinline__ void issue(const Ctx& ctx, const TokWork& c, Chunk (&buf)[CU]) {
    const TileRef tr = c.count ? ctx.tref(c) : idle_tile();
    const uint32_t c0 = c.col;
#pragma unroll
    for (uint32_t i = 0; i < CU; ++i) {
        const bool live = i < c.count;
        tok_load<FMT>(live ? tr : idle_tile(), live ? c0 + i : 0u, ctx.ng, buf[i]);
    }
}

// A fragment of one token's limbs from LDS into v. The token occupies A rows 0, 1, 4 and 5 (its
// four limbs). Row m of the product depends on A row m alone, and the rows of other token slots
// are never read from the result, so only the eight lanes that supply the token's rows read LDS
// (an eighth of a full-wave read) and the other lanes keep whatever v held.
__device__ __forceinline__ void tok_afrag(i32x4& v, uint32_t addr) {
    if (((threadIdx.x & 31u) & ~5u) == 0u) v = lds_load<i32x4>(addr);
}

// One unit of one token: the lane's share of the partial dot products of its row (the high limbs'
// share in lanes 32..63, scaled by hs = 65536 there) over the unit's columns, times fs = 2^-e of the
// token's exponent block. The A fragments come from LDS (aoff: this lane's limb row; groups 128
// bytes apart) one group ahead of their MFMA, with the next group's table reads; exact integer
// sums per group and superblock as in process_chunk.
template <uint32_t FMT>
__device__ __forceinline__ float tok_unit(const Chunk& ch, uint32_t c, uint32_t ng, uint32_t aoff, float hs,
                                          float fs) {
    const uint32_t lane = threadIdx.x & 63u;
    const int hh = (int)(lane >> 5);
    const uint32_t lane_off = (lane % kTabCopies) * 8u;
    const i32x16 zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    if (FMT == VL_TYPE_Q8_0) {
        float acc = 0.0f;
        i32x4 anext = {0, 0, 0, 0};
        tok_afrag(anext, aoff + 4u * c * 128u);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t G = 4u * c + b;
            if (G >= ng) break;
            const i32x4 afr = anext;
            if (b + 1 < 4 && G + 1 < ng) tok_afrag(anext, aoff + (G + 1u) * 128u);
            const uint4& q = b == 0 ? ch.q0 : b == 1 ? ch.q1 : b == 2 ? ch.q2 : ch.q3;
            i32x4 bfr;
            bfr[0] = (int)q.x; bfr[1] = (int)q.y; bfr[2] = (int)q.z; bfr[3] = (int)q.w;
            const i32x16 r = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr, bfr, zero16, 0, 0, 0);
            const uint32_t dw = b < 2 ? ch.d0 : ch.d1;
            const float d = half_bits_to_float(dw >> (16 * (b & 1))) * hs;
            acc += (d * fs) * ((float)r[0] + 256.0f * (float)r[1]);
        }
        return acc;
    }
    int acc0 = 0, acc1 = 0;
    i32x4 anext = {0, 0, 0, 0};
    tok_afrag(anext, aoff + 8u * c * 128u);
    if (FMT == VL_TYPE_IQ2_XXS) {
        ChunkDecoder<FMT> dec;
        dec.init(ch);
        Iq2Fetch tnext = fetch_iq2_xxs(dec.w, 0, lane_off);
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const i32x4 afr = anext;
            const Iq2Fetch t = tnext;
            if (g + 1 < 8) {
                tok_afrag(anext, aoff + (8u * c + g + 1u) * 128u);
                tnext = fetch_iq2_xxs(dec.w, g + 1, lane_off);
            }
            const int sc = (int)bfe(g < 4 ? dec.sc_lo : dec.sc_hi, 8u * (uint32_t)(g & 3), 8);
            const i32x16 r = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr, finish_iq2_xxs(t), zero16, 0, 0, 0);
            acc0 += __mul24(sc, r[0]);
            acc1 += __mul24(sc, r[1]);
        }
    } else {  // IQ1_S
        auto qs = [&](int g) { return word(g < 4 ? ch.q0 : ch.q1, g & 3); };
        auto qh = [&](int g) { return (word(ch.q2, g >> 1) >> (16 * (g & 1))) & 0xffffu; };
        Iq1Fetch tnext = fetch_iq1_s(qs(0), qh(0), hh);
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const i32x4 afr = anext;
            const Iq1Fetch t = tnext;
            if (g + 1 < 8) {
                tok_afrag(anext, aoff + (8u * c + g + 1u) * 128u);
                tnext = fetch_iq1_s(qs(g + 1), qh(g + 1), hh);
            }
            const int sc = 2 * (int)((qh(g) >> 12) & 7u) + 1;
            const i32x16 r = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr, finish_iq1_s(t), zero16, 0, 0, 0);
            acc0 += __mul24(sc, r[0]);
            acc1 += __mul24(sc, r[1]);
        }
    }
    const float df = half_bits_to_float(ch.d0) * (unit_factor<FMT>() * hs);
    return (df * fs) * ((float)acc0 + 256.0f * (float)acc1);
}

// Processes a chunk and stores its partials; true when it completed its stream-K segment in this
// block (Ctx::done counts it).
template <uint32_t FMT, uint32_t CU, typename Ctx>
__device__ __forceinline__ bool consume(const Ctx& ctx, const TokWork& c, uint32_t k, const Chunk (&buf)[CU]) {
    const uint32_t aoff = ctx.asrc(c).off;
    const uint32_t c0 = c.col;
    const float hs = (threadIdx.x & 32u) ? 65536.0f : 1.0f;
    float acc = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < CU; ++i)
        if (i < c.count) acc += tok_unit<FMT>(buf[i], c0 + i, ctx.ng, aoff, hs, ctx.scale(c, c0 + i));
    lds_st_f32(ctx.part + k * 256u + (threadIdx.x & 63u) * 4u, acc);
    return ctx.done(c);
}

// The segment a stream pass completed (n = 1), to be handed off; `next` is a chunk index taken
// from the counter, already issued into the wave's buffer when pf is set and not yet loaded
// otherwise.
struct TokPass {
    uint32_t n, next, pf;
    TokWork s0;
};

// One pass of the wave loop: chunk ka (already issued into bufA when `issued`; count 0: none),
// then chunks from the block's counter. A wave has one chunk in flight: sixteen waves per CU with
// one unit each keep the memory system busiest on MI355X, while deeper per-wave queues let the
// CU's oldest waves take more than their share and lengthen the block's tail. IQ2_XXS waves issue
// the next chunk before processing the current one, so a load is in flight while they compute
// (iq2_moe 49.2 -> 47.9 us per layer); Q8_0 chunks, four loads each, measured slower that way
// (q8_moe 40.4 -> 41.4 us) and are loaded after the previous chunk is processed. The next chunk
// index is taken before the current chunk is processed, so the LDS counter's latency is hidden.
// A pass ends when the counter passes the block's last chunk (n = 0), or after a chunk completed
// a stream-K segment; the pass then returns the segment and the chunk index taken next (pf: that
// chunk is already issued into bufA).
template <uint32_t FMT>
__host__ __device__ constexpr bool tok_prefetch() { return FMT == VL_TYPE_IQ2_XXS; }

template <uint32_t FMT, uint32_t CU, typename Ctx>
__device__ __forceinline__ TokPass tok_pass(const Ctx& ctx, uint32_t ka, TokWork ca, Chunk (&bufA)[CU], bool issued) {
    TokPass r;
    r.n = 0;
    r.next = 0;
    r.pf = 0;
    if (!issued) issue<FMT, CU>(ctx, ca, bufA);
    if (!ca.count) {
        ka = grab(ctx.misc);
        ca = ctx.chunk(ka);
        issue<FMT, CU>(ctx, ca, bufA);
    }
    if constexpr (tok_prefetch<FMT>()) {
        Chunk bufB[CU];
        for (;;) {
            if (!ca.count) break;
            const uint32_t kn = grab(ctx.misc);
            const TokWork cn = ctx.chunk(kn);
            issue<FMT, CU>(ctx, cn, bufB);
            issue_fence();  // the next chunk's loads stay ahead of this chunk's processing
            const bool seg = consume<FMT, CU>(ctx, ca, ka, bufA);
#pragma unroll
            for (uint32_t i = 0; i < CU; ++i) bufA[i] = bufB[i];
            if (seg) {
                r.n = 1;
                r.s0 = ca;
                r.next = kn;
                r.pf = 1;
                return r;
            }
            ka = kn;
            ca = cn;
        }
    } else {
        for (;;) {
            if (!ca.count) break;
            const uint32_t kn = grab(ctx.misc);
            if (consume<FMT, CU>(ctx, ca, ka, bufA)) {
                r.n = 1;
                r.s0 = ca;
                r.next = kn;
                return r;
            }
            ka = kn;
            ca = ctx.chunk(ka);
            issue<FMT, CU>(ctx, ca, bufA);
        }
    }
    return r;
}

// The wave loop: passes until the block's chunks are exhausted, each completed segment handed off
// (Ctx::segment, out of line) between passes.
template <uint32_t FMT, uint32_t CU, typename Ctx>
__device__ __forceinline__ void tok_stream(const Ctx& ctx, uint32_t ka, TokWork ca, Chunk (&bufA)[CU]) {
    bool issued = true;
    for (;;) {
        const TokPass r = tok_pass<FMT, CU>(ctx, ka, ca, bufA, issued);
        if (!r.n) return;
        ctx.segment(r.s0);
        ka = r.next;
        ca = ctx.chunk(ka);
        issued = r.pf != 0;
    }
}

// ------------------------------------------------------------------------------------------
// Routing of the token (gate/up prologue).
// ------------------------------------------------------------------------------------------

// The route of the token in wave 0: lane k < K holds the expert of rank k and its weight.
struct TokRoute {
    uint32_t id;
    float wt;
    bool bad;  // the token is refused (wave-uniform)
};

// Learned and softmax routing of the token by the whole block. The reference takes the K largest
// selection keys, ties to the lower id, in rank order (deepseek_v4_reference.cpp:243-247,
// qwen3_8_flash_next_reference.cpp:1217-1221); here every expert's key is paired with its
// complemented id into a 64-bit key, so that rank order is descending 64-bit order, and the rank
// of a candidate is the number of candidates with a larger 64-bit key.
//
// Only keys at or above a threshold compete: the maxima of groups of G consecutive experts bound
// the top-k from below (the K-th largest group maximum is at most the K-th largest key, since K
// groups each hold a key at least that large). With fewer than 2K groups every expert competes.
__host__ __device__ inline uint32_t tok_group(uint32_t E, uint32_t K) {
    return E >= 32u * K ? 16u : E >= 16u * K ? 8u : E >= 8u * K ? 4u : 0u;
}

// Maximum over aligned groups of G = 4, 8 or 16 lanes (every lane active); every lane of a group
// receives its group's maximum. The DPP "old" value 0 is the identity of the maximum.
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v, uint32_t G) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xb1, 0xf, 0xf, false));  // quad [1,0,3,2]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4e, 0xf, 0xf, false));  // quad [2,3,0,1]
    if (G >= 8u) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false));  // half-row mirror
    if (G >= 16u) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xf, 0xf, false));  // row mirror
    return v;
}

__device__ __forceinline__ uint64_t route_key64(uint32_t key, uint32_t id) { return ((uint64_t)key << 32) | (uint32_t)~id; }

// A candidate in LDS: its 64-bit key and its value (learned: the score; softmax: the logit).
struct TokCand {
    uint64_t ck;
    float val;
    uint32_t pad;
};

// Before the first barrier, every thread (thread tid holds expert tid's key and score): the
// expert's value into LDS, its group's maximum, and per wave whether any key marks a non-finite
// logit, score or selection bias (a key of 1 or less; activate_gate_logits and require_finite,
// deepseek_v4_reference.cpp:155-165, :236-239). Returns the expert's value.
__device__ __forceinline__ float route_stage(const MoeShape& s, uint32_t key, float score, uint32_t val,
                                             uint32_t gmax, uint32_t misc, uint32_t G) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, E = s.experts;
    const bool live = tid < E;
    const uint32_t k = live ? key : 0u;
    const float v = s.routing == kRouteSoftmax ? (k > 1u ? key_float(k) : 0.0f) : score;
    if (live) lds_st_f32(val + 4u * tid, v);
    const bool bad = __any(live && k <= 1u);
    if (lane == 0) lds_st_u32(misc + 4u * (kMiscKeyFlags + wave), bad ? 1u : 0u);
    if (G && (tid & ~63u) < E) {
        const uint32_t m = group_max_u32(k, G);
        if (live && tid % G == 0u) lds_st_u32(gmax + 4u * (tid / G), m);
    }
    return v;
}

// After the first barrier, the waves that hold experts: the threshold (the K-th largest group
// maximum, equal maxima ranked by group) and the candidates, the experts whose key reaches it,
// appended to the candidate list in any order (their ranks do not depend on it). Lane i reads
// group i's maximum once; the comparisons go through readlane, not LDS.
__device__ __forceinline__ void route_candidates(const MoeShape& s, uint32_t key, float v, uint32_t gmax,
                                                 uint32_t cand, uint32_t misc, uint32_t G) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, E = s.experts, K = s.top_k;
    if ((tid & ~63u) >= E) return;
    uint32_t t0 = 0;
    if (G) {
        const uint32_t ng = (E + G - 1u) / G;  // 2K <= ng <= 64
        const uint32_t gm = lane < ng ? lds_u32(gmax + 4u * lane) : 0u;
        uint32_t rank = 0;
        for (uint32_t j = 0; j < ng; ++j) {
            const uint32_t gj = (uint32_t)__builtin_amdgcn_readlane((int)gm, j);
            rank += (gj > gm || (gj == gm && j < lane)) ? 1u : 0u;
        }
        const uint64_t hit = __ballot(lane < ng && rank == K - 1u);
        t0 = (uint32_t)__builtin_amdgcn_readlane((int)gm, (uint32_t)__builtin_ctzll(hit));
    }
    if (tid < E && key >= t0) {
        const uint32_t i = lds_add(misc + 4u * kMiscCand, 1u);
        VL_LDS TokCand* c = lptr<TokCand>(cand + 16u * i);
        c->ck = route_key64(key, tid);
        c->val = v;
    }
}

// Ranks of the candidates; those of rank < K go to the top-k list (sel: id and value by rank).
// Up to 64 candidates: wave 0, lane i holding candidate i and comparing through readlane. More:
// thread i of the block for candidate i, comparing against LDS.
__device__ __forceinline__ void route_rank_wave(uint32_t n, uint32_t K, uint32_t cand, uint32_t sel) {
    const uint32_t lane = threadIdx.x & 63u;
    uint64_t c = 0;
    float v = 0.0f;
    if (lane < n) {
        const VL_LDS TokCand* e = lptr<TokCand>(cand + 16u * lane);
        c = e->ck;
        v = e->val;
    }
    const uint32_t clo = (uint32_t)c, chi = (uint32_t)(c >> 32);
    uint32_t rank = 0;
    for (uint32_t j = 0; j < n; ++j) {
        const uint64_t cj = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)chi, j) << 32) |
                            (uint32_t)__builtin_amdgcn_readlane((int)clo, j);
        rank += cj > c ? 1u : 0u;
    }
    if (lane < n && rank < K) {
        lds_st_u32(sel + 8u * rank, ~clo);
        lds_st_f32(sel + 8u * rank + 4u, v);
    }
}
__device__ __forceinline__ void route_rank_block(uint32_t n, uint32_t K, uint32_t cand, uint32_t sel) {
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const VL_LDS TokCand* e = lptr<TokCand>(cand + 16u * i);
        const uint64_t c = e->ck;
        uint32_t rank = 0;
        for (uint32_t j = 0; j < n; ++j) rank += lptr<TokCand>(cand + 16u * j)->ck > c ? 1u : 0u;
        if (rank < K) {
            lds_st_u32(sel + 8u * rank, ~(uint32_t)c);
            lds_st_f32(sel + 8u * rank + 4u, e->val);
        }
    }
}

// Learned and softmax routing of the token by wave 0 alone, for pools of up to kTokWaveRoute
// experts: lane l holds the keys and scores of experts l, l + 64, l + 128 and l + 192. The same
// threshold, candidates and ranks as the block version above; the candidate list is formed with a
// ballot prefix instead of an LDS counter. Every LDS word it writes is read back by the same wave,
// so no barrier is needed and the other waves fill LDS meanwhile. Leaves the top-k list in sel and
// the non-finite-key flag in misc (the first key-flag word; the others zero) for route_weights.
constexpr uint32_t kTokWaveRoute = 256;
__device__ __forceinline__ void route_wave0(const MoeShape& s, const uint32_t (&key)[4], const float (&score)[4],
                                            uint32_t val, uint32_t gmax, uint32_t cand, uint32_t sel,
                                            uint32_t misc) {
    const uint32_t lane = threadIdx.x & 63u, E = s.experts, K = s.top_k, G = tok_group(E, K);
    uint32_t k[4];
    float v[4];
    bool bad = false;
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t e = lane + 64u * j;
        const bool live = e < E;
        k[j] = live ? key[j] : 0u;
        v[j] = s.routing == kRouteSoftmax ? (k[j] > 1u ? key_float(k[j]) : 0.0f) : score[j];
        if (live) lds_st_f32(val + 4u * e, v[j]);
        bad |= live && k[j] <= 1u;
        if (G && 64u * j < E) {
            const uint32_t m = group_max_u32(k[j], G);
            if (live && e % G == 0u) lds_st_u32(gmax + 4u * (e / G), m);
        }
    }
    const bool anybad = __any(bad);
    if (lane < kTokWaves) lds_st_u32(misc + 4u * (kMiscKeyFlags + lane), lane == 0 && anybad ? 1u : 0u);
    issue_fence();  // the stores above stay ahead of the reads below (one wave: LDS keeps its order)
    uint32_t t0 = 0;
    if (G) {
        const uint32_t ng = (E + G - 1u) / G;  // 2K <= ng <= 64
        const uint32_t gm = lane < ng ? lds_u32(gmax + 4u * lane) : 0u;
        uint32_t rank = 0;
        for (uint32_t j = 0; j < ng; ++j) {
            const uint32_t gj = (uint32_t)__builtin_amdgcn_readlane((int)gm, j);
            rank += (gj > gm || (gj == gm && j < lane)) ? 1u : 0u;
        }
        const uint64_t hit = __ballot(lane < ng && rank == K - 1u);
        t0 = (uint32_t)__builtin_amdgcn_readlane((int)gm, (uint32_t)__builtin_ctzll(hit));
    }
    uint32_t n = 0;
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t e = lane + 64u * j;
        const bool c = e < E && k[j] >= t0;
        const uint64_t mask = __ballot(c);
        if (c) {
            const uint32_t i = n + __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                             __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
            VL_LDS TokCand* cc = lptr<TokCand>(cand + 16u * i);
            cc->ck = route_key64(k[j], e);
            cc->val = v[j];
        }
        n += (uint32_t)__builtin_popcountll(mask);
    }
    issue_fence();
    if (n <= 64u) {
        route_rank_wave(n, K, cand, sel);
    } else {
        for (uint32_t i = lane; i < n; i += 64u) {
            const VL_LDS TokCand* e = lptr<TokCand>(cand + 16u * i);
            const uint64_t c = e->ck;
            uint32_t rank = 0;
            for (uint32_t j = 0; j < n; ++j) rank += lptr<TokCand>(cand + 16u * j)->ck > c ? 1u : 0u;
            if (rank < K) {
                lds_st_u32(sel + 8u * rank, ~(uint32_t)c);
                lds_st_f32(sel + 8u * rank + 4u, e->val);
            }
        }
    }
    issue_fence();
}

// Wave 0 once the top-k list is complete: lane k < K takes the expert of rank k and forms its
// weight with the reference's float64 arithmetic. Learned: the selected scores over their sum in
// rank order, times route_scale (route_from_indices, deepseek_v4_reference.cpp:80-121). Softmax:
// float64 softmax over every logit, the top-k probabilities, optional renormalisation
// (qwen38_moe_route, qwen3_8_flash_next_reference.cpp:1186-1240).
__device__ TokRoute route_weights(const MoeShape& s, uint32_t sel, uint32_t val, uint32_t misc) {
    const uint32_t lane = threadIdx.x & 63u, K = s.top_k, E = s.experts;
    uint32_t id = 0;
    float vk = 0.0f;
    if (lane < K) {
        id = lds_u32(sel + 8u * lane);
        vk = lds_f32(sel + 8u * lane + 4u);
    }
    bool bad = false;
    for (uint32_t i = 0; i < kTokWaves; ++i) bad |= lds_u32(misc + 4u * (kMiscKeyFlags + i)) != 0u;
    float wk = 0.0f;
    if (s.routing != kRouteSoftmax) {
        double sum = 0.0;  // the selected scores in rank order
        for (uint32_t k = 0; k < K; ++k) sum += (double)readlane_f32(vk, k);
        bad |= !(sum > 0.0) || isinf(sum);
        wk = (float)((double)vk / sum * (double)s.route_scale);
    } else {
        const double mx = (double)readlane_f32(vk, 0);
        double all = 0.0;
        for (uint32_t e = lane; e < E; e += 64u) all += exp((double)lds_f32(val + 4u * e) - mx);
        all = wave_sum_f64(all);
        const double pk = exp((double)vk - mx) * (all > 0.0 ? 1.0 / all : 0.0);
        double selsum = 0.0;
        for (uint32_t k = 0; k < K; ++k) selsum += readlane_f64(pk, k);
        wk = (float)pk;
        if (s.renormalize && selsum > 0.0) wk = (float)((double)wk * (1.0 / selsum));
    }
    return TokRoute{lane < K ? id : 0u, lane < K ? wk : 0.0f, bad};
}

// Table and given routing of the token by wave 0. An id out of range or repeated, any non-finite
// logit (table) and weights that cannot be normalised refuse the token.
__device__ TokRoute route_listed(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w) {
    const uint32_t lane = threadIdx.x & 63u, K = s.top_k, E = s.experts;
    bool bad = false;
    uint32_t id = 0;
    if (lane < K) {
        id = s.routing == kRouteTable ? *gp(in.table_ids + lane) : (in.given_ids ? *gp(in.given_ids + lane) : 0u);
        if (id >= E) {
            bad = true;
            id = 0;
        }
    }
    for (uint32_t k = 0; k < K; ++k)
        bad |= lane < K && k < lane && (uint32_t)__builtin_amdgcn_readlane((int)id, k) == id;
    float wk = 1.0f;
    if (s.routing == kRouteTable) {
        const uint32_t* keys = ws_ptr<const uint32_t>(w, w.off_keys);
        for (uint32_t e = lane; e < E; e += 64u) bad |= *gp(keys + e) <= 1u;
        const float sk = lane < K ? *gp(ws_ptr<const float>(w, w.off_scores) + id) : 0.0f;
        double sum = 0.0;
        for (uint32_t k = 0; k < K; ++k) sum += (double)readlane_f32(sk, k);
        bad |= !(sum > 0.0) || isinf(sum);
        wk = (float)((double)sk / sum * (double)s.route_scale);
    } else if (lane < K && in.given_weights) {
        wk = *gp(in.given_weights + lane);
    }
    return TokRoute{id, lane < K ? wk : 0.0f, __any(bad) != 0};
}

// Wave 0, after routing: the active list (routed experts in ascending id, then the shared
// expert), the combine entries, and their publication by block 0. Returns the position in the
// active list of the expert of rank `lane` (lanes < K).
__device__ uint32_t tok_active(const MoeShape& s, const MoeWorkspace& w, const TokRoute& rt, uint32_t act,
                               uint32_t comb, bool publish) {
    const uint32_t lane = threadIdx.x & 63u, K = s.top_k, E = s.experts;
    const uint32_t id = rt.id;
    const float wt = rt.wt;
    const bool bad = rt.bad;
    uint32_t a = 0;
    for (uint32_t k = 0; k < K; ++k) a += (uint32_t)__builtin_amdgcn_readlane((int)id, k) < id ? 1u : 0u;
    VL_LDS ActiveExpert* A = lptr<ActiveExpert>(act);
    VL_LDS CombineEntry* C = lptr<CombineEntry>(comb);
    const bool deepseek = s.semantics == kSemDeepseek;
    if (lane < K && !bad) {
        VL_LDS ActiveExpert& e = A[a];
        e.expert = id;
        e.ntok = 1;
        e.apply_w = deepseek ? 1u : 0u;
        e.limit = s.routed_limit;
        e.tok[0] = 0;
        e.route_w[0] = wt;
        VL_LDS CombineEntry& ce = C[deepseek ? a : lane];
        ce.src = a << 3;
        ce.w = s.semantics == kSemQwen ? wt : 1.0f;
    }
    if (lane == 0 && s.has_shared) {
        VL_LDS ActiveExpert& e = A[K];
        e.expert = E;
        e.ntok = 1;
        e.apply_w = 0;
        e.limit = s.shared_limit;
        e.tok[0] = 0;
        e.route_w[0] = 1.0f;
        C[K].src = K << 3;
        C[K].w = 1.0f;
    }
    if (!publish) return a;
    const uint32_t nA = K + (s.has_shared ? 1u : 0u);
    if (lane < K) {
        *gp(ws_ptr<uint32_t>(w, w.off_route_idx) + lane) = id;
        *gp(ws_ptr<float>(w, w.off_route_w) + lane) = wt;
    }
    lds_settle();
    const uint32_t words = nA * (uint32_t)(sizeof(ActiveExpert) / 4u);
    for (uint32_t i = lane; i < words && !bad; i += 64u)
        *gp(ws_ptr<uint32_t>(w, w.off_active) + i) = lds_u32(act + 4u * i);
    for (uint32_t i = lane; i < 2u * (K + 1u) && !bad; i += 64u)
        *gp(ws_ptr<uint32_t>(w, w.off_combine) + i) = lds_u32(comb + 4u * i);
    if (lane == 0) {
        MoeHeader* hdr = ws_ptr<MoeHeader>(w, w.off_header);
        *gp(&hdr->n_active) = bad ? 0u : nA;
        if (bad) or_bits(&hdr->status, kStatusBadRoute);
    }
    return a;
}

// ------------------------------------------------------------------------------------------
// Gate/up.
// ------------------------------------------------------------------------------------------

// h rows t*32 + n (n = lane < 32) of active expert a from the per-lane sums of gate (g) and up (u)
// (lane n + 32 holds the high limbs' share): SwiGLU, stores, the 256-row block maximum of |h|.
__device__ __attribute__((noinline)) void gu_finish(float g, float u, uint32_t a, uint32_t t, uint32_t inter,
                                                    uint32_t hblocks, uint32_t semantics, float limit,
                                                    uint32_t apply_w, float route_w, float* hout,
                                                    uint32_t* hmax, uint32_t* status) {
    const uint32_t lane = threadIdx.x & 63u, n = lane & 31u, row = t * 32u + n;
    const float gs = g + __shfl_xor(g, 32), us = u + __shfl_xor(u, 32);
    float hmag = 0.0f;
    bool bad = false;
    if (lane < 32u && row < inter) {
        const float h = swiglu(semantics, gs, us, limit, apply_w != 0, route_w);
        bad = !isfinite(gs) || !isfinite(us) || !isfinite(h);
        *gp(hout + (uint64_t)a * inter + row) = h;
        hmag = isfinite(h) ? fabsf(h) : 0.0f;
    }
    for (int o = 16; o > 0; o >>= 1) hmag = fmaxf(hmag, __shfl_xor(hmag, o));
    if (lane == 0)
        __hip_atomic_fetch_max(gp(hmax + ((uint64_t)a * hblocks + t / 8u) * 8u), __float_as_uint(hmag),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__any(bad) && lane == 0) or_bits(status, kStatusNonFiniteOutput);
}

// The last chunk of a stream-K segment of a gate/up block is done: the segment's chunks k0 .. k0+n-1
// (the first ngate of the gate matrix) are added per lane into the block's record; the job's last
// contributing block adds every record in block order and finishes the job.
__device__ __attribute__((noinline)) void gu_segment(uint32_t part, uint32_t k0, uint32_t n, uint32_t ngate,
                                                     uint32_t region, uint32_t b, uint32_t seg, uint32_t job,
                                                     uint32_t job0, uint32_t total, uint32_t blocks, uint32_t UJ,
                                                     uint32_t grid, uint32_t tiles, uint32_t act, uint32_t inter,
                                                     uint32_t hblocks, uint32_t semantics, float* h, uint32_t* hmax,
                                                     uint32_t* status, uint32_t* counters, float* rec) {
    const uint32_t lane = threadIdx.x & 63u;
    const float sg = sum_parts(part, k0, ngate < n ? ngate : n);
    const float su = ngate < n ? sum_parts(part, k0 + ngate, n - ngate) : 0.0f;
    auto record = [&](uint32_t blk, uint32_t sg) {
        return rec + (((uint64_t)region * grid + blk) * kTokMaxSeg + sg) * 128u;
    };
    float* r = record(b, seg);
    store_shared(r + lane, sg);
    store_shared(r + 64u + lane, su);
    const TokRegion X{total, blocks, job0};
    const uint32_t lo = (job - job0) * UJ, fb = tok_block_of(X, lo), lb = tok_block_of(X, lo + UJ - 1u);
    if (!arrive(counters + job, lb - fb + 1u)) return;
    // The contributors' records in block order, the loads of eight records in flight at once.
    constexpr uint32_t B = 8;
    float g = 0.0f, u = 0.0f;
    for (uint32_t b0 = fb; b0 <= lb; b0 += B) {
        float vg[B], vu[B];
#pragma unroll
        for (uint32_t i = 0; i < B; ++i) {
            const uint32_t bb = b0 + i <= lb ? b0 + i : lb;  // clamped loads are not added
            const float* rb = record(bb, (job - job0) - tok_piece_lo(X, bb) / UJ);
            vg[i] = load_shared(rb + lane);
            vu[i] = load_shared(rb + 64u + lane);
        }
#pragma unroll
        for (uint32_t i = 0; i < B; ++i)
            if (b0 + i <= lb) {
                g += vg[i];
                u += vu[i];
            }
    }
    const uint32_t a = job / tiles, t = job - a * tiles;
    const VL_LDS ActiveExpert* ae = lptr<ActiveExpert>(act) + a;
    gu_finish(g, u, a, t, inter, hblocks, semantics, ae->limit, ae->apply_w, ae->route_w[0], h, hmax, status);
}

// What the rare paths (segment hand-offs, finishing jobs) need, kept in LDS: the wave loop's
// registers then hold only what every chunk uses.
struct TokRare {
    TokPlan p;
    TokPiece ps, pr;
    uint32_t b, act, comb, inter, hblocks, semantics, K, has_shared, width;
    float* h;
    uint32_t* hmax;
    uint32_t* status;
    uint32_t* counters;
    float* rec;
    float* out;
};

template <uint32_t FMT>
struct GuCtx {
    static constexpr uint32_t CU = tok_chunk_units(FMT);
    uint32_t part, desc, misc, ng, nchunks, rare;
    vl_tiled_layout L;
    uint32_t xstage, xscale, wptr;

    __device__ TokWork chunk(uint32_t k) const {
        TokWork c{0, 0, 0, 0, 0, 2, 0};
        if (k < nchunks) {
            const u32x2 d = lds_load<u32x2>(desc + 8u * k);
            const u32x2 du = {uni(d.x), uni(d.y)};
            c = decode_work(du);
        }
        return c;
    }
    __device__ TileRef tref(const TokWork& c) const {
        return tile_ref<FMT>(L, uni_ptr(reinterpret_cast<const uint8_t*>(lds_load<uint64_t>(wptr + 16u * c.a + 8u * c.m))), c.t);
    }
    __device__ ASrc<true, 128u> asrc(const TokWork&) const {
        const uint32_t m = threadIdx.x & 31u, kh = (threadIdx.x >> 5) & 1u;
        ASrc<true, 128u> as;
        as.ptr = nullptr;
        as.off = xstage + a_limb(m) * 32u + 16u * kh;
        as.stride = 128u;
        return as;
    }
    __device__ float scale(const TokWork&, uint32_t c) const {
        return lds_f32(xscale + 4u * (FMT == VL_TYPE_Q8_0 ? c / 2u : c));
    }
    __device__ bool done(const TokWork& c) const {
        if (c.region == 2) return false;
        lds_settle();
        const uint32_t slot = c.region * kTokMaxSeg + c.seg;
        uint32_t old = 0;
        if ((threadIdx.x & 63u) == 0) old = lds_add(misc + 4u * (kMiscSeg + slot), 1u);
        return uni(old) + 1u == lds_u32(misc + 4u * (kMiscSegN + slot));
    }
    // The block's record of a completed segment and the job's hand-off.
    __device__ void segment(const TokWork& c) const {
        const TokRare r = lds_get<TokRare>(rare);
        const bool sh = c.region == 0;
        TokPiece P;  // field by field: a choice between two objects would be made through memory
        P.lo = sh ? r.ps.lo : r.pr.lo;
        P.hi = sh ? r.ps.hi : r.pr.hi;
        P.n = sh ? r.ps.n : r.pr.n;
        P.c0 = sh ? r.ps.c0 : r.pr.c0;
        TokRegion X;
        X.total = sh ? r.p.S.total : r.p.R.total;
        X.blocks = sh ? r.p.S.blocks : r.p.R.blocks;
        X.job0 = sh ? r.p.S.job0 : r.p.R.job0;
        uint32_t first = 0, n = 0;
        seg_chunks<CU>(r.p, P, c.seg, first, n);
        const uint32_t job = c.a * r.p.tiles + c.t;
        const uint32_t k0 = (sh ? 0u : r.ps.n) + first;
        // The segment starts at unit vlo of the job; chunk boundaries fall on the gate/up boundary C.
        const uint32_t vlo = c.seg == 0 ? P.lo % r.p.UJ : 0u;
        const uint32_t C = r.p.C;
        const uint32_t ngate = vlo < C ? (C / CU - vlo / CU < n ? C / CU - vlo / CU : n) : 0u;
        gu_segment(part, k0, n, ngate, c.region, r.b, c.seg, job, X.job0, X.total, X.blocks, r.p.UJ, r.p.grid,
                   r.p.tiles, r.act, r.inter, r.hblocks, r.semantics, r.h, r.hmax, r.status, r.counters, r.rec);
    }
};

// The block's chunk table and the chunk count of each stream-K segment of its pieces, into LDS.
template <uint32_t CU>
__device__ __forceinline__ void fill_work(const TokPlan p, uint32_t b, const TokPiece ps, const TokPiece pr,
                                          uint32_t nchunks, uint32_t desc, uint32_t misc, bool gate_up,
                                          uint32_t t, uint32_t nt) {
    for (uint32_t k = t; k < nchunks; k += nt)
        *lptr<u32x2>(desc + 8u * k) = encode_work(tok_chunk<CU>(p, b, ps, pr, k), p.tiles, p.C, gate_up);
    if (t < 2u * kTokMaxSeg) {
        const uint32_t r = t / kTokMaxSeg, sg = t % kTokMaxSeg;
        TokPiece P;  // field by field: a per-lane choice of struct would be made through memory
        P.lo = r == 0 ? ps.lo : pr.lo;
        P.hi = r == 0 ? ps.hi : pr.hi;
        P.n = r == 0 ? ps.n : pr.n;
        P.c0 = r == 0 ? ps.c0 : pr.c0;
        uint32_t first = 0, n = 0;
        if (P.hi > P.lo && sg <= (P.hi - 1u) / p.UJ - P.lo / p.UJ) seg_chunks<CU>(p, P, sg, first, n);
        lds_st_u32(misc + 4u * (kMiscSegN + t), n);
    }
}

static_assert((kTokWaves - 1u) * 64u >= 384u && 3u * (kTokWaves - 1u) * 64u >= 2048u,
              "the tables are filled by the waves other than the routing wave");

template <uint32_t FMT>
__global__ void __launch_bounds__(kTokWaves * 64u) k_tok_gateup(const MoeShape s, const MoeInputs in,
                                                                const MoeWorkspace w, const TokPlan p) {
    constexpr uint32_t TB = table_bytes<FMT>(), CU = tok_chunk_units(FMT);
    const TokGuLds lay = tok_lds_gu(TB, s.width, p.max_chunks, s.experts);
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, nw = blockDim.x >> 6;
    const uint32_t b = blockIdx.x, K = s.top_k, E = s.experts;
    const bool ranked = s.routing == kRouteLearned || s.routing == kRouteSoftmax;
    const bool ptab = tok_has_ptab(E);
    const uint32_t G = tok_group(E, K);

    // 1. Requests, every one issued unconditionally (clamped indices), so that they are waited for
    //    as one group: every expert's selection key and score (thread e: expert e) and gate/up
    //    pointers, the shared expert's pointers, the decode tables, the token's limbs, exponents and
    //    flags. The first weight chunk is requested only after these have arrived and been stored:
    //    loads complete in order, and a chunk from HBM ahead of them would delay every wait of the
    //    prologue.
    //    Pools of up to kTokWaveRoute experts are routed by wave 0 alone, which requests the keys,
    //    scores and gate/up pointers of four experts per lane; larger pools by the whole block.
    const bool wave_route = E <= kTokWaveRoute;
    uint32_t key = 0, rk[4] = {0, 0, 0, 0};
    float score = 0.0f, rs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    uint64_t pg = 0, pu = 0, rg[4] = {0, 0, 0, 0}, ru[4] = {0, 0, 0, 0};
    const uint32_t elast = s.has_shared ? E : E - 1u;
    if (!wave_route) {
        const uint32_t ek = tid < E ? tid : E - 1u;
        key = *gp(ws_ptr<const uint32_t>(w, w.off_keys) + ek);
        score = *gp(ws_ptr<const float>(w, w.off_scores) + ek);
        const MoeExpert* ex = in.experts + (tid < elast ? tid : elast);
        pg = reinterpret_cast<uint64_t>(ex->gate);
        pu = reinterpret_cast<uint64_t>(ex->up);
    } else if (wave == 0) {
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const uint32_t e = lane + 64u * j < E ? lane + 64u * j : E - 1u;
            rk[j] = *gp(ws_ptr<const uint32_t>(w, w.off_keys) + e);
            rs[j] = *gp(ws_ptr<const float>(w, w.off_scores) + e);
            rg[j] = reinterpret_cast<uint64_t>(in.experts[e].gate);
            ru[j] = reinterpret_cast<uint64_t>(in.experts[e].up);
        }
    }
    const MoeExpert* exs = in.experts + elast;
    const uint64_t shg = reinterpret_cast<uint64_t>(exs->gate), shu = reinterpret_cast<uint64_t>(exs->up);
    // The LDS fill below is shared by the waves that do not route: all of them for a larger pool,
    // waves 1.. when wave 0 routes (its thread index pt and count npt; wave 0 then fills nothing
    // and routes as soon as its keys arrive).
    const bool filler = !wave_route || wave != 0;
    const uint32_t pt = wave_route ? tid - 64u : tid, npt = wave_route ? blockDim.x - 64u : blockDim.x;
    TokTables<FMT> tt;
    const uint32_t xn = (s.width / 32u) * 128u / 16u;  // 16-byte words of the token's limbs
    const uint4* xsrc = ws_ptr<const uint4>(w, w.off_xlimbs);
    constexpr uint32_t XB = 2;
    uint4 xv[XB];
    int ev = 0;
    uint32_t fv = 0;
    if (filler) {
        tt.load(pt, npt);
#pragma unroll
        for (uint32_t j = 0; j < XB; ++j) {
            const uint32_t i = pt + j * npt;
            xv[j] = ld_u4(xsrc + (i < xn ? i : xn - 1u));
        }
        const uint32_t xb = pt < w.xblocks ? pt : w.xblocks - 1u;
        ev = *gp(ws_ptr<const int>(w, w.off_xexp) + (uint64_t)w.estride * xb);
        fv = *gp(ws_ptr<const uint32_t>(w, w.off_xflags) + (uint64_t)w.estride * xb);
    }
    issue_fence();
    // The block's pieces and the wave loop's view, formed while the requests are in flight.
    const TokPiece ps = tok_piece(p.S, b, CU), pr = tok_piece(p.R, b, CU);
    GuCtx<FMT> ctx;
    ctx.part = lay.part;
    ctx.desc = lay.desc;
    ctx.misc = lay.misc;
    ctx.rare = lay.rare;
    vl_make_layout(FMT, s.inter, s.width, &ctx.L);
    ctx.ng = ctx.L.groups;
    ctx.nchunks = ps.n + pr.n + p.q * p.UJ / CU;
    ctx.xstage = lay.xstage;
    ctx.xscale = lay.xscale;
    ctx.wptr = lay.wptr;
    const uint32_t nS = ps.n, nstatic = nS < nw ? nS : nw;

    // 2. LDS stores: tables, limbs, 2^-e, pointers, counters and flags, the chunk table, the
    //    rare-path record, the routing keys and group maxima.
    uint4* xdst = reinterpret_cast<uint4*>(lds_base() + lay.xstage);
    if (filler) {
        tt.store(lds_base(), pt, npt);
#pragma unroll
        for (uint32_t j = 0; j < XB; ++j)
            if (pt + j * npt < xn) xdst[pt + j * npt] = xv[j];
        for (uint32_t i = pt + XB * npt; i < xn; i += npt) xdst[i] = ld_u4(xsrc + i);
        if (pt < w.xblocks) lds_st_f32(lay.xscale + 4u * pt, __builtin_amdgcn_ldexpf(1.0f, -ev));
    }
    if (!wave_route && ptab && tid <= E) {
        *lptr<uint64_t>(lay.ptab + 16u * tid) = pg;
        *lptr<uint64_t>(lay.ptab + 16u * tid + 8u) = pu;
    }
    // Counters start at zero (the chunk counter past the statically taken chunks); the flag words
    // are written by their own waves and the refusal flag by wave 0 alone. The counters and
    // fill_work's segment counts are stored by one wave, in that order.
    if (filler && pt < kMiscBad) lds_st_u32(lay.misc + 4u * pt, pt == kMiscGrab ? nstatic : 0u);
    if (filler && pt == kMiscWaveFlags) lds_st_u32(lay.misc + 4u * kMiscCand, 0u);
    const bool xflag = __any(filler && pt < w.xblocks && fv != 0u);
    if (lane == 0) lds_st_u32(lay.misc + 4u * (kMiscWaveFlags + wave), xflag ? 1u : 0u);
    const float rv = ranked && !wave_route ? route_stage(s, key, score, lay.val, lay.gmax, lay.misc, G) : 0.0f;
    if (filler) fill_work<CU>(p, b, ps, pr, ctx.nchunks, lay.desc, lay.misc, true, pt, npt);
    if (filler && pt == 0) {
        TokRare r;
        r.p = p;
        r.ps = ps;
        r.pr = pr;
        r.b = b;
        r.act = lay.act;
        r.comb = lay.comb;
        r.inter = s.inter;
        r.hblocks = w.hblocks;
        r.semantics = s.semantics;
        r.K = K;
        r.has_shared = s.has_shared;
        r.width = s.width;
        r.h = ws_ptr<float>(w, w.off_h);
        r.hmax = counters_of(w).hmax;
        r.status = &ws_ptr<MoeHeader>(w, w.off_header)->status;
        r.counters = counters_of(w).gu;
        r.rec = ws_ptr<float>(w, w.off_trec);
        r.out = in.out;
        lds_put(lay.rare, r);
    }
    // Routes: wave 0 alone (pools of up to kTokWaveRoute experts: every route, the active list
    // and the active experts' pointers, before the first barrier), or the listed routes of a larger
    // pool (wave 0). Then this wave's first chunk of the shared expert.
    TokRoute rt{0, 0.0f, false};
    if (wave == 0 && (wave_route || !ranked)) {
        if (ranked) {
            route_wave0(s, rk, rs, lay.val, lay.gmax, lay.cand, lay.sel, lay.misc);
            rt = route_weights(s, lay.sel, lay.val, lay.misc);
        } else {
            rt = route_listed(s, in, w);
        }
    }
    if (wave == 0 && wave_route) {
        const bool bad = rt.bad;
        const uint32_t a = tok_active(s, w, rt, lay.act, lay.comb, b == 0);
        // Lane k < K: the pointers of its expert, from the lane that requested them.
        const uint32_t src = rt.id & 63u, jj = rt.id >> 6;
        uint64_t g = 0, u = 0;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const uint64_t gj = ((uint64_t)(uint32_t)__shfl((int)(uint32_t)(rg[j] >> 32), (int)src) << 32) |
                                (uint32_t)__shfl((int)(uint32_t)rg[j], (int)src);
            const uint64_t uj = ((uint64_t)(uint32_t)__shfl((int)(uint32_t)(ru[j] >> 32), (int)src) << 32) |
                                (uint32_t)__shfl((int)(uint32_t)ru[j], (int)src);
            g = jj == j ? gj : g;
            u = jj == j ? uj : u;
        }
        if (lane < K && !bad) {
            *lptr<uint64_t>(lay.wptr + 16u * a) = g;
            *lptr<uint64_t>(lay.wptr + 16u * a + 8u) = u;
        }
        if (lane < 2u && s.has_shared) *lptr<uint64_t>(lay.wptr + 16u * K + 8u * lane) = lane ? shu : shg;
        if (lane == 0) lds_st_u32(lay.misc + 4u * kMiscBad, bad ? 1u : 0u);
    }
    Chunk bufA[CU];
    TokWork ca{0, 0, 0, 0, 0, 2, 0};
    const uint32_t ka = wave;
    if (wave < nstatic) {
        ca = decode_work(encode_work(tok_chunk<CU>(p, b, ps, pr, ka), p.tiles, p.C, true));
        const uint8_t* mp = reinterpret_cast<const uint8_t*>(ca.m ? shu : shg);
        const TileRef tr = tile_ref<FMT>(ctx.L, uni_ptr(mp), ca.t);
#pragma unroll
        for (uint32_t i = 0; i < CU; ++i)
            tok_load<FMT>(i < ca.count ? tr : idle_tile(), i < ca.count ? ca.col + i : 0u, ctx.ng, bufA[i]);
    }
    __syncthreads();

    // 3. Routing of a larger pool: candidates, their ranks, then wave 0 forms the weights, the
    //    active list and the active experts' pointers.
    if (ranked && !wave_route) {
        route_candidates(s, key, rv, lay.gmax, lay.cand, lay.misc, G);
        __syncthreads();
        const uint32_t n = uni(lds_u32(lay.misc + 4u * kMiscCand));
        if (n <= 64u) {
            if (wave == 0) route_rank_wave(n, K, lay.cand, lay.sel);
        } else {
            route_rank_block(n, K, lay.cand, lay.sel);
            __syncthreads();
        }
    }
    if (wave == 0 && !wave_route) {
        if (ranked) {
            lds_settle();
            rt = route_weights(s, lay.sel, lay.val, lay.misc);
        }
        const bool bad = rt.bad;
        const uint32_t a = tok_active(s, w, rt, lay.act, lay.comb, b == 0);
        if (lane < K && !bad) {
            uint64_t g = 0, u = 0;
            if (ptab) {
                g = *lptr<uint64_t>(lay.ptab + 16u * rt.id);
                u = *lptr<uint64_t>(lay.ptab + 16u * rt.id + 8u);
            } else {
                g = reinterpret_cast<uint64_t>(in.experts[rt.id].gate);
                u = reinterpret_cast<uint64_t>(in.experts[rt.id].up);
            }
            *lptr<uint64_t>(lay.wptr + 16u * a) = g;
            *lptr<uint64_t>(lay.wptr + 16u * a + 8u) = u;
        }
        if (lane < 2u && s.has_shared) *lptr<uint64_t>(lay.wptr + 16u * K + 8u * lane) = lane ? shu : shg;
        if (lane == 0) lds_st_u32(lay.misc + 4u * kMiscBad, bad ? 1u : 0u);
    }
    if (!wave_route) __syncthreads();
    if (b == 0 && tid == 0) {
        uint32_t xb = 0;
        for (uint32_t i = 0; i < nw; ++i) xb |= lds_u32(lay.misc + 4u * (kMiscWaveFlags + i));
        if (xb) or_bits(&ws_ptr<MoeHeader>(w, w.off_header)->status, kStatusNonFiniteInput);
    }
    if (lds_u32(lay.misc + 4u * kMiscBad)) return;  // refused: the down kernel writes zeros
    // 4. Stream: this wave's chunk of the shared expert, then chunks from the counter.
    tok_stream<FMT, CU>(ctx, ka, ca, bufA);
    __syncthreads();
    // 5. Data-parallel jobs: the sums of each job's gate and of its up chunks in chunk order, a wave
    //    per matrix (into the token's limb area, no longer read), then a wave per job finishes it.
    const TokRare r = lds_get<TokRare>(lay.rare);
    const uint32_t nd0 = r.ps.n + r.pr.n, cpm = r.p.C / CU;
    for (uint32_t m = wave; m < 2u * r.p.q; m += nw)
        lds_st_f32(lay.xstage + m * 256u + lane * 4u, sum_parts(lay.part, nd0 + m * cpm, cpm));
    __syncthreads();
    for (uint32_t jj = wave; jj < r.p.q; jj += nw) {
        const float g = lds_f32(lay.xstage + 2u * jj * 256u + lane * 4u);
        const float u = lds_f32(lay.xstage + (2u * jj + 1u) * 256u + lane * 4u);
        const uint32_t job = r.b * r.p.q + jj, a = job / r.p.tiles, t = job - a * r.p.tiles;
        const VL_LDS ActiveExpert* ae = lptr<ActiveExpert>(r.act) + a;
        gu_finish(g, u, a, t, r.inter, r.hblocks, r.semantics, ae->limit, ae->apply_w, ae->route_w[0], r.h, r.hmax,
                  r.status);
    }
}

// ------------------------------------------------------------------------------------------
// Down.
// ------------------------------------------------------------------------------------------

// Output rows t*32 + n (n = lane < 32) of a stream-K tile: each active expert's rows (lane n + 32
// holding the high limbs' share) summed over the records of the contributing blocks fb..lb in block
// order (record of block bb: rec + ((bb * kTokMaxSeg + seg(bb)) * A + a) * 64), then added in the
// combine order.
// Combine entry k's sum y of an output row into acc: Qwen weighs the routed experts' rows by their
// route weights, DeepSeek adds them as they are (the weights were applied to h).
__device__ __forceinline__ float dn_combine(float acc, float y, uint32_t k, uint32_t K, uint32_t semantics,
                                            const VL_LDS CombineEntry* C) {
    return (semantics == kSemQwen && k < K) ? __fadd_rn(acc, __fmul_rn(y, C[k].w)) : __fadd_rn(acc, y);
}

// Output rows t*32 + lane (lanes < 32) and the non-finite output flag.
__device__ __forceinline__ void dn_store(uint32_t t, float acc, uint32_t width, float* out, uint32_t* status) {
    const uint32_t lane = threadIdx.x & 63u, row = t * 32u + (lane & 31u);
    const bool live = lane < 32u && row < width;
    if (live) *gp(out + row) = acc;
    if (__any(live && !isfinite(acc)) && lane == 0) or_bits(status, kStatusNonFiniteOutput);
}

__device__ __attribute__((noinline)) void dn_finish(uint32_t t, const float* rec, uint32_t fb, uint32_t lb,
                                                    uint32_t job0,
                                                    uint32_t total, uint32_t blocks, uint32_t UJ, uint32_t A,
                                                    uint32_t comb, uint32_t K, uint32_t has_shared,
                                                    uint32_t semantics, uint32_t width, float* out, uint32_t* status) {
    const uint32_t lane = threadIdx.x & 63u;
    const VL_LDS CombineEntry* C = lptr<CombineEntry>(comb);
    const uint32_t nent = K + (has_shared ? 1u : 0u);
    float acc = 0.0f;
    auto combine = [&](float v, uint32_t k) { acc = dn_combine(acc, v + __shfl_xor(v, 32), k, K, semantics, C); };
    {
        // Pairs (entry k, contributor bb) in order, k-major: each entry's records added in block
        // order, then combined; the loads of B pairs in flight at once.
        constexpr uint32_t B = 16;
        const TokRegion X{total, blocks, job0};
        const uint32_t nb = lb - fb + 1u, np = nent * nb;
        uint32_t lk = 0, lj = 0, ck = 0, cj = 0;  // next pair to load, next pair to add
        float v = 0.0f;
        for (uint32_t p0 = 0; p0 < np; p0 += B) {
            float tv[B];
#pragma unroll
            for (uint32_t i = 0; i < B; ++i) {
                tv[i] = 0.0f;
                if (p0 + i < np) {
                    const uint32_t a = C[lk].src >> 3, bb = fb + lj;
                    const uint32_t seg = (t - job0) - tok_piece_lo(X, bb) / UJ;
                    tv[i] = load_shared(rec + (((uint64_t)bb * kTokMaxSeg + seg) * A + a) * 64u + lane);
                    if (++lj == nb) {
                        lj = 0;
                        ++lk;
                    }
                }
            }
#pragma unroll
            for (uint32_t i = 0; i < B; ++i)
                if (p0 + i < np) {
                    v += tv[i];
                    if (++cj == nb) {
                        combine(v, ck);
                        v = 0.0f;
                        cj = 0;
                        ++ck;
                    }
                }
        }
    }
    dn_store(t, acc, width, out, status);
}

// The last chunk of a stream-K segment of a down block is done: the segment's chunks k0 .. k0+n-1 of
// cu units, whose first unit is unit v0 of the tile, are added per expert and lane into the block's
// record;
// the tile's last contributing block combines every record.
__device__ __attribute__((noinline)) void dn_segment(uint32_t part, uint32_t k0, uint32_t n, uint32_t v0, uint32_t cu,
                                                     uint32_t b,
                                                     uint32_t seg, uint32_t t, uint32_t job0, uint32_t total,
                                                     uint32_t blocks, uint32_t UJ, uint32_t C, uint32_t A,
                                                     uint32_t comb, uint32_t K, uint32_t has_shared,
                                                     uint32_t semantics, uint32_t width, float* out,
                                                     uint32_t* status, uint32_t* counters, float* rec) {
    const uint32_t lane = threadIdx.x & 63u;
    float* r = rec + ((uint64_t)b * kTokMaxSeg + seg) * A * 64u;
    uint32_t cur = 0xffffffffu;
    float sum = 0.0f;
    for (uint32_t a = 0; a < A; ++a) store_shared(r + a * 64u + lane, 0.0f);
    for (uint32_t i = 0; i < n; ++i) {
        // Chunk i starts at unit max(v0, (v0 / cu + i) * cu) of the tile; C is a multiple of cu.
        const uint32_t a = ((v0 / cu + i) * cu > v0 ? (v0 / cu + i) * cu : v0) / C;
        if (a != cur) {
            if (cur != 0xffffffffu) store_shared(r + cur * 64u + lane, sum);
            cur = a;
            sum = 0.0f;
        }
        sum += lds_f32(part + (k0 + i) * 256u + lane * 4u);
    }
    if (cur != 0xffffffffu) store_shared(r + cur * 64u + lane, sum);
    const TokRegion X{total, blocks, job0};
    const uint32_t lo = (t - job0) * UJ, fb = tok_block_of(X, lo), lb = tok_block_of(X, lo + UJ - 1u);
    if (!arrive(counters + t, lb - fb + 1u)) return;
    dn_finish(t, rec, fb, lb, job0, total, blocks, UJ, A, comb, K, has_shared, semantics, width, out, status);
}

template <uint32_t FMT>
struct DnCtx {
    static constexpr uint32_t CU = tok_chunk_units(FMT);
    uint32_t part, desc, misc, ng, nchunks, rare;
    vl_tiled_layout L;
    uint32_t hstage, hscale, dptr, hb, ebytes;

    __device__ TokWork chunk(uint32_t k) const {
        TokWork c{0, 0, 0, 0, 0, 2, 0};
        if (k < nchunks) {
            const u32x2 d = lds_load<u32x2>(desc + 8u * k);
            const u32x2 du = {uni(d.x), uni(d.y)};
            c = decode_work(du);
        }
        return c;
    }
    __device__ TileRef tref(const TokWork& c) const {
        return tile_ref<FMT>(L, uni_ptr(reinterpret_cast<const uint8_t*>(lds_load<uint64_t>(dptr + 8u * c.a))), c.t);
    }
    __device__ ASrc<true, 128u> asrc(const TokWork& c) const {
        const uint32_t m = threadIdx.x & 31u, kh = (threadIdx.x >> 5) & 1u;
        ASrc<true, 128u> as;
        as.ptr = nullptr;
        as.off = hstage + c.a * ebytes + a_limb(m) * 32u + 16u * kh;
        as.stride = 128u;
        return as;
    }
    __device__ float scale(const TokWork& c, uint32_t cc) const {
        return lds_f32(hscale + 4u * (c.a * hb + (FMT == VL_TYPE_Q8_0 ? cc / 2u : cc)));
    }
    __device__ bool done(const TokWork& c) const {
        if (c.region == 2) return false;
        lds_settle();
        const uint32_t slot = kTokMaxSeg + c.seg;
        uint32_t old = 0;
        if ((threadIdx.x & 63u) == 0) old = lds_add(misc + 4u * (kMiscSeg + slot), 1u);
        return uni(old) + 1u == lds_u32(misc + 4u * (kMiscSegN + slot));
    }
    // The block's record of a completed segment and the tile's hand-off.
    __device__ void segment(const TokWork& c) const {
        const TokRare r = lds_get<TokRare>(rare);
        uint32_t first = 0, n = 0;
        seg_chunks<CU>(r.p, r.pr, c.seg, first, n);
        const uint32_t vlo = c.seg == 0 ? r.pr.lo % r.p.UJ : 0u;
        dn_segment(part, r.ps.n + first, n, vlo, CU, r.b, c.seg, c.t, r.p.R.job0, r.p.R.total, r.p.R.blocks, r.p.UJ,
                   r.p.C, r.p.A, r.comb, r.K, r.has_shared, r.semantics, r.width, r.out, r.status, r.counters, r.rec);
    }
};

template <uint32_t FMT>
__global__ void __launch_bounds__(kTokWaves * 64u) k_tok_down(const MoeShape s, const MoeInputs in,
                                                              const MoeWorkspace w, const TokPlan p) {
    constexpr uint32_t TB = table_bytes<FMT>(), CU = tok_chunk_units(FMT);
    const uint32_t A = p.A, F = s.inter, K = s.top_k, E = s.experts, HB = w.hblocks;
    const TokDnLds lay = tok_lds_dn(TB, A, F, p.max_chunks);
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, nw = blockDim.x >> 6;
    const uint32_t b = blockIdx.x;
    const MoeHeader* hdr = ws_ptr<const MoeHeader>(w, w.off_header);
    // 1. Requests, issued unconditionally (clamped indices) and together: the active experts' ids
    //    (lane a of every wave: active expert a), the active count, the combine entries, every
    //    expert's down pointer, the decode tables, the active experts' h with the maxima of its
    //    256-row blocks. Then the down pointer of the expert of this wave's first chunk (as the
    //    chunk table will hold it), picked from the ids once they arrive.
    const ActiveExpert* act = ws_ptr<const ActiveExpert>(w, w.off_active);
    const uint32_t eid = *gp(&act[lane < A ? lane : A - 1u].expert);
    const uint32_t n_active_raw = *gp(&hdr->n_active);
    const uint32_t nc = 2u * (K + 1u);
    const uint32_t cw = *gp(ws_ptr<const uint32_t>(w, w.off_combine) + (tid < nc ? tid : nc - 1u));
    const uint32_t pn = E + 1u <= kTokPtrTab + 1u ? E + 1u : 0u;
    const uint32_t elast = s.has_shared ? E : E - 1u;
    const uint64_t pv = reinterpret_cast<uint64_t>(in.experts[tid < elast ? tid : elast].down);
    TokTables<FMT> tt;
    tt.load(tid, blockDim.x);
    const float* h = ws_ptr<const float>(w, w.off_h);
    const uint32_t* hmax = counters_of(w).hmax;
    const uint32_t quads = F / 4u, hq_total = A * quads;
    constexpr uint32_t HQ = 8;
    float4 hv[HQ];
    uint32_t hvm[HQ];
#pragma unroll
    for (uint32_t j = 0; j < HQ; ++j) {
        if (j * blockDim.x >= hq_total) break;  // uniform
        const uint32_t i = tid + j * blockDim.x < hq_total ? tid + j * blockDim.x : hq_total - 1u;
        const uint32_t a = i / quads, col = 4u * (i - a * quads);
        hv[j] = ld_f4(h + (uint64_t)a * F + col);
        hvm[j] = *gp(hmax + ((uint64_t)a * HB + col / 256u) * 8u);
    }
    const uint32_t hb = A * HB;
    const uint32_t hm = *gp(hmax + (uint64_t)(tid < hb ? tid : hb - 1u) * 8u);
    issue_fence();
    // The block's pieces and the wave loop's view, formed while the requests are in flight.
    const TokPiece ps = tok_piece(p.S, b, CU), pr = tok_piece(p.R, b, CU);
    DnCtx<FMT> ctx;
    ctx.part = lay.part;
    ctx.desc = lay.desc;
    ctx.misc = lay.misc;
    ctx.rare = lay.rare;
    vl_make_layout(FMT, s.width, s.inter, &ctx.L);
    ctx.ng = ctx.L.groups;
    ctx.nchunks = ps.n + pr.n + p.q * p.UJ / CU;
    ctx.hstage = lay.hstage;
    ctx.hscale = lay.hscale;
    ctx.dptr = lay.dptr;
    ctx.hb = HB;
    ctx.ebytes = (F / 32u) * 128u;
    // The first chunk's matrix (a stale id of a refused layer still names a real expert): requested
    // now, waited for only when the chunk is issued.
    const uint32_t ka = wave;
    const TokWork ca = ka < ctx.nchunks ? decode_work(encode_work(tok_chunk<CU>(p, b, ps, pr, ka), p.tiles, p.C, false))
                                        : TokWork{0, 0, 0, 0, 0, 2, 0};
    const uint32_t ea = (uint32_t)__builtin_amdgcn_readlane((int)eid, ca.a < A ? ca.a : 0u);
    const uint64_t pa_raw = reinterpret_cast<uint64_t>(in.experts[ea < elast ? ea : elast].down);
    issue_fence();

    // 2. LDS stores: pointers, ids, combine entries, counters, the chunk table, the rare-path
    //    record, the tables, and the active experts' h -> limbs with one exponent per 256 rows.
    if (tid <= elast && tid < pn) *lptr<uint64_t>(lay.ptab + 8u * tid) = pv;
    if (tid < A) lds_st_u32(lay.eid + 4u * tid, eid);
    if (tid < 2u * (K + 1u)) lds_st_u32(lay.comb + 4u * tid, cw);
    if (tid < kMiscSegN) lds_st_u32(lay.misc + 4u * tid, tid == kMiscGrab ? nw : 0u);
    fill_work<CU>(p, b, ps, pr, ctx.nchunks, lay.desc, lay.misc, false, tid, blockDim.x);
    if (tid == 0) {
        TokRare r;
        r.p = p;
        r.ps = ps;
        r.pr = pr;
        r.b = b;
        r.act = 0;
        r.comb = lay.comb;
        r.inter = s.inter;
        r.hblocks = HB;
        r.semantics = s.semantics;
        r.K = K;
        r.has_shared = s.has_shared;
        r.width = s.width;
        r.h = nullptr;
        r.hmax = nullptr;
        r.status = &ws_ptr<MoeHeader>(w, w.off_header)->status;
        r.counters = counters_of(w).tile;
        r.rec = ws_ptr<float>(w, w.off_trec) + gu_record_bytes(w.blocks) / 4u;
        r.out = in.out;
        lds_put(lay.rare, r);
    }
    tt.store(lds_base(), tid, blockDim.x);
    {
        auto convert = [&](uint32_t i, const float4& f4, uint32_t mx) {
            const uint32_t a = i / quads, col = 4u * (i - a * quads);
            const float v[4] = {f4.x, f4.y, f4.z, f4.w};
            uint32_t packed[4];
            limbs4(v, limb_exponent(__uint_as_float(mx)), packed);
            const uint32_t d = lay.hstage + a * ctx.ebytes + (col / 32u) * 128u + (col % 32u);
#pragma unroll
            for (int l = 0; l < 4; ++l) lds_st_u32(d + 32u * l, packed[l]);
        };
#pragma unroll
        for (uint32_t j = 0; j < HQ; ++j) {
            const uint32_t i = tid + j * blockDim.x;
            if (j * blockDim.x >= hq_total) break;
            if (i < hq_total) convert(i, hv[j], hvm[j]);
        }
        for (uint32_t i = tid + HQ * blockDim.x; i < hq_total; i += blockDim.x) {
            const uint32_t a = i / quads, col = 4u * (i - a * quads);
            convert(i, ld_f4(h + (uint64_t)a * F + col), *gp(hmax + ((uint64_t)a * HB + col / 256u) * 8u));
        }
        if (tid < A * HB)
            lds_st_f32(lay.hscale + 4u * tid, __builtin_amdgcn_ldexpf(1.0f, -limb_exponent(__uint_as_float(hm))));
        for (uint32_t i = tid + blockDim.x; i < A * HB; i += blockDim.x) {
            const int e = limb_exponent(__uint_as_float(*gp(hmax + (uint64_t)i * 8u)));
            lds_st_f32(lay.hscale + 4u * i, __builtin_amdgcn_ldexpf(1.0f, -e));
        }
    }
    // 3. This wave's first chunk, requested after every prologue load has been waited for.
    Chunk bufA[CU];
    {
        const TileRef tr =
            ca.count ? tile_ref<FMT>(ctx.L, uni_ptr(reinterpret_cast<const uint8_t*>(pa_raw)), ca.t) : idle_tile();
#pragma unroll
        for (uint32_t i = 0; i < CU; ++i)
            tok_load<FMT>(i < ca.count ? tr : idle_tile(), i < ca.count ? ca.col + i : 0u, ctx.ng, bufA[i]);
    }
    __syncthreads();
    const uint32_t n_active = uni(n_active_raw);
    if (n_active == 0) {
        // A refused route: the layer's output is zero (the status word says why).
        for (uint32_t i = b * blockDim.x + tid; i < s.width; i += gridDim.x * blockDim.x) *gp(in.out + i) = 0.0f;
        return;
    }
    // 4. The active experts' down pointers, for the chunks taken from the counter.
    if (tid < A) {
        const uint32_t e = lds_u32(lay.eid + 4u * tid);
        *lptr<uint64_t>(lay.dptr + 8u * tid) =
            pn ? *lptr<uint64_t>(lay.ptab + 8u * e) : reinterpret_cast<uint64_t>(in.experts[e].down);
    }
    __syncthreads();
    // 5. Stream.
    tok_stream<FMT, CU>(ctx, ka, ca, bufA);
    __syncthreads();
    // 6. Data-parallel tiles: each (tile, combine entry)'s expert sum over its chunks in order, a
    //    wave per pair (into the h limb area, no longer read), then a wave per tile combines.
    const TokRare r = lds_get<TokRare>(lay.rare);
    const uint32_t nd0 = r.ps.n + r.pr.n, cpe = r.p.C / CU, nent = r.K + (r.has_shared ? 1u : 0u);
    const VL_LDS CombineEntry* C = lptr<CombineEntry>(r.comb);
    for (uint32_t i = wave; i < r.p.q * nent; i += nw) {
        const uint32_t jj = i / nent, k = i - jj * nent, a = C[k].src >> 3;
        const float v = sum_parts(lay.part, nd0 + jj * (r.p.UJ / CU) + a * cpe, cpe);
        lds_st_f32(lay.hstage + i * 256u + lane * 4u, v + __shfl_xor(v, 32));
    }
    __syncthreads();
    for (uint32_t jj = wave; jj < r.p.q; jj += nw) {
        float acc = 0.0f;
        for (uint32_t k = 0; k < nent; ++k)
            acc = dn_combine(acc, lds_f32(lay.hstage + (jj * nent + k) * 256u + lane * 4u), k, r.K, r.semantics, C);
        dn_store(r.b * r.p.q + jj, acc, r.width, r.out, r.status);
    }
}

// ------------------------------------------------------------------------------------------
// Launches.
// ------------------------------------------------------------------------------------------

template <typename Kern, typename... Args>
static hipError_t tok_launch(Kern kernel, uint32_t grid, uint32_t shm, hipStream_t st, hipEvent_t* ev,
                             Args... args) {
    hipError_t e = ensure_dynamic_lds((const void*)kernel, shm);
    if (e != hipSuccess) return e;
    if (ev) hipExtLaunchKernelGGL(kernel, dim3(grid), dim3(kTokWaves * 64u), shm, st, ev[0], ev[1], 0u, args...);
    else hipLaunchKernelGGL(kernel, dim3(grid), dim3(kTokWaves * 64u), shm, st, args...);
    return hipGetLastError();
}

template <uint32_t FMT>
static hipError_t tok_gateup_fmt(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                                 hipStream_t st, hipEvent_t* ev) {
    const TokPlan p = tok_plan_gateup(s, w.blocks);
    const uint32_t shm = tok_lds_gu(table_bytes<FMT>(), s.width, p.max_chunks, s.experts).bytes;
    return tok_launch(k_tok_gateup<FMT>, p.grid, shm, st, ev, s, in, w, p);
}

template <uint32_t FMT>
static hipError_t tok_down_fmt(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                               hipStream_t st, hipEvent_t* ev) {
    const TokPlan p = tok_plan_down(s, w.blocks);
    const uint32_t shm = tok_lds_dn(table_bytes<FMT>(), p.A, s.inter, p.max_chunks).bytes;
    return tok_launch(k_tok_down<FMT>, p.grid, shm, st, ev, s, in, w, p);
}

hipError_t launch_tok_gateup(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                             hipStream_t st, hipEvent_t* ev) {
    switch (s.gate_type) {
        case VL_TYPE_IQ2_XXS: return tok_gateup_fmt<VL_TYPE_IQ2_XXS>(s, in, w, st, ev);
        case VL_TYPE_IQ3_XXS: return tok_gateup_fmt<VL_TYPE_IQ3_XXS>(s, in, w, st, ev);
        case VL_TYPE_IQ1_S: return tok_gateup_fmt<VL_TYPE_IQ1_S>(s, in, w, st, ev);
        case VL_TYPE_Q8_0: return tok_gateup_fmt<VL_TYPE_Q8_0>(s, in, w, st, ev);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_tok_down(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                           hipStream_t st, hipEvent_t* ev) {
    switch (s.down_type) {
        case VL_TYPE_IQ2_XXS: return tok_down_fmt<VL_TYPE_IQ2_XXS>(s, in, w, st, ev);
        case VL_TYPE_IQ3_XXS: return tok_down_fmt<VL_TYPE_IQ3_XXS>(s, in, w, st, ev);
        case VL_TYPE_IQ1_S: return tok_down_fmt<VL_TYPE_IQ1_S>(s, in, w, st, ev);
        case VL_TYPE_Q8_0: return tok_down_fmt<VL_TYPE_Q8_0>(s, in, w, st, ev);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace vl
