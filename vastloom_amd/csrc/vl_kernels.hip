// HIP kernels for the quantized routed-expert path on gfx950 (MI355X).
//
//   k_pack      GGUF block bytes -> tiled device layout (vl_layout.h), once per resident matrix
//   k_dequant   tiled matrix -> float32 rows, through the same chunk loads and decoders as the
//               matvec; used to prove the decode bit-exact against the reference
//   k_prep_x    float32 activations -> int8 limbs, one exponent per 256 columns and token
//   k_matvec    persistent quantized matvec (vl_stream.h): every wave streams an equal share of
//               the matrix's (tile, superblock) units; the last wave of each tile adds the
//               tile's partials in a fixed order and writes the rows
//
// Q4_K, Q5_K, Q6_K, MXFP4, BF16 and F32 matrices stay in their GGUF bytes and are handed on to the
// kernels of vl_gguf.hip by the launchers below.
//
// Numerics of k_matvec: every product w*x is formed exactly in integers (weights are exact small
// integers times a per-group float factor, activations are 30-bit fixed point per 256-column
// block); each group's int32 MFMA result is scaled by the group's integer scale, summed exactly
// over the superblock and converted to float once per superblock. The result is deterministic
// and its error is a few float roundings of the row's partial sums, well inside
// 1e-5 * |w| * |x|.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vl_kernels.h"
#include "vl_layout.h"
#include "vl_stream.h"

namespace vl {

uint32_t stream_blocks() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return cus > 0 ? (uint32_t)cus : 0u;
}

hipError_t ensure_dynamic_lds(const void* kernel, uint32_t bytes) {
    static thread_local const void* done[128];
    static thread_local uint32_t limit[128];
    static thread_local uint32_t n = 0;
    for (uint32_t i = 0; i < n; ++i)
        if (done[i] == kernel && limit[i] >= bytes) return hipSuccess;
    // The kernels address their dynamic LDS from LDS address 0 (vl_decode.h), which holds only
    // when they declare no static LDS.
    hipFuncAttributes attr{};
    hipError_t e = hipFuncGetAttributes(&attr, kernel);
    if (e != hipSuccess) return e;
    if (attr.sharedSizeBytes != 0) return hipErrorInvalidKernelFile;
    e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e != hipSuccess) return e;
    if (n < 128) {
        done[n] = kernel;
        limit[n++] = bytes;
    }
    return hipSuccess;
}

// ------------------------------------------------------------------------------------------
// Pack: GGUF -> tiled. One thread per (row, superblock) for the IQ formats and per (row,
// block) for Q8_0; padded rows are written as zeros.
// ------------------------------------------------------------------------------------------

__device__ __forceinline__ void copy_bytes(uint8_t* dst, const uint8_t* src, int n, bool zero) {
    for (int i = 0; i < n; ++i) dst[i] = zero ? 0 : src[i];
}

__device__ __forceinline__ uint32_t ld_u32_bytes(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// Rows [row0, row1) of the padded matrix; gguf points at the GGUF bytes of row row0.
__global__ void k_pack(vl_tiled_layout L, const uint8_t* __restrict__ gguf,
                       uint8_t* __restrict__ out, uint32_t row0, uint32_t row1) {
    const uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool q8 = L.type == VL_TYPE_Q8_0;
    const uint32_t units = q8 ? L.groups : L.superblocks;  // blocks per row
    if (id >= (uint64_t)(row1 - row0) * units) return;
    const uint32_t r = row0 + (uint32_t)(id / units), b = (uint32_t)(id % units);
    const uint32_t t = r / 32u, j = r % 32u;
    const bool pad = r >= L.rows;
    // Padded rows read nothing; their source pointer stays on the first block.
    const uint8_t* src = pad ? gguf : gguf + ((uint64_t)(r - row0) * units + b) * L.block_bytes;
    const uint32_t NG = L.groups, NB = L.superblocks;
    uint8_t* S = out + L.plane2;
    switch (L.type) {
        case VL_TYPE_IQ2_XXS: {
            // GGUF group g: 4 grid bytes at 2 + 8g, then the sign/scale word.
            uint32_t grid[8], aux[8];
            for (int g = 0; g < 8; ++g) {
                grid[g] = pad ? 0u : ld_u32_bytes(src + 2 + 8 * g);
                aux[g] = pad ? 0u : ld_u32_bytes(src + 6 + 8 * g);
            }
            for (uint32_t h = 0; h < 2; ++h) {
                uint32_t wv[8];
                for (int q = 0; q < 4; ++q) {
                    const uint32_t ga = grid[2 * q] >> (16 * h), gb = grid[2 * q + 1] >> (16 * h);
                    wv[q] = (ga & 0xffffu) | ((gb & 0xffffu) << 16);
                    const uint32_t sa = aux[2 * q] >> (14 * h), sb = aux[2 * q + 1] >> (14 * h);
                    wv[4 + q] = (sa & 0x3fffu) | ((sb & 0x3fffu) << 14) | ((aux[4 * h + q] >> 28) << 28);
                }
                uint32_t* dst = reinterpret_cast<uint32_t*>(
                    out + ((((uint64_t)t * NB + b) * 2u + h) * 32u + j) * 32u);
                for (int q = 0; q < 8; ++q) dst[q] = wv[q];
            }
            copy_bytes(out + L.plane1 + (((uint64_t)t * NB + b) * 32u + j) * 2u, src, 2, pad);
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

hipError_t launch_pack_rows(const vl_tiled_layout& L, const uint8_t* gguf_row0, uint8_t* tiled,
                            uint32_t row0, uint32_t row1, hipStream_t stream) {
    if (!vl_type_tiled(L.type)) return launch_gguf_copy_rows(L, gguf_row0, tiled, row0, row1, stream);
    if (row0 >= row1 || row1 > L.rows_padded) return hipErrorInvalidValue;
    const uint64_t units = (uint64_t)(row1 - row0) * (L.type == VL_TYPE_Q8_0 ? L.groups : L.superblocks);
    const uint32_t block = 256;
    const uint64_t grid = (units + block - 1) / block;
    hipLaunchKernelGGL(k_pack, dim3((uint32_t)grid), dim3(block), 0, stream, L, gguf_row0, tiled,
                       row0, row1);
    return hipGetLastError();
}

hipError_t launch_pack(const vl_tiled_layout& L, const uint8_t* gguf, uint8_t* tiled,
                       hipStream_t stream) {
    return launch_pack_rows(L, gguf, tiled, 0u, L.rows_padded, stream);
}

// ------------------------------------------------------------------------------------------
// Dequantize (tiled -> float rows), one wave per (tile, unit). Lane (n, hh) writes 16 weights of
// every group of the unit: w = (float)(q * sc) * (d * factor), the reference value exactly.
// ------------------------------------------------------------------------------------------

template <uint32_t FMT>
__global__ void __launch_bounds__(256) k_dequant(vl_tiled_layout L, const uint8_t* __restrict__ w,
                                                 float* __restrict__ out) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) uint8_t lds[];
    fill_tables<FMT>(lds);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t n = lane & 31u;
    const int hh = (int)(lane >> 5);
    const uint32_t units = units_per_row(FMT, L.cols);
    const uint64_t item = (uint64_t)blockIdx.x * 4u + wave;
    if (item >= (uint64_t)L.tiles * units) return;
    const uint32_t t = (uint32_t)(item / units), c = (uint32_t)(item % units);
    const uint32_t row = t * 32u + n;
    Chunk ch;
    load_chunk<FMT>(tile_ref<FMT>(L, w, t), c, L.groups, ch);
    if (FMT == VL_TYPE_Q8_0) {
        if (row >= L.rows) return;
        for (int b = 0; b < 4; ++b) {
            const uint32_t G = 4u * c + b;
            if (G >= L.groups) break;
            const uint4& q = b == 0 ? ch.q0 : b == 1 ? ch.q1 : b == 2 ? ch.q2 : ch.q3;
            const float d = half_bits_to_float((b < 2 ? ch.d0 : ch.d1) >> (16 * (b & 1)));
            float* dst = out + (uint64_t)row * L.cols + G * 32u + 16u * hh;
            for (int e = 0; e < 16; ++e) {
                const int qv = (int)(int8_t)(word(q, e >> 2) >> (8 * (e & 3)));
                dst[e] = (float)qv * d;
            }
        }
        return;
    }
    ChunkDecoder<FMT> dec;
    dec.init(ch);  // all lanes: the IQ2_XXS halves exchange scale bytes
    if (row >= L.rows) return;
    const float df = half_bits_to_float(ch.d0) * unit_factor<FMT>();
    const uint32_t lane_off = (n % kTabCopies) * 8u;
    for (int g = 0; g < 8; ++g) {
        int sc = 1;
        const i32x4 frag = dec.group(ch, g, lane_off, hh, sc);
        float* dst = out + (uint64_t)row * L.cols + (uint64_t)c * 256u + 32u * g + 16u * hh;
        for (int e = 0; e < 16; ++e) {
            const int q = (int)(int8_t)((uint32_t)frag[e >> 2] >> (8 * (e & 3)));
            dst[e] = (float)(q * sc) * df;
        }
    }
}

template <uint32_t FMT>
static hipError_t launch_dequant_fmt(const vl_tiled_layout& L, const uint8_t* tiled, float* out,
                                     hipStream_t stream) {
    const uint64_t items = (uint64_t)L.tiles * units_per_row(FMT, L.cols);
    const uint32_t shm = table_bytes<FMT>() + 16u;
    const hipError_t e = ensure_dynamic_lds((const void*)k_dequant<FMT>, shm);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_dequant<FMT>, dim3((uint32_t)((items + 3) / 4)), dim3(256), shm, stream,
                       L, tiled, out);
    return hipGetLastError();
}

hipError_t launch_dequant(const vl_tiled_layout& L, const uint8_t* tiled, float* out,
                          hipStream_t stream) {
    if (!vl_type_tiled(L.type)) return launch_gguf_dequant(L, tiled, out, stream);
    switch (L.type) {
        case VL_TYPE_IQ2_XXS: return launch_dequant_fmt<VL_TYPE_IQ2_XXS>(L, tiled, out, stream);
        case VL_TYPE_IQ3_XXS: return launch_dequant_fmt<VL_TYPE_IQ3_XXS>(L, tiled, out, stream);
        case VL_TYPE_IQ1_S: return launch_dequant_fmt<VL_TYPE_IQ1_S>(L, tiled, out, stream);
        case VL_TYPE_Q8_0: return launch_dequant_fmt<VL_TYPE_Q8_0>(L, tiled, out, stream);
        default: return hipErrorInvalidValue;
    }
}

// ------------------------------------------------------------------------------------------
// Matvec.
// ------------------------------------------------------------------------------------------

// Workspace of one matvec call.
struct MatvecWs {
    uint64_t off_xexp, off_xflags, off_xlimbs, off_counters, off_rec, bytes;
    uint32_t xblocks, slots, tiles;
};

static inline uint64_t al256(uint64_t v) { return (v + 255u) & ~uint64_t(255); }

static MatvecWs matvec_ws(uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t blocks) {
    MatvecWs m{};
    m.xblocks = exp_blocks(cols);
    m.slots = limb_slots(tokens);
    m.tiles = (rows + 31u) / 32u;
    uint64_t o = 256;  // status word and padding
    m.off_xexp = o; o = al256(o + (uint64_t)m.xblocks * 8u * 4u);
    m.off_xflags = o; o = al256(o + (uint64_t)m.xblocks * 8u * 4u);
    m.off_xlimbs = o; o = al256(o + (uint64_t)(cols / 32u) * m.slots * 128u);
    m.off_counters = o; o = al256(o + (uint64_t)m.tiles * 4u);
    m.off_rec = o; o = al256(o + ((uint64_t)blocks * kStreamWaves + m.tiles) * m.slots * 64u * 4u);
    m.bytes = o;
    return m;
}

uint64_t matvec_workspace_bytes(uint32_t type, uint32_t rows, uint32_t cols, uint32_t tokens,
                                uint32_t blocks) {
    if (!vl_type_tiled(type)) return 256u;  // the status word alone
    return matvec_ws(rows, cols, tokens, blocks).bytes;
}

__global__ void __launch_bounds__(256) k_prep_x(const float* __restrict__ x, uint32_t cols,
                                                uint32_t tokens, uint8_t* ws, MatvecWs m) {
    if (blockIdx.x == 0) {
        if (threadIdx.x == 0) *reinterpret_cast<uint32_t*>(ws) = 0;
        uint32_t* cnt = reinterpret_cast<uint32_t*>(ws + m.off_counters);
        for (uint32_t i = threadIdx.x; i < m.tiles; i += blockDim.x) cnt[i] = 0;
    }
    prep_x_block(x, cols, cols, 0u, tokens, m.slots, 8u, blockIdx.x,
                 reinterpret_cast<int8_t*>(ws + m.off_xlimbs), reinterpret_cast<int*>(ws + m.off_xexp),
                 reinterpret_cast<uint32_t*>(ws + m.off_xflags));
}

template <uint32_t FMT, int NT, bool LDS>
struct Matvec {
    uint32_t chunks, nmat, ng;
    ASrc<LDS, NT * 128u> as;
    float hscale;
    vl_tiled_layout L;
    const uint8_t* W;
    uint32_t tokens, UJ, TU, NW, wid;
    uint32_t stage_off, scale_off;
    const uint8_t* lds;
    const uint8_t* ws;
    MatvecWs m;
    float* y;

    __device__ TileRef tref(uint32_t j, uint32_t) const { return tile_ref<FMT>(L, W, j); }

    __device__ void job_begin(uint32_t) {
        const uint32_t mm = threadIdx.x & 31u, kh = (threadIdx.x >> 5) & 1u;
        const uint32_t sl = a_slot(mm), limb = a_limb(mm);
        const uint32_t off = (sl < tokens ? sl : 0u) * 128u + limb * 32u + 16u * kh;
        if (LDS) as.off = stage_off + off;
        else as.ptr = reinterpret_cast<const int8_t*>(ws + m.off_xlimbs) + off;
    }

    __device__ void scales(uint32_t, uint32_t c, float (&fs)[NT]) const {
        const uint32_t eb = FMT == VL_TYPE_Q8_0 ? c / 2u : c;
#pragma unroll
        for (int s = 0; s < NT; ++s) fs[s] = lds_load<float>(scale_off + 4u * (8u * eb + s));
    }

    static constexpr bool kPrefetch = false;

    __device__ uint32_t* store(uint32_t j, const float (&m0)[NT], const float (&)[NT], uint32_t& kc) const {
        const uint32_t lane = threadIdx.x & 63u;
        float* rec = reinterpret_cast<float*>(const_cast<uint8_t*>(ws) + m.off_rec);
        float* r = rec + (uint64_t)(wid + j) * (NT * 64u);
#pragma unroll
        for (int s = 0; s < NT; ++s) store_shared(r + s * 64u + lane, m0[s]);
        kc = wave_of_unit(j * UJ + UJ - 1u, NW, TU) - wave_of_unit(j * UJ, NW, TU) + 1u;
        return reinterpret_cast<uint32_t*>(const_cast<uint8_t*>(ws) + m.off_counters) + j;
    }

    __device__ void fixup(uint32_t j) const {
        const uint32_t lane = threadIdx.x & 63u;
        const float* rec = reinterpret_cast<const float*>(ws + m.off_rec);
        const uint32_t first = wave_of_unit(j * UJ, NW, TU);
        const uint32_t last = wave_of_unit(j * UJ + UJ - 1u, NW, TU);
        const uint32_t n = lane & 31u, hh = lane >> 5, row = j * 32u + n;
        bool bad = false;
#pragma unroll
        for (int i = 0; i < (NT + 1) / 2; ++i) {
            const uint32_t sl = 2u * i + hh;
            if (sl < tokens) {
                float v[1];
                sum_records<NT, 1>(rec, NT * 64u, j, first, last, sl, n, v);
                if (row < L.rows) {
                    bad |= !isfinite(v[0]);
                    *gp(y + (uint64_t)sl * L.rows + row) = v[0];
                }
            }
        }
        if (__any(bad) && lane == 0)
            or_bits(reinterpret_cast<uint32_t*>(const_cast<uint8_t*>(ws)), kStatusNonFiniteOutput);
    }
};

template <uint32_t FMT, int NT, bool LDS>
__global__ void __launch_bounds__(stream_threads<NT>()) k_matvec(vl_tiled_layout L, const uint8_t* W,
                                                           uint32_t tokens, float* y, uint8_t* ws,
                                                           MatvecWs m) {
    extern __shared__ __align__(16) uint8_t lds[];
    fill_tables<FMT>(lds);
    constexpr uint32_t TB = table_bytes<FMT>();
    const uint32_t stage_bytes = LDS ? (L.cols / 32u) * NT * 128u : 0u;
    const uint32_t scale_off = TB + stage_bytes;  // then m.xblocks * 8 scales and the wave flags
    if (LDS) {
        const uint4* src = reinterpret_cast<const uint4*>(ws + m.off_xlimbs);
        uint4* dst = reinterpret_cast<uint4*>(lds + TB);
        copy_to_lds(dst, src, stage_bytes / 16u, threadIdx.x, blockDim.x);
    }
    int nonfinite = 0;
    {
        const int* xe = reinterpret_cast<const int*>(ws + m.off_xexp);
        const uint32_t* xf = reinterpret_cast<const uint32_t*>(ws + m.off_xflags);
        float* sc = reinterpret_cast<float*>(lds + scale_off);
        for (uint32_t i = threadIdx.x; i < m.xblocks * 8u; i += blockDim.x) {
            const bool live = (i & 7u) < tokens;
            sc[i] = live ? __builtin_amdgcn_ldexpf(1.0f, -*gp(xe + i)) : 0.0f;
            if (live && *gp(xf + i)) nonfinite = 1;
        }
    }
    const bool any_nonfinite =
        block_any(nonfinite != 0, reinterpret_cast<uint32_t*>(lds + scale_off + m.xblocks * 32u));
    if (blockIdx.x == 0 && threadIdx.x == 0 && any_nonfinite)
        or_bits(reinterpret_cast<uint32_t*>(ws), kStatusNonFiniteInput);
    Matvec<FMT, NT, LDS> pol;
    pol.L = L;
    pol.W = W;
    pol.tokens = tokens;
    pol.chunks = units_per_row(FMT, L.cols);
    pol.nmat = 1;
    pol.ng = L.groups;
    pol.UJ = pol.chunks;
    pol.TU = L.tiles * pol.UJ;
    pol.NW = active_waves(gridDim.x * stream_waves<NT>(), pol.TU);
    pol.wid = blockIdx.x * stream_waves<NT>() + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    pol.stage_off = TB;
    pol.scale_off = scale_off;
    pol.lds = lds;
    pol.ws = ws;
    pol.m = m;
    pol.y = y;
    pol.hscale = (threadIdx.x & 32u) ? 65536.0f : 1.0f;
    stream_range<FMT, NT, LDS>(pol, range_begin(pol.wid, pol.NW, pol.TU),
                               range_begin(pol.wid + 1u, pol.NW, pol.TU));
}

// Dynamic LDS of one workgroup on gfx950 (the matvec kernel has no static LDS).
constexpr uint32_t kMatvecLdsBudget = 160u * 1024u - 256u;

template <uint32_t FMT, int NT>
static hipError_t launch_matvec_nt(const vl_tiled_layout& L, const uint8_t* w, uint32_t tokens,
                                   float* y, uint8_t* ws, const MatvecWs& m, uint32_t blocks,
                                   hipStream_t st) {
    const uint32_t stage = (L.cols / 32u) * NT * 128u;
    const uint32_t TB = table_bytes<FMT>();
    const uint32_t base = TB + m.xblocks * 8u * 4u + kStreamWaves * 4u;  // tables, scales, flags
    if (base + stage <= kMatvecLdsBudget) {
        const uint32_t shm = base + stage;
        const hipError_t e = ensure_dynamic_lds((const void*)k_matvec<FMT, NT, true>, shm);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((k_matvec<FMT, NT, true>), dim3(blocks), dim3(stream_threads<NT>()), shm, st,
                           L, w, tokens, y, ws, m);
    } else {
        const uint32_t shm = base;
        const hipError_t e = ensure_dynamic_lds((const void*)k_matvec<FMT, NT, false>, shm);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((k_matvec<FMT, NT, false>), dim3(blocks), dim3(stream_threads<NT>()), shm, st,
                           L, w, tokens, y, ws, m);
    }
    return hipGetLastError();
}

template <uint32_t FMT>
static hipError_t launch_matvec_fmt(const vl_tiled_layout& L, const uint8_t* w, uint32_t tokens,
                                    float* y, uint8_t* ws, const MatvecWs& m, uint32_t blocks,
                                    hipStream_t st) {
    switch (m.slots) {
        case 1: return launch_matvec_nt<FMT, 1>(L, w, tokens, y, ws, m, blocks, st);
        case 2: return launch_matvec_nt<FMT, 2>(L, w, tokens, y, ws, m, blocks, st);
        case 4: return launch_matvec_nt<FMT, 4>(L, w, tokens, y, ws, m, blocks, st);
        default: return launch_matvec_nt<FMT, 8>(L, w, tokens, y, ws, m, blocks, st);
    }
}

hipError_t launch_matvec(const vl_tiled_layout& L, const uint8_t* w, const float* x,
                         uint32_t tokens, float* y, uint8_t* workspace, uint32_t blocks,
                         hipStream_t stream) {
    if (!vl_type_tiled(L.type)) return launch_gguf_matvec(L, w, x, tokens, y, workspace, stream);
    if (tokens == 0 || tokens > 8 || L.cols % 32u != 0 || blocks == 0) return hipErrorInvalidValue;
    const MatvecWs m = matvec_ws(L.rows, L.cols, tokens, blocks);
    hipLaunchKernelGGL(k_prep_x, dim3(m.xblocks), dim3(256), 0, stream, x, L.cols, tokens,
                       workspace, m);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    switch (L.type) {
        case VL_TYPE_IQ2_XXS: return launch_matvec_fmt<VL_TYPE_IQ2_XXS>(L, w, tokens, y, workspace, m, blocks, stream);
        case VL_TYPE_IQ3_XXS: return launch_matvec_fmt<VL_TYPE_IQ3_XXS>(L, w, tokens, y, workspace, m, blocks, stream);
        case VL_TYPE_IQ1_S: return launch_matvec_fmt<VL_TYPE_IQ1_S>(L, w, tokens, y, workspace, m, blocks, stream);
        case VL_TYPE_Q8_0: return launch_matvec_fmt<VL_TYPE_Q8_0>(L, w, tokens, y, workspace, m, blocks, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace vl
