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
#include "vl_qmv_core.h"
#include "vl_kernels.h"
#include "vl_layout.h"
#include "vl_tables.h"

namespace vl {


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

template <uint32_t FMT, int NT, bool LDS_A>
__global__ void __launch_bounds__(256) k_qmv(const QmvBatch batch, uint32_t* status) {
    __shared__ LdsTables lds;
    __shared__ float partial[4][NT][32];
    extern __shared__ __align__(16) int8_t dyn_lds[];
    __shared__ __align__(16) int8_t s_zero[16];
    const QmvJob job = batch.device_jobs ? batch.device_jobs[blockIdx.y]
                                         : batch.inline_jobs[blockIdx.y];
    vl_tiled_layout L;
    if (job.rows == 0 || !vl_make_layout(FMT, job.rows, job.cols, &L)) return;
    const uint32_t t = blockIdx.x;
    if (t >= L.tiles) return;
    constexpr int S = Acc<NT>::kSlots;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = lane & 31;
    const int hh = lane >> 5;
    const uint32_t chunks = chunks_of<FMT>(L);
    const int slot = a_slot_of_lane();
    const bool on = slot < (int)job.tokens;
    const uint32_t lane_off = ((uint32_t)slot * 4u + a_limb_of_lane()) * 32u + 16u * hh;
    float accf[S];
    tile_partial<FMT, NT>(L, job.w, t, chunks * wave / 4u, chunks * (wave + 1) / 4u,
                          NT * 128u, lds, accf, [&](uint32_t& stride) -> const int8_t* {
        load_tables<FMT>(lds);
        if (threadIdx.x < 4) reinterpret_cast<uint32_t*>(s_zero)[threadIdx.x] = 0;
        if (LDS_A) stage_limbs<NT>(dyn_lds, job.xl, L.groups, NT, job.tokens,
                                   [](uint32_t s) { return s; });
        __syncthreads();
        if (!on) {
            stride = 0;
            return s_zero;
        }
        return LDS_A ? dyn_lds + lane_off : job.xl + lane_off;
    });
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
            const float sum = ((partial[0][tok][r] + partial[1][tok][r]) + partial[2][tok][r]) +
                              partial[3][tok][r];
            const float y = ldexpf(sum, -job.xe[tok]);
            if (!isfinite(y)) atomicOr(status, kStatusNonFiniteOutput);
            job.y[(uint64_t)tok * job.y_stride + row] = y;
        }
    }
}

template <uint32_t FMT>
static hipError_t launch_qmv_fmt(uint32_t slots, const QmvBatch& jobs, uint32_t njobs,
                                 uint32_t max_tiles, uint32_t lds_cols, uint32_t* status,
                                 hipStream_t stream) {
    const dim3 grid(max_tiles, njobs), block(256);
    // Activations are staged in LDS when every job's limbs fit.
    const uint32_t lds_bytes = lds_cols / 32u * slots * 128u;
    const bool lds_a = lds_bytes <= kMaxLdsLimbBytes;
    const uint32_t shm = lds_a ? lds_bytes : 0u;
    switch (slots * 2 + (lds_a ? 1 : 0)) {
        case 2: hipLaunchKernelGGL((k_qmv<FMT, 1, false>), grid, block, shm, stream, jobs, status); break;
        case 3: hipLaunchKernelGGL((k_qmv<FMT, 1, true>), grid, block, shm, stream, jobs, status); break;
        case 4: hipLaunchKernelGGL((k_qmv<FMT, 2, false>), grid, block, shm, stream, jobs, status); break;
        case 5: hipLaunchKernelGGL((k_qmv<FMT, 2, true>), grid, block, shm, stream, jobs, status); break;
        case 8: hipLaunchKernelGGL((k_qmv<FMT, 4, false>), grid, block, shm, stream, jobs, status); break;
        case 9: hipLaunchKernelGGL((k_qmv<FMT, 4, true>), grid, block, shm, stream, jobs, status); break;
        case 16: hipLaunchKernelGGL((k_qmv<FMT, 8, false>), grid, block, shm, stream, jobs, status); break;
        case 17: hipLaunchKernelGGL((k_qmv<FMT, 8, true>), grid, block, shm, stream, jobs, status); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_qmv(uint32_t type, uint32_t token_slots, const QmvBatch& jobs, uint32_t njobs,
                      uint32_t max_tiles, uint32_t max_cols, uint32_t* status, hipStream_t stream) {
    if (njobs == 0 || max_tiles == 0) return hipSuccess;
    if (!jobs.device_jobs && njobs > kInlineJobs) return hipErrorInvalidValue;
    switch (type) {
        case VL_TYPE_IQ2_XXS: return launch_qmv_fmt<VL_TYPE_IQ2_XXS>(token_slots, jobs, njobs, max_tiles, max_cols, status, stream);
        case VL_TYPE_IQ3_XXS: return launch_qmv_fmt<VL_TYPE_IQ3_XXS>(token_slots, jobs, njobs, max_tiles, max_cols, status, stream);
        case VL_TYPE_IQ1_S: return launch_qmv_fmt<VL_TYPE_IQ1_S>(token_slots, jobs, njobs, max_tiles, max_cols, status, stream);
        case VL_TYPE_Q8_0: return launch_qmv_fmt<VL_TYPE_Q8_0>(token_slots, jobs, njobs, max_tiles, max_cols, status, stream);
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
