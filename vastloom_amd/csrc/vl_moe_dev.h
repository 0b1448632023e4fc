// Device-side definitions shared by the MoE-layer kernels (vl_moe.hip, vl_moe_token.hip): the
// workspace records that pass between launches, score and key functions of the routing, wave
// reductions and the SwiGLU of each semantics.
#ifndef VL_MOE_DEV_H
#define VL_MOE_DEV_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vl_kernels.h"
#include "vl_moe.h"
#include "vl_stream.h"

namespace vl {

struct ActiveExpert {
    uint32_t expert;   // expert id; the shared expert is `experts`
    uint32_t ntok;     // tokens routed to it (slots 0..ntok-1)
    uint32_t apply_w;  // multiply h by the slot's route weight before the down projection
    float limit;       // SwiGLU clamp (0 = none)
    uint32_t tok[kMoeMaxTokens];
    float route_w[kMoeMaxTokens];
};

struct MoeHeader {
    uint32_t status;
    uint32_t n_active;
    uint32_t reserved[14];
};

struct CombineEntry {
    uint32_t src;  // (active index << 3) | slot
    float w;
};

constexpr uint32_t kMaxActive = kMoeMaxTokens * kMoeMaxTopK + 1;

// Bytes of one expert's h limbs, [inter/32][slots][4][32].
__host__ __device__ inline uint32_t down_expert_bytes(uint32_t inter, uint32_t slots) {
    return (inter / 32u) * slots * 128u;
}

template <typename T>
__device__ __forceinline__ T* ws_ptr(const MoeWorkspace& w, uint64_t off) {
    return reinterpret_cast<T*>(w.base + off);
}

// Counter regions (u32 words at off_counters).
struct MoeCounters {
    uint32_t* gu;    // [A][tiles_gu]   gate/up tile handoff
    uint32_t* dn;    // [A][tiles_dn]   down tile handoff
    uint32_t* tile;  // [tiles_dn]      experts done per output tile
    uint32_t* hmax;  // [A][hblocks][8] max |h| bits per 256-row block of h and slot
};

__device__ __forceinline__ MoeCounters counters_of(const MoeWorkspace& w) {
    MoeCounters c;
    uint32_t* p = ws_ptr<uint32_t>(w, w.off_counters);
    const uint32_t A = w.max_active;
    c.gu = p;
    c.dn = c.gu + A * w.tiles_gu;
    c.tile = c.dn + A * w.tiles_dn;
    c.hmax = c.tile + w.tiles_dn;
    return c;
}

__device__ __forceinline__ float score_of(float logit, uint32_t fn) {
    const double p = (double)logit;
    if (fn == kScoreSigmoid) {
        if (p >= 0.0) return (float)(1.0 / (1.0 + exp(-p)));
        const double q = exp(p);
        return (float)(q / (1.0 + q));
    }
    const double sp = (p > 0.0 ? p : 0.0) + log1p(exp(-fabs(p)));
    return (float)sqrt(sp);
}

// Order-preserving map of a float to uint32: a larger float gives a larger key, equal floats
// (+0 and -0 included) give equal keys, and every key of a finite float is above 1 (non-finite
// keys are 1; such a token is refused anyway).
__device__ __forceinline__ uint32_t float_key(float f) {
    if (!isfinite(f)) return 1u;
    const uint32_t b = __float_as_uint(f == 0.0f ? 0.0f : f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// The float a key of a finite float stands for (inverse of float_key above 1).
__device__ __forceinline__ float key_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ double wave_sum_f64(double v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Maximum over the wave, by DPP row operations (all lanes active); the result is uniform.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    // The DPP source's "old" value is 0, the identity of the maximum, so rows a step leaves out
    // add nothing and each step folds into one v_max_u32 with a DPP operand.
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xb1, 0xf, 0xf, false));   // quad [1,0,3,2]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4e, 0xf, 0xf, false));   // quad [2,3,0,1]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false));  // row half mirror
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xf, 0xf, false));  // row mirror
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false));  // row bcast 15
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false));  // row bcast 31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    // As wave_max_u32, with 0xffffffff, the identity of the minimum, as the DPP "old" value.
    constexpr int kId = -1;
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0xb1, 0xf, 0xf, false));
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x4e, 0xf, 0xf, false));
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x141, 0xf, 0xf, false));
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x140, 0xf, 0xf, false));
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x142, 0xa, 0xf, false));
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x143, 0xc, 0xf, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ float silu_f(float v) {
    // sigmoid_f / silu_f of qwen3_8_flash_next_reference.cpp:244-255, in float.
    float sg;
    if (v >= 0.0f) {
        sg = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-v)));
    } else {
        const float z = expf(v);
        sg = __fdiv_rn(z, __fadd_rn(1.0f, z));
    }
    return __fmul_rn(v, sg);
}

__device__ __forceinline__ float swiglu(uint32_t sem, float g, float u, float limit,
                                        bool apply_w, float route_w) {
    if (sem == kSemDeepseek) {
        double gv = (double)g, uv = (double)u;
        if (limit > 0.0f) {
            const double L = (double)limit;
            gv = gv < L ? gv : L;
            uv = uv < -L ? -L : (uv > L ? L : uv);
        }
        double v = __dmul_rn(__ddiv_rn(gv, __dadd_rn(1.0, exp(-gv))), uv);
        if (apply_w) v = __dmul_rn(v, (double)route_w);
        return (float)v;
    }
    if (sem == kSemQwen) return __fmul_rn(silu_f(g), u);
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u);
}

}  // namespace vl

#endif  // VL_MOE_DEV_H
