// MoE layer on the device, for up to 8 tokens routed to top-k of E experts plus a shared expert:
//
//   k_moe_router   gate logits, float64 accumulation per expert row (the reference's linear_f /
//                  gate_logits numerics), and the per-call status/maximum words zeroed
//   k_moe_route    per-token scores and top-k (one wave per token), then the active-expert list:
//                  distinct experts in ascending id with their tokens, and each token's combine
//                  order
//   k_prep_limbs   the tokens' int8 limbs (vl_kernels.hip)
//   k_moe_gateup   per (active expert, 32-row tile): gate and up tiles in one block (4 waves each,
//                  int8 MFMA), then the SwiGLU of the semantics into h; |h| maxima per token
//   k_moe_hprep    h -> limbs with one exponent per (expert, token)
//   k_moe_down     per (active expert, 32-row tile) down projection into per-expert partials
//   k_moe_combine  partials -> layer output in the reference's combine order
//
// The routing, clamp, route-weight placement and combine order follow the reference code named
// in vl_moe.h. Every reduction has a fixed order, so results are deterministic.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vl_kernels.h"
#include "vl_moe.h"
#include "vl_qmv_core.h"

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

static inline uint64_t align256(uint64_t v) { return (v + 255u) & ~uint64_t(255); }

bool moe_shape_ok(const MoeShape& s) {
    uint32_t be = 0, bb = 0;
    if (s.tokens == 0 || s.tokens > kMoeMaxTokens || s.top_k == 0 || s.top_k > kMoeMaxTopK ||
        s.experts == 0 || s.experts > 1024 || s.top_k > s.experts)
        return false;
    if (!vl_block_shape(s.gate_type, &be, &bb) || s.width % be || s.width % 256u) return false;
    if (s.width > 8192u) return false;  // the routing block stages one token row in registers
    if (!vl_block_shape(s.down_type, &be, &bb) || s.inter % be || s.inter % 32u) return false;
    if (s.semantics > kSemPlain || s.routing > kRouteGiven || s.score_fn > kScoreSigmoid) return false;
    return true;
}

static uint32_t max_active(const MoeShape& s) {
    const uint32_t routed = s.tokens * s.top_k < s.experts ? s.tokens * s.top_k : s.experts;
    return routed + (s.has_shared ? 1u : 0u);
}

MoeWorkspace moe_workspace_layout(const MoeShape& s, void* base) {
    MoeWorkspace w{};
    w.base = static_cast<uint8_t*>(base);
    w.max_active = max_active(s);
    const uint64_t A = w.max_active, T = s.tokens, K = s.top_k;
    uint64_t o = 0;
    w.off_header = o; o = align256(o + sizeof(MoeHeader));
    w.off_logits = o; o = align256(o + T * s.experts * 4u);
    w.off_route_idx = o; o = align256(o + T * K * 4u);
    w.off_route_w = o; o = align256(o + T * K * 4u);
    w.off_active = o; o = align256(o + A * sizeof(ActiveExpert));
    w.off_combine = o; o = align256(o + T * (K + 1) * sizeof(CombineEntry));
    w.off_hmax = o; o = align256(o + A * kMoeMaxTokens * 4u);
    w.off_hexp = o; o = align256(o + A * kMoeMaxTokens * 4u);
    w.off_xexp = o; o = align256(o + kMoeMaxTokens * 4u);
    w.off_xlimbs = o; o = align256(o + limb_bytes(s.width, s.tokens));
    w.off_h = o; o = align256(o + A * kMoeMaxTokens * s.inter * 4u);
    w.off_hlimbs = o; o = align256(o + A * (s.inter / 32u) * kMoeMaxTokens * 128u);
    w.off_ypart = o; o = align256(o + A * kMoeMaxTokens * (uint64_t)s.width * 4u);
    w.bytes = o;
    return w;
}

uint64_t moe_workspace_bytes(const MoeShape& s) { return moe_workspace_layout(s, nullptr).bytes; }

template <typename T>
__device__ __forceinline__ T* ws_ptr(const MoeWorkspace& w, uint64_t off) {
    return reinterpret_cast<T*>(w.base + off);
}

// ------------------------------------------------------------------------------------------
// Router logits: one wave per expert row, float64 products and sums, one rounding.
// ------------------------------------------------------------------------------------------

__device__ __forceinline__ double wave_sum_f64(double v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// One block per expert row; the four waves take interleaved quarters of the row (every lane
// keeps its float4 loads in flight), then the partial sums are added in wave order.
__global__ void __launch_bounds__(256) k_moe_router(const MoeShape s, const MoeInputs in,
                                                    const MoeWorkspace w) {
    __shared__ double red[kMoeMaxTokens][4];
    // Per-call words later kernels accumulate into.
    if (blockIdx.x == 0) {
        MoeHeader* h = ws_ptr<MoeHeader>(w, w.off_header);
        if (threadIdx.x < 2) (&h->status)[threadIdx.x] = 0;
        uint32_t* hmax = ws_ptr<uint32_t>(w, w.off_hmax);
        for (uint32_t i = threadIdx.x; i < w.max_active * kMoeMaxTokens; i += blockDim.x) hmax[i] = 0;
    }
    if (s.routing == kRouteGiven) return;
    const uint32_t e = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float4* row = reinterpret_cast<const float4*>(in.router + (uint64_t)e * s.width);
    const uint32_t n4 = s.width / 4u;
    float4 wv[8];
    int nv = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t i = threadIdx.x + 256u * j;
        if (i < n4) { wv[j] = row[i]; nv = j + 1; }
    }
    for (uint32_t t = 0; t < s.tokens; ++t) {
        const float4* xr = reinterpret_cast<const float4*>(in.x + (uint64_t)t * s.width);
        double acc = 0.0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j < nv) {
                const float4 a = wv[j], b = xr[threadIdx.x + 256u * j];
                acc += (double)a.x * (double)b.x;
                acc += (double)a.y * (double)b.y;
                acc += (double)a.z * (double)b.z;
                acc += (double)a.w * (double)b.w;
            }
        }
        // Rows wider than 8192 continue with plain loads.
        for (uint32_t i = threadIdx.x + 2048u; i < n4; i += 256u) {
            const float4 a = row[i], b = xr[i];
            acc += (double)a.x * (double)b.x;
            acc += (double)a.y * (double)b.y;
            acc += (double)a.z * (double)b.z;
            acc += (double)a.w * (double)b.w;
        }
        acc = wave_sum_f64(acc);
        if (lane == 0) red[t][wave] = acc;
    }
    __syncthreads();
    if (threadIdx.x < s.tokens) {
        const uint32_t t = threadIdx.x;
        ws_ptr<float>(w, w.off_logits)[t * s.experts + e] =
            (float)(((red[t][0] + red[t][1]) + red[t][2]) + red[t][3]);
    }
}

// ------------------------------------------------------------------------------------------
// Routing.
// ------------------------------------------------------------------------------------------

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

// Key order for selection: larger key first, ties to the lower id.
__device__ __forceinline__ bool beats(float ka, uint32_t ia, float kb, uint32_t ib) {
    return ka > kb || (ka == kb && ia < ib);
}

__device__ __forceinline__ bool beats_d(double ka, uint32_t ia, double kb, uint32_t ib) {
    return ka > kb || (ka == kb && ia < ib);
}

// Limbs of one token's activations by the whole block: max |x| (all loads issued at once,
// kept in registers), exponent, then the four digits of round(x * 2^e) for every column, the
// same encoding as k_prep_limbs. cols <= 4 * 4 * blockDim.x.
__device__ void prep_token_block(const float* __restrict__ x, uint32_t cols, uint32_t slots,
                                 uint32_t tok, int8_t* __restrict__ xl, int* __restrict__ xe,
                                 uint32_t* status, float* red) {
    constexpr int kPer = 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const uint32_t n4 = cols / 4u;
    float4 v[kPer];
    float m = 0.0f;
    bool finite = true;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const uint32_t i = threadIdx.x + blockDim.x * j;
        v[j] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        finite &= isfinite(v[j].x) && isfinite(v[j].y) && isfinite(v[j].z) && isfinite(v[j].w);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    }
    if (!finite) {
        atomicOr(status, kStatusNonFiniteInput);
        m = 0.0f;
    }
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = 0.0f;
    for (int i = 0; i < nwaves; ++i) m = fmaxf(m, red[i]);
    __syncthreads();
    int q = 0;
    frexpf(m, &q);
    const int e = m > 0.0f && isfinite(m) ? 30 - q : 0;
    if (threadIdx.x == 0) xe[tok] = e;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const uint32_t i = threadIdx.x + blockDim.x * j;
        if (i >= n4) continue;
        const float vs[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        uint32_t packed[4] = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            int X = isfinite(vs[k]) ? (int)rintf(ldexpf(vs[k], e)) : 0;
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const int digit = l < 3 ? (int)(int8_t)(X & 0xff) : X;
                packed[l] |= ((uint32_t)digit & 0xffu) << (8 * k);
                X = (X - digit) >> 8;
            }
        }
        const uint32_t k4 = 4u * i;
        const uint64_t base = ((uint64_t)(k4 / 32u) * slots + tok) * 128u + (k4 % 32u);
#pragma unroll
        for (int l = 0; l < 4; ++l) *reinterpret_cast<uint32_t*>(xl + base + 32u * l) = packed[l];
    }
}

// Top-k of one token by one wave. Lane l holds experts l, l + 64, ... (PER of them, in
// registers). Learned routing ranks score + bias with the reference's float keys; softmax
// ranks float64 probabilities. Returns true when the token cannot be routed (non-finite logits
// or a non-positive weight sum).
template <int PER>
__device__ bool route_token(const float* lg, const float* bias, uint32_t E, uint32_t K,
                            bool softmax, const MoeShape& s, uint32_t* out_idx, float* out_w) {
    const int lane = threadIdx.x & 63;
    double key[PER];
    float sc[PER];
    bool taken[PER];
    bool bad = false;
    double mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const uint32_t e = lane + 64u * i;
        taken[i] = e >= E;
        sc[i] = 0.0f;
        key[i] = -INFINITY;
        if (e < E) {
            const float l = lg[e];
            bad |= !isfinite(l);
            if (!softmax) {
                sc[i] = score_of(l, s.score_fn);
                key[i] = (double)(sc[i] + (bias ? bias[e] : 0.0f));
            } else {
                mx = fmax(mx, (double)l);
            }
        }
    }
    if (softmax) {
        for (int o = 32; o > 0; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o));
        double sum = 0.0;
#pragma unroll
        for (int i = 0; i < PER; ++i)
            if (lane + 64u * i < E) {
                key[i] = exp((double)lg[lane + 64u * i] - mx);
                sum += key[i];
            }
        sum = wave_sum_f64(sum);
        const double inv = sum > 0.0 ? 1.0 / sum : 0.0;
#pragma unroll
        for (int i = 0; i < PER; ++i)
            if (lane + 64u * i < E) key[i] = key[i] * inv;
    }
    double sel_sum = 0.0;
    for (uint32_t k = 0; k < K; ++k) {
        double bk = -INFINITY;
        uint32_t bi = 0xffffffffu;
        float bs = 0.0f;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const uint32_t e = lane + 64u * i;
            if (!taken[i] && (bi == 0xffffffffu || beats_d(key[i], e, bk, bi))) {
                bk = key[i];
                bi = e;
                bs = sc[i];
            }
        }
        for (int o = 32; o > 0; o >>= 1) {
            const double ok = __shfl_xor(bk, o);
            const uint32_t oi = __shfl_xor(bi, o);
            const float os = __shfl_xor(bs, o);
            if (oi != 0xffffffffu && (bi == 0xffffffffu || beats_d(ok, oi, bk, bi))) {
                bk = ok;
                bi = oi;
                bs = os;
            }
        }
#pragma unroll
        for (int i = 0; i < PER; ++i)
            if (lane + 64u * i == bi) taken[i] = true;
        if (bi >= E) bad = true;
        const double v = softmax ? bk : (double)bs;
        if (lane == 0) {
            out_idx[k] = bi < E ? bi : 0u;
            out_w[k] = softmax ? (float)bk : bs;
        }
        sel_sum += v;
    }
    if (lane == 0) {
        if (!softmax) {
            bad |= !(sel_sum > 0.0) || isinf(sel_sum);
            for (uint32_t k = 0; k < K; ++k)
                out_w[k] = (float)((double)out_w[k] / sel_sum * (double)s.route_scale);
        } else if (s.renormalize && sel_sum > 0.0) {
            const double scale = 1.0 / sel_sum;
            for (uint32_t k = 0; k < K; ++k) out_w[k] = (float)((double)out_w[k] * scale);
        }
    }
    return __any(bad);
}

__global__ void __launch_bounds__(512) k_moe_route(const MoeShape s, const MoeInputs in,
                                                   const MoeWorkspace w) {
    __shared__ uint32_t s_idx[kMoeMaxTokens * kMoeMaxTopK];
    __shared__ float s_w[kMoeMaxTokens * kMoeMaxTopK];
    __shared__ uint32_t s_bad;
    MoeHeader* hdr = ws_ptr<MoeHeader>(w, w.off_header);
    const float* logits = ws_ptr<float>(w, w.off_logits);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t K = s.top_k, E = s.experts;
    if (threadIdx.x == 0) s_bad = 0;
    __syncthreads();

    // Phase A: one wave per token.
    if (wave < (int)s.tokens) {
        const uint32_t t = wave;
        const float* lg = logits + (uint64_t)t * E;
        if (s.routing == kRouteGiven || s.routing == kRouteTable) {
            for (uint32_t k = lane; k < K; k += 64) {
                uint32_t id = 0;
                if (s.routing == kRouteGiven) id = in.given_ids ? in.given_ids[t * K + k] : 0u;
                else id = in.table_ids[t * K + k];
                if (id >= E) { atomicOr(&s_bad, 1u); id = 0; }
                s_idx[t * K + k] = id;
            }
            __builtin_amdgcn_wave_barrier();
            // Duplicate experts within one token are refused.
            for (uint32_t k = lane; k < K; k += 64)
                for (uint32_t j = 0; j < k; ++j)
                    if (s_idx[t * K + j] == s_idx[t * K + k]) atomicOr(&s_bad, 1u);
            if (s.routing == kRouteGiven) {
                for (uint32_t k = lane; k < K; k += 64)
                    s_w[t * K + k] = in.given_weights ? in.given_weights[t * K + k] : 1.0f;
            } else if (lane == 0) {
                double sum = 0.0;
                float sc[kMoeMaxTopK];
                for (uint32_t k = 0; k < K; ++k) {
                    sc[k] = score_of(lg[s_idx[t * K + k]], s.score_fn);
                    sum += (double)sc[k];
                }
                if (!(sum > 0.0) || isinf(sum)) atomicOr(&s_bad, 1u);
                for (uint32_t k = 0; k < K; ++k)
                    s_w[t * K + k] = (float)((double)sc[k] / sum * (double)s.route_scale);
            }
        } else {
            const float* bias = s.routing == kRouteLearned ? in.bias : nullptr;
            const bool softmax = s.routing == kRouteSoftmax;
            float* sw = s_w + t * K;
            uint32_t* si = s_idx + t * K;
            bool bad = false;
            if (E <= 64) bad = route_token<1>(lg, bias, E, K, softmax, s, si, sw);
            else if (E <= 128) bad = route_token<2>(lg, bias, E, K, softmax, s, si, sw);
            else if (E <= 256) bad = route_token<4>(lg, bias, E, K, softmax, s, si, sw);
            else if (E <= 512) bad = route_token<8>(lg, bias, E, K, softmax, s, si, sw);
            else bad = route_token<16>(lg, bias, E, K, softmax, s, si, sw);
            if (bad && lane == 0) atomicOr(&s_bad, 1u);
        }
    }
    __syncthreads();

    // Phase B: the active-expert list. Distinct experts are numbered in ascending id by a
    // prefix count over per-expert "used" flags; each (token, slot) pair then finds its expert's
    // active index, its slot among that expert's tokens (ascending token), and its place in the
    // token's combine order.
    const uint32_t P = s.tokens * K;
    ActiveExpert* act = ws_ptr<ActiveExpert>(w, w.off_active);
    CombineEntry* comb = ws_ptr<CombineEntry>(w, w.off_combine);
    uint32_t* ridx = ws_ptr<uint32_t>(w, w.off_route_idx);
    float* rw = ws_ptr<float>(w, w.off_route_w);
    __shared__ uint32_t s_used[1024];
    __shared__ uint32_t s_wave_count[8];
    for (uint32_t e = threadIdx.x; e < 1024; e += blockDim.x) s_used[e] = 0;
    __syncthreads();
    if (threadIdx.x < P) s_used[s_idx[threadIdx.x]] = 1;
    __syncthreads();
    // Exclusive prefix over 1024 flags: wave v owns experts [128v, 128v + 128).
    const uint32_t e0 = 128u * wave + lane, e1 = e0 + 64u;
    const uint64_t m0 = __ballot(s_used[e0] != 0), m1 = __ballot(s_used[e1] != 0);
    const uint64_t below = (1ull << lane) - 1ull;
    if (lane == 0) s_wave_count[wave] = (uint32_t)(__popcll(m0) + __popcll(m1));
    __syncthreads();
    uint32_t base = 0, n_routed = 0;
    for (int v = 0; v < 8; ++v) {
        if (v < wave) base += s_wave_count[v];
        n_routed += s_wave_count[v];
    }
    const uint32_t pre0 = base + (uint32_t)__popcll(m0 & below);
    const uint32_t pre1 = base + (uint32_t)__popcll(m0) + (uint32_t)__popcll(m1 & below);
    __syncthreads();
    s_used[e0] = pre0;
    s_used[e1] = pre1;
    __syncthreads();
    const uint32_t p = threadIdx.x;
    if (p < P) {
        const uint32_t e = s_idx[p], t = p / K, k = p % K;
        const float wt = s_w[p];
        ridx[p] = e;
        rw[p] = wt;
        const uint32_t a = s_used[e];
        uint32_t slot = 0, ntok = 0, pos = 0;
        for (uint32_t q = 0; q < P; ++q) {
            if (s_idx[q] == e) {
                ++ntok;
                if (q < p) ++slot;
            }
        }
        for (uint32_t j = 0; j < K; ++j) pos += s_idx[t * K + j] < e ? 1u : 0u;
        act[a].tok[slot] = t;
        act[a].route_w[slot] = wt;
        if (slot == 0) {
            act[a].expert = e;
            act[a].ntok = ntok;
            act[a].apply_w = s.semantics == kSemDeepseek ? 1u : 0u;
            act[a].limit = s.routed_limit;
        }
        const uint32_t at = s.semantics == kSemDeepseek ? pos : k;
        comb[t * (K + 1) + at] = CombineEntry{(a << 3) | slot, s.semantics == kSemQwen ? wt : 1.0f};
    }
    if (threadIdx.x == 0) {
        if (s.has_shared) {
            ActiveExpert& sh = act[n_routed];
            sh.expert = E;
            sh.ntok = s.tokens;
            sh.apply_w = 0;
            sh.limit = s.shared_limit;
            for (uint32_t t = 0; t < s.tokens; ++t) {
                sh.tok[t] = t;
                sh.route_w[t] = 1.0f;
                comb[t * (K + 1) + K] = CombineEntry{(n_routed << 3) | t, 1.0f};
            }
        }
        hdr->n_active = s_bad ? 0u : n_routed + (s.has_shared ? 1u : 0u);
        if (s_bad) atomicOr(&hdr->status, kStatusBadRoute);
    }
    // The tokens' activations as MFMA limbs.
    __shared__ float s_red[16];
    for (uint32_t t = 0; t < s.tokens; ++t)
        prep_token_block(in.x + (uint64_t)t * s.width, s.width, limb_slots(s.tokens), t,
                         ws_ptr<int8_t>(w, w.off_xlimbs), ws_ptr<int>(w, w.off_xexp),
                         &hdr->status, s_red);
}

// ------------------------------------------------------------------------------------------
// Expert projections.
// ------------------------------------------------------------------------------------------

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

// Gate and up projections of one active expert over two 32-row tiles, then the SwiGLU.
// Eight waves: wave w takes tile 2*blockIdx.x + w/4, matrix w%2 (gate, up) and half (w/2)%2 of
// the columns; the two halves are added in order. Two tiles per block let the grid fit the
// GPU in one round and halve the activation staging per row.
template <uint32_t FMT, int NT, bool LDS_A>
__global__ void __launch_bounds__(512) k_moe_gateup(const MoeShape s, const MoeInputs in,
                                                    const MoeWorkspace w) {
    __shared__ LdsTables lds;
    __shared__ float partial[2][2][2][NT][32];  // [tile][matrix][half][slot][row]
    extern __shared__ __align__(16) int8_t dyn_lds[];
    __shared__ __align__(16) int8_t s_zero[16];
    const MoeHeader* hdr = ws_ptr<MoeHeader>(w, w.off_header);
    const uint32_t a = blockIdx.y;
    if (a >= hdr->n_active) return;
    const ActiveExpert* aep = ws_ptr<ActiveExpert>(w, w.off_active) + a;
    const uint32_t ntok = aep->ntok;
    vl_tiled_layout L;
    vl_make_layout(FMT, s.inter, s.width, &L);

    constexpr int S = Acc<NT>::kSlots;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tw = wave >> 2, mat = wave & 1, half = (wave >> 1) & 1;
    const uint32_t t = 2u * blockIdx.x + tw;
    const bool tile_on = t < L.tiles;
    const uint32_t n = lane & 31;
    const int hh = lane >> 5;
    const MoeExpert ex = in.experts[aep->expert];
    const uint8_t* W = mat == 0 ? ex.gate : ex.up;
    const uint32_t chunks = chunks_of<FMT>(L);
    const uint32_t c0 = tile_on ? chunks * half / 2u : 0u;
    const uint32_t c1 = tile_on ? chunks * (half + 1) / 2u : 0u;
    const uint32_t xslots = limb_slots(s.tokens);
    const int slot = a_slot_of_lane();
    const bool on = slot < (int)ntok;
    const int8_t* xl = ws_ptr<int8_t>(w, w.off_xlimbs);
    const uint32_t limb_off = (uint32_t)a_limb_of_lane() * 32u + 16u * hh;
    float accf[S];
    tile_partial<FMT, NT>(L, W, tile_on ? t : 0u, c0, c1, (LDS_A ? NT : xslots) * 128u, lds, accf,
                          [&](uint32_t& stride) -> const int8_t* {
        load_tables<FMT>(lds);
        if (threadIdx.x < 4) reinterpret_cast<uint32_t*>(s_zero)[threadIdx.x] = 0;
        if (LDS_A) stage_limbs<NT>(dyn_lds, xl, L.groups, xslots, ntok,
                                   [&](uint32_t sl) { return aep->tok[sl]; });
        __syncthreads();
        if (!on) {
            stride = 0;
            return s_zero;
        }
        return LDS_A ? dyn_lds + (uint32_t)slot * 128u + limb_off
                     : xl + (uint64_t)aep->tok[slot] * 128u + limb_off;
    });
#pragma unroll
    for (int i = 0; i < S; ++i) {
        const int sl = 2 * i + hh;
        if (sl < NT) partial[tw][mat][half][sl][n] = accf[i];
    }
    __syncthreads();
    for (uint32_t idx = threadIdx.x; idx < 2u * NT * 32u; idx += blockDim.x) {
        const uint32_t tt = idx / (NT * 32u), sl = (idx / 32u) % NT, r = idx % 32u;
        const uint32_t row = (2u * blockIdx.x + tt) * 32u + r;
        if (sl < ntok && row < s.inter) {
            const int e = ws_ptr<int>(w, w.off_xexp)[aep->tok[sl]];
            const float g = ldexpf(partial[tt][0][0][sl][r] + partial[tt][0][1][sl][r], -e);
            const float u = ldexpf(partial[tt][1][0][sl][r] + partial[tt][1][1][sl][r], -e);
            const float h = swiglu(s.semantics, g, u, aep->limit, aep->apply_w != 0, aep->route_w[sl]);
            MoeHeader* hw = ws_ptr<MoeHeader>(w, w.off_header);
            if (!isfinite(g) || !isfinite(u) || !isfinite(h)) atomicOr(&hw->status, kStatusNonFiniteOutput);
            ws_ptr<float>(w, w.off_h)[((uint64_t)a * kMoeMaxTokens + sl) * s.inter + row] = h;
            atomicMax(ws_ptr<uint32_t>(w, w.off_hmax) + a * kMoeMaxTokens + sl,
                      __float_as_uint(isfinite(h) ? fabsf(h) : 0.0f));
        }
    }
}

// h of (active expert, token) -> limbs, layout [a][group][8 slots][4][32].
__global__ void __launch_bounds__(256) k_moe_hprep(const MoeShape s, const MoeWorkspace w) {
    const MoeHeader* hdr = ws_ptr<MoeHeader>(w, w.off_header);
    const uint32_t sl = blockIdx.x, a = blockIdx.y;
    if (a >= hdr->n_active) return;
    const ActiveExpert* act = ws_ptr<ActiveExpert>(w, w.off_active);
    if (sl >= act[a].ntok) return;
    const float m = __uint_as_float(ws_ptr<uint32_t>(w, w.off_hmax)[a * kMoeMaxTokens + sl]);
    int q = 0;
    frexpf(m, &q);
    const int e = m > 0.0f ? 30 - q : 0;
    if (threadIdx.x == 0) ws_ptr<int>(w, w.off_hexp)[a * kMoeMaxTokens + sl] = e;
    const float* h = ws_ptr<float>(w, w.off_h) + ((uint64_t)a * kMoeMaxTokens + sl) * s.inter;
    int8_t* out = ws_ptr<int8_t>(w, w.off_hlimbs) + (uint64_t)a * (s.inter / 32u) * kMoeMaxTokens * 128u;
    for (uint32_t k4 = threadIdx.x * 4u; k4 < s.inter; k4 += blockDim.x * 4u) {
        uint32_t packed[4] = {0, 0, 0, 0};
        for (int i = 0; i < 4; ++i) {
            const float v = h[k4 + i];
            int X = isfinite(v) ? (int)rintf(ldexpf(v, e)) : 0;
            for (int l = 0; l < 4; ++l) {
                const int digit = l < 3 ? (int)(int8_t)(X & 0xff) : X;
                packed[l] |= ((uint32_t)digit & 0xffu) << (8 * i);
                X = (X - digit) >> 8;
            }
        }
        const uint64_t base = ((uint64_t)(k4 / 32u) * kMoeMaxTokens + sl) * 128u + (k4 % 32u);
        for (int l = 0; l < 4; ++l) *reinterpret_cast<uint32_t*>(out + base + 32u * l) = packed[l];
    }
}

// Down projection of one active expert over four 32-row tiles: wave w takes tile
// 4*blockIdx.x + w/2 and half w%2 of the columns. The block stages the expert's activation
// limbs once for its 128 rows.
template <uint32_t FMT, int NT, bool LDS_A>
__global__ void __launch_bounds__(512) k_moe_down(const MoeShape s, const MoeInputs in,
                                                  const MoeWorkspace w) {
    __shared__ LdsTables lds;
    __shared__ float partial[4][2][NT][32];  // [tile][half][slot][row]
    extern __shared__ __align__(16) int8_t dyn_lds[];
    __shared__ __align__(16) int8_t s_zero[16];
    const MoeHeader* hdr = ws_ptr<MoeHeader>(w, w.off_header);
    const uint32_t a = blockIdx.y;
    if (a >= hdr->n_active) return;
    const ActiveExpert* act = ws_ptr<ActiveExpert>(w, w.off_active);
    const uint32_t ntok = act[a].ntok;
    vl_tiled_layout L;
    vl_make_layout(FMT, s.width, s.inter, &L);

    constexpr int S = Acc<NT>::kSlots;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tw = wave >> 1, half = wave & 1;
    const uint32_t t = 4u * blockIdx.x + tw;
    const bool tile_on = t < L.tiles;
    const uint32_t n = lane & 31;
    const int hh = lane >> 5;
    const uint8_t* W = in.experts[act[a].expert].down;
    const uint32_t chunks = chunks_of<FMT>(L);
    const uint32_t c0 = tile_on ? chunks * half / 2u : 0u;
    const uint32_t c1 = tile_on ? chunks * (half + 1) / 2u : 0u;
    const int slot = a_slot_of_lane();
    const bool on = slot < (int)ntok;
    const int8_t* hl = ws_ptr<int8_t>(w, w.off_hlimbs) + (uint64_t)a * (s.inter / 32u) * kMoeMaxTokens * 128u;
    const uint32_t lane_off = ((uint32_t)slot * 4u + a_limb_of_lane()) * 32u + 16u * hh;
    float accf[S];
    tile_partial<FMT, NT>(L, W, tile_on ? t : 0u, c0, c1, (LDS_A ? NT : kMoeMaxTokens) * 128u, lds,
                          accf, [&](uint32_t& stride) -> const int8_t* {
        load_tables<FMT>(lds);
        if (threadIdx.x < 4) reinterpret_cast<uint32_t*>(s_zero)[threadIdx.x] = 0;
        if (LDS_A) stage_limbs<NT>(dyn_lds, hl, L.groups, kMoeMaxTokens, ntok,
                                   [](uint32_t sl) { return sl; });
        __syncthreads();
        if (!on) {
            stride = 0;
            return s_zero;
        }
        return LDS_A ? dyn_lds + lane_off : hl + lane_off;
    });
#pragma unroll
    for (int i = 0; i < S; ++i) {
        const int sl = 2 * i + hh;
        if (sl < NT) partial[tw][half][sl][n] = accf[i];
    }
    __syncthreads();
    for (uint32_t idx = threadIdx.x; idx < 4u * NT * 32u; idx += blockDim.x) {
        const uint32_t tt = idx / (NT * 32u), sl = (idx / 32u) % NT, r = idx % 32u;
        const uint32_t row = (4u * blockIdx.x + tt) * 32u + r;
        if (sl < ntok && row < s.width) {
            const int e = ws_ptr<int>(w, w.off_hexp)[a * kMoeMaxTokens + sl];
            const float y = ldexpf(partial[tt][0][sl][r] + partial[tt][1][sl][r], -e);
            ws_ptr<float>(w, w.off_ypart)[((uint64_t)a * kMoeMaxTokens + sl) * s.width + row] = y;
        }
    }
}

__global__ void __launch_bounds__(256) k_moe_combine(const MoeShape s, const MoeInputs in,
                                                     const MoeWorkspace w) {
    MoeHeader* hdr = ws_ptr<MoeHeader>(w, w.off_header);
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)s.tokens * s.width) return;
    const uint32_t t = (uint32_t)(i / s.width), c = (uint32_t)(i % s.width);
    if (hdr->n_active == 0) {
        in.out[i] = 0.0f;
        return;
    }
    const CombineEntry* comb = ws_ptr<CombineEntry>(w, w.off_combine) + (uint64_t)t * (s.top_k + 1u);
    const float* yp = ws_ptr<float>(w, w.off_ypart);
    const uint32_t n = s.top_k + (s.has_shared ? 1u : 0u);
    // All loads first (independent), then the additions in the combine order.
    float y[kMoeMaxTopK + 1];
    float wt[kMoeMaxTopK + 1];
#pragma unroll
    for (uint32_t k = 0; k < kMoeMaxTopK + 1; ++k) {
        if (k < n) {
            const CombineEntry ce = comb[k];
            wt[k] = ce.w;
            y[k] = yp[((uint64_t)(ce.src >> 3) * kMoeMaxTokens + (ce.src & 7u)) * s.width + c];
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < kMoeMaxTopK + 1; ++k) {
        if (k < n)
            acc = (s.semantics == kSemQwen && k < s.top_k) ? __fadd_rn(acc, __fmul_rn(y[k], wt[k]))
                                                           : __fadd_rn(acc, y[k]);
    }
    if (!isfinite(acc)) atomicOr(&hdr->status, kStatusNonFiniteOutput);
    in.out[i] = acc;
}

// ------------------------------------------------------------------------------------------
// Launch sequence.
// ------------------------------------------------------------------------------------------

template <uint32_t FMT>
static void launch_gateup_fmt(uint32_t slots, dim3 grid, const MoeShape& s, const MoeInputs& in,
                              const MoeWorkspace& w, hipStream_t st) {
    const uint32_t bytes = s.width / 32u * slots * 128u;
    const bool lds_a = bytes <= kMaxLdsLimbBytes;
    const uint32_t shm = lds_a ? bytes : 0u;
    const dim3 blk(512);
    switch (slots * 2 + (lds_a ? 1 : 0)) {
        case 2: hipLaunchKernelGGL((k_moe_gateup<FMT, 1, false>), grid, blk, shm, st, s, in, w); break;
        case 3: hipLaunchKernelGGL((k_moe_gateup<FMT, 1, true>), grid, blk, shm, st, s, in, w); break;
        case 4: hipLaunchKernelGGL((k_moe_gateup<FMT, 2, false>), grid, blk, shm, st, s, in, w); break;
        case 5: hipLaunchKernelGGL((k_moe_gateup<FMT, 2, true>), grid, blk, shm, st, s, in, w); break;
        case 8: hipLaunchKernelGGL((k_moe_gateup<FMT, 4, false>), grid, blk, shm, st, s, in, w); break;
        case 9: hipLaunchKernelGGL((k_moe_gateup<FMT, 4, true>), grid, blk, shm, st, s, in, w); break;
        case 16: hipLaunchKernelGGL((k_moe_gateup<FMT, 8, false>), grid, blk, shm, st, s, in, w); break;
        default: hipLaunchKernelGGL((k_moe_gateup<FMT, 8, true>), grid, blk, shm, st, s, in, w); break;
    }
}

template <uint32_t FMT>
static void launch_down_fmt(uint32_t slots, dim3 grid, const MoeShape& s, const MoeInputs& in,
                            const MoeWorkspace& w, hipStream_t st) {
    const uint32_t bytes = s.inter / 32u * slots * 128u;
    const bool lds_a = bytes <= kMaxLdsLimbBytes;
    const uint32_t shm = lds_a ? bytes : 0u;
    const dim3 blk(512);
    switch (slots * 2 + (lds_a ? 1 : 0)) {
        case 2: hipLaunchKernelGGL((k_moe_down<FMT, 1, false>), grid, blk, shm, st, s, in, w); break;
        case 3: hipLaunchKernelGGL((k_moe_down<FMT, 1, true>), grid, blk, shm, st, s, in, w); break;
        case 4: hipLaunchKernelGGL((k_moe_down<FMT, 2, false>), grid, blk, shm, st, s, in, w); break;
        case 5: hipLaunchKernelGGL((k_moe_down<FMT, 2, true>), grid, blk, shm, st, s, in, w); break;
        case 8: hipLaunchKernelGGL((k_moe_down<FMT, 4, false>), grid, blk, shm, st, s, in, w); break;
        case 9: hipLaunchKernelGGL((k_moe_down<FMT, 4, true>), grid, blk, shm, st, s, in, w); break;
        case 16: hipLaunchKernelGGL((k_moe_down<FMT, 8, false>), grid, blk, shm, st, s, in, w); break;
        default: hipLaunchKernelGGL((k_moe_down<FMT, 8, true>), grid, blk, shm, st, s, in, w); break;
    }
}

hipError_t launch_moe(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                      hipStream_t st, hipEvent_t* ev) {
    if (!moe_shape_ok(s)) return hipErrorInvalidValue;
    const uint32_t slots = limb_slots(s.tokens);
    auto mark = [&](uint32_t stage) {
        if (ev) (void)hipEventRecord(ev[stage], st);
    };
    mark(kStageRouter);
    hipLaunchKernelGGL(k_moe_router, dim3(s.routing == kRouteGiven ? 1u : s.experts), dim3(256), 0, st, s, in, w);
    mark(kStageRoute);
    hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(512), 0, st, s, in, w);
    mark(kStagePrep);
    mark(kStageGateUp);
    const dim3 g_gu((s.inter + 63) / 64, w.max_active);
    switch (s.gate_type) {
        case VL_TYPE_IQ2_XXS: launch_gateup_fmt<VL_TYPE_IQ2_XXS>(slots, g_gu, s, in, w, st); break;
        case VL_TYPE_IQ3_XXS: launch_gateup_fmt<VL_TYPE_IQ3_XXS>(slots, g_gu, s, in, w, st); break;
        case VL_TYPE_IQ1_S: launch_gateup_fmt<VL_TYPE_IQ1_S>(slots, g_gu, s, in, w, st); break;
        case VL_TYPE_Q8_0: launch_gateup_fmt<VL_TYPE_Q8_0>(slots, g_gu, s, in, w, st); break;
        default: return hipErrorInvalidValue;
    }
    mark(kStageHPrep);
    hipLaunchKernelGGL(k_moe_hprep, dim3(kMoeMaxTokens, w.max_active), dim3(256), 0, st, s, w);
    mark(kStageDown);
    const dim3 g_dn((s.width + 127) / 128, w.max_active);
    switch (s.down_type) {
        case VL_TYPE_IQ2_XXS: launch_down_fmt<VL_TYPE_IQ2_XXS>(slots, g_dn, s, in, w, st); break;
        case VL_TYPE_IQ3_XXS: launch_down_fmt<VL_TYPE_IQ3_XXS>(slots, g_dn, s, in, w, st); break;
        case VL_TYPE_IQ1_S: launch_down_fmt<VL_TYPE_IQ1_S>(slots, g_dn, s, in, w, st); break;
        case VL_TYPE_Q8_0: launch_down_fmt<VL_TYPE_Q8_0>(slots, g_dn, s, in, w, st); break;
        default: return hipErrorInvalidValue;
    }
    mark(kStageCombine);
    const uint64_t total = (uint64_t)s.tokens * s.width;
    hipLaunchKernelGGL(k_moe_combine, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, st, s, in, w);
    mark(kStageCount);
    return hipGetLastError();
}

}  // namespace vl
