// MoE layer on the device, for up to 8 tokens routed to top-k of E experts plus a shared expert,
// in three launches:
//
//   k_moe_router   gate logits (float64 accumulation per expert row, the reference's linear_f /
//                  gate_logits numerics); the tokens' int8 limbs with one exponent per 256
//                  columns; the per-call status word and handoff counters zeroed
//   k_moe_gateup   persistent: every block first routes (per-token scores and top-k, then the
//                  active-expert list: distinct experts in ascending id with their tokens, and
//                  each token's combine order; block 0 publishes it), then its waves stream the
//                  gate and up tiles of all active experts (vl_stream.h). The last wave of a tile
//                  adds its partials, applies the SwiGLU of the semantics and stores h; the last
//                  tile of each 256-row block of h turns it into limbs for the down projection
//   k_moe_down     persistent: the waves stream the down tiles of all active experts; the last
//                  wave of a tile stores the expert's rows, and the last expert of a tile combines
//                  the layer output rows in the reference's combine order
//
// The routing, clamp, route-weight placement and combine order follow the reference code named
// in vl_moe.h. Every reduction has a fixed order, so results are deterministic.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <mutex>

#include "vl_kernels.h"
#include "vl_moe.h"
#include "vl_moe_dev.h"
#include "vl_moe_token.h"
#include "vl_moe_wide.h"
#include "vl_stream.h"

namespace vl {

static inline uint64_t align256(uint64_t v) { return (v + 255u) & ~uint64_t(255); }

// Groups of the grouped path, at most: each selected expert's tokens in groups of
// kMoeMaxTokens (a partial group per expert at most), then the shared expert's.
static uint64_t max_groups(const MoeShape& s) {
    const uint64_t assign = (uint64_t)s.tokens * s.top_k;
    const uint64_t used = assign < s.experts ? assign : s.experts;
    return assign / kMoeMaxTokens + used + (s.has_shared ? (s.tokens + kMoeMaxTokens - 1u) / kMoeMaxTokens : 0u);
}

bool moe_shape_ok(const MoeShape& s) {
    uint32_t be = 0, bb = 0;
    if (s.tokens == 0 || s.tokens > kMoeMaxTokensGrouped || s.top_k == 0 || s.top_k > kMoeMaxTopK ||
        s.experts == 0 || s.experts > 1024 || s.top_k > s.experts)
        return false;
    if (s.tokens > kMoeMaxTokens &&
        ((uint64_t)s.tokens * s.top_k > kMoeMaxGroupAssign || max_groups(s) > kMoeMaxGroups))
        return false;
    // GGUF-layout down matrices take any gate/up type; GGUF-layout gate/up matrices need a
    // GGUF-layout down (the tiled down stage reads the h magnitudes the tiled gate/up forms).
    if (!vl_type_tiled(s.gate_type) && vl_type_tiled(s.down_type)) return false;
    if (!vl_block_shape(s.gate_type, &be, &bb) || s.width % be || s.width % 256u) return false;
    if (!vl_block_shape(s.down_type, &be, &bb) || s.inter % be || s.inter % 32u) return false;
    if (s.semantics > kSemPlain || s.routing > kRouteGiven || s.score_fn > kScoreSigmoid) return false;
    // Learned and table routes scale their weights by route_scale, which the reference requires
    // to be finite and positive (route_from_indices, deepseek_v4_reference.cpp:80-90).
    const bool scaled = s.routing == kRouteLearned || s.routing == kRouteTable;
    if (scaled && !(std::isfinite(s.route_scale) && s.route_scale > 0.0f)) return false;
    return true;
}

static uint32_t max_active(const MoeShape& s) {
    const uint32_t routed = s.tokens * s.top_k < s.experts ? s.tokens * s.top_k : s.experts;
    return routed + (s.has_shared ? 1u : 0u);
}

// Router logits of grouped layers as a tiled product: kLgT tokens x kLgE experts per block,
// kLgK columns staged per step.
constexpr uint32_t kLgT = 64, kLgE = 64, kLgK = 32;

// Column slices of the grouped router product: about two blocks per persistent block, at least
// one k-step each, and at most 2^21 partial sums in all.
static uint32_t router_slices(const MoeShape& s, uint32_t blocks) {
    const uint64_t tiles = (uint64_t)((s.experts + kLgE - 1u) / kLgE) * ((s.tokens + kLgT - 1u) / kLgT);
    uint64_t n = (2u * (uint64_t)blocks + tiles - 1u) / tiles;
    const uint64_t steps = s.width / kLgK, cap = (1ull << 21) / ((uint64_t)s.tokens * s.experts);
    if (n > steps) n = steps;
    if (n > cap) n = cap;
    return n ? (uint32_t)n : 1u;
}

MoeWorkspace moe_workspace_layout(const MoeShape& s, uint32_t blocks, void* base) {
    MoeWorkspace w{};
    w.base = static_cast<uint8_t*>(base);
    // GGUF-layout matrices run on the grouped layer's plan at every token count.
    w.grouped = s.tokens > kMoeMaxTokens || !vl_type_tiled(s.gate_type) || !vl_type_tiled(s.down_type) ? 1u : 0u;
    w.wide = w.grouped && wide_shape_ok(s) ? 1u : 0u;
    w.max_active = w.grouped ? (uint32_t)max_groups(s) : max_active(s);
    w.max_items = w.wide ? w.max_active : 0u;
    w.slots = w.grouped ? kMoeMaxTokens : limb_slots(s.tokens);
    w.xslots = w.grouped ? s.tokens : w.slots;
    w.estride = w.grouped ? s.tokens : 8u;
    w.blocks = blocks;
    w.waves = blocks * kStreamWaves;
    w.tiles_gu = (s.inter + 31u) / 32u;
    w.tiles_dn = (s.width + 31u) / 32u;
    w.hblocks = exp_blocks(s.inter);
    w.xblocks = exp_blocks(s.width);
    const uint64_t A = w.max_active, T = s.tokens, K = s.top_k, NT = w.slots;
    // Most experts the units of one down block can touch, for any number of active experts.
    const uint64_t UJ = units_per_row(s.down_type, s.inter);
    const uint64_t per_block = blocks ? (A * w.tiles_dn * UJ + blocks - 1u) / blocks : 1u;
    const uint64_t stage = (per_block > 0 ? per_block - 1u : 0u) / (w.tiles_dn * UJ) + 2u;
    w.stage = (uint32_t)(stage < A ? stage : A);
    // The fp16 kernels use neither the hand-off counters and records nor the int8 limbs.
    const uint64_t limbs = w.wide ? 0u : 1u;
    w.counters = (uint32_t)(limbs * (A * w.tiles_gu + A * w.tiles_dn + w.tiles_dn + A * w.hblocks * 8u));
    uint64_t o = 0;
    w.off_header = o; o = align256(o + sizeof(MoeHeader));
    w.off_logits = o; o = align256(o + T * s.experts * 4u);
    w.off_scores = o; o = align256(o + T * s.experts * 4u);
    w.off_keys = o; o = align256(o + T * s.experts * 4u);
    w.off_route_idx = o; o = align256(o + T * K * 4u);
    w.off_route_w = o; o = align256(o + T * K * 4u);
    w.off_active = o; o = align256(o + A * sizeof(ActiveExpert));
    w.off_combine = o; o = align256(o + T * (K + 1) * sizeof(CombineEntry));
    w.off_xexp = o; o = align256(o + (uint64_t)w.xblocks * w.estride * 4u);
    w.off_xflags = o; o = align256(o + (uint64_t)w.xblocks * w.estride * 4u);
    w.off_xlimbs = o; o = align256(o + limbs * (s.width / 32u) * w.xslots * 128u);
    w.off_counters = o; o = align256(o + (uint64_t)w.counters * 4u);
    w.off_rec_gu = o; o = align256(o + limbs * (w.waves + A * w.tiles_gu) * 2u * NT * 64u * 4u);
    w.off_rec_dn = o; o = align256(o + limbs * (w.waves + A * w.tiles_dn) * NT * 64u * 4u);
    w.off_h = o; o = align256(o + limbs * A * NT * s.inter * 4u);
    w.off_hslab = o; o = align256(o + limbs * blocks * w.stage * down_expert_bytes(s.inter, w.slots));
    const uint64_t wide = w.wide ? 1u : 0u;
    w.off_x16 = o; o = align256(o + wide * T * s.width * 4u);
    w.off_xsc = o; o = align256(o + wide * T * 4u);
    w.off_h16 = o; o = align256(o + wide * A * kMoeMaxTokens * s.inter * 4u);
    w.off_hsc = o; o = align256(o + wide * A * kMoeMaxTokens * w.hblocks * 4u);
    w.off_items = o; o = align256(o + wide * w.max_items * sizeof(WideItem));
    w.off_ypart = o; o = align256(o + A * NT * (uint64_t)s.width * 4u);
    w.off_gweights = o; o = align256(o + (w.grouped ? A * sizeof(MoeExpert) : 0u));
    // Grouped layers: f64 partial router logits of each column slice, [slice][token][expert].
    w.lg_slices = w.grouped ? router_slices(s, blocks) : 0u;
    w.off_lgpart = o; o = align256(o + (uint64_t)w.lg_slices * T * s.experts * 8u);
    // Single-token layers: the hand-off records of jobs split between blocks.
    w.off_trec = o; o = align256(o + tok_record_bytes(s, blocks));
    w.bytes = o;
    return w;
}

uint64_t moe_workspace_bytes(const MoeShape& s, uint32_t blocks) {
    return moe_workspace_layout(s, blocks, nullptr).bytes;
}

// ------------------------------------------------------------------------------------------
// Scores and selection keys.
// ------------------------------------------------------------------------------------------

// ------------------------------------------------------------------------------------------
// Router logits and activation limbs.
// ------------------------------------------------------------------------------------------

// Threads 0..255: the first 8 float4 of their share of expert row b (its first 8192 weights)
// and the same columns of token t0's activations, requested together and early by the caller,
// so that both arrive within one memory latency.
struct RouterRow {
    float4 wv[8];
    float4 xv[8];
    int nv;
};
__device__ __forceinline__ void router_row_load(const MoeShape& s, const MoeInputs& in, uint32_t b,
                                                uint32_t t0, RouterRow& rr) {
    const uint32_t r = threadIdx.x;
    const float4* row = reinterpret_cast<const float4*>(in.router + (uint64_t)b * s.width);
    const float4* xr = reinterpret_cast<const float4*>(in.x + (uint64_t)t0 * s.width);
    const uint32_t n4 = s.width / 4u;
    rr.nv = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t i = r + 256u * j;
        if (i < n4) {
            rr.wv[j] = row[i];
            rr.xv[j] = xr[i];
            rr.nv = j + 1;
        }
    }
}

// Threads 0..255 of the block: partial sums of expert row b's logits for tokens [t0, t1) into
// red[t - t0][wave] (four waves take interleaved quarters of the row with every lane's float4
// loads in flight).
__device__ __forceinline__ void router_row_partials(const MoeShape& s, const MoeInputs& in, uint32_t b,
                                                    uint32_t t0, uint32_t t1, double (*red)[4],
                                                    const RouterRow& rr) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t r = threadIdx.x;
    const float4* row = reinterpret_cast<const float4*>(in.router + (uint64_t)b * s.width);
    const uint32_t n4 = s.width / 4u;
    const float4 (&wv)[8] = rr.wv;
    const int nv = rr.nv;
    for (uint32_t t = t0; t < t1; ++t) {
        const float4* xr = reinterpret_cast<const float4*>(in.x + (uint64_t)t * s.width);
        double acc = 0.0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j < nv) {
                const float4 a = wv[j], c = t == t0 ? rr.xv[j] : xr[r + 256u * j];
                acc += (double)a.x * (double)c.x;
                acc += (double)a.y * (double)c.y;
                acc += (double)a.z * (double)c.z;
                acc += (double)a.w * (double)c.w;
            }
        }
        // Rows wider than 8192 continue with plain loads.
        for (uint32_t i = r + 2048u; i < n4; i += 256u) {
            const float4 a = row[i], c = xr[i];
            acc += (double)a.x * (double)c.x;
            acc += (double)a.y * (double)c.y;
            acc += (double)a.z * (double)c.z;
            acc += (double)a.w * (double)c.w;
        }
        acc = wave_sum_f64(acc);
        if (lane == 0) red[t - t0][wave] = acc;
    }
}

// Token t's logit of expert b from the four partial sums (added in wave order), its score and
// its selection key: learned routing ranks score + bias (the reference's float keys), softmax
// routing ranks probabilities, which order as the logits do.
__device__ __forceinline__ void router_logit_store(const MoeShape& s, const MoeInputs& in,
                                                   const MoeWorkspace& w, uint32_t b, uint32_t t,
                                                   double sum) {
    const uint64_t i = (uint64_t)t * s.experts + b;
    const float logit = (float)sum;
    float score = 0.0f;
    uint32_t key;
    if (s.routing == kRouteSoftmax) {
        key = float_key(logit);
    } else {
        score = score_of(logit, s.score_fn);
        key = float_key(score + ((s.routing == kRouteLearned && in.bias) ? *gp(in.bias + b) : 0.0f));
    }
    // A non-finite logit refuses the token even where its score is finite (a sigmoid of +inf):
    // its key is the refusal key 1, like a non-finite score or selection bias.
    if (!isfinite(logit)) key = 1u;
    store_shared(ws_ptr<float>(w, w.off_logits) + i, logit);
    store_shared(ws_ptr<float>(w, w.off_scores) + i, score);
    store_shared_u32(ws_ptr<uint32_t>(w, w.off_keys) + i, key);
}
__device__ __forceinline__ void router_logit_finish(const MoeShape& s, const MoeInputs& in,
                                                    const MoeWorkspace& w, uint32_t b, uint32_t t,
                                                    const double (&red)[4]) {
    router_logit_store(s, in, w, b, t, ((red[0] + red[1]) + red[2]) + red[3]);
}

// Grouped layers: the router logits as a tiled product. Block (i, j, z) sums columns of slice z
// for tokens kLgT*j .. and experts kLgE*i ..; each thread holds 4 tokens x 4 experts of f64 sums,
// adding the exact f64 products of the f32 inputs column by column in ascending order. The next
// step's inputs are loaded while the current step is summed.
__global__ void __launch_bounds__(256) k_moe_logits_part(const MoeShape s, const MoeInputs in,
                                                         const MoeWorkspace w) {
    __shared__ __align__(16) float xs[kLgK][kLgT + 4];
    __shared__ __align__(16) float rs[kLgK][kLgE + 4];
    const uint32_t T = s.tokens, E = s.experts, H = s.width;
    const uint32_t e0 = blockIdx.x * kLgE, t0 = blockIdx.y * kLgT, z = blockIdx.z;
    const uint32_t steps = H / kLgK, S = w.lg_slices;
    const uint32_t k0 = (uint32_t)((uint64_t)z * steps / S), k1 = (uint32_t)((uint64_t)(z + 1u) * steps / S);
    const uint32_t tid = threadIdx.x, tx = tid % 16u, ty = tid / 16u;
    // Staging: 512 float4 per operand tile, two per thread: row q / 8, columns 4 (q % 8) ...
    float4 xv[2], rv[2];
    auto load = [&](uint32_t ks) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t q = tid + 256u * h, row = q / 8u, col = ks * kLgK + 4u * (q % 8u);
            xv[h] = t0 + row < T ? *reinterpret_cast<const float4*>(in.x + (uint64_t)(t0 + row) * H + col)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
            rv[h] = e0 + row < E ? *reinterpret_cast<const float4*>(in.router + (uint64_t)(e0 + row) * H + col)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    double acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
    if (k0 < k1) load(k0);
    for (uint32_t ks = k0; ks < k1; ++ks) {
        __syncthreads();  // the previous step's reads are done
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t q = tid + 256u * h, row = q / 8u, c = 4u * (q % 8u);
            xs[c][row] = xv[h].x; xs[c + 1][row] = xv[h].y; xs[c + 2][row] = xv[h].z; xs[c + 3][row] = xv[h].w;
            rs[c][row] = rv[h].x; rs[c + 1][row] = rv[h].y; rs[c + 2][row] = rv[h].z; rs[c + 3][row] = rv[h].w;
        }
        __syncthreads();
        if (ks + 1u < k1) load(ks + 1u);
#pragma unroll 8
        for (uint32_t k = 0; k < kLgK; ++k) {
            const float4 a = *reinterpret_cast<const float4*>(&xs[k][4u * ty]);
            const float4 b = *reinterpret_cast<const float4*>(&rs[k][4u * tx]);
            const double av[4] = {(double)a.x, (double)a.y, (double)a.z, (double)a.w};
            const double bv[4] = {(double)b.x, (double)b.y, (double)b.z, (double)b.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fma(av[i], bv[j], acc[i][j]);
        }
    }
    double* part = ws_ptr<double>(w, w.off_lgpart);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t t = t0 + 4u * ty + i;
        if (t >= T) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t e = e0 + 4u * tx + j;
            if (e < E) part[((uint64_t)z * T + t) * E + e] = acc[i][j];
        }
    }
}

// Grouped layers: each (token, expert) logit is the sum of its slices' partial sums in slice
// order, rounded to f32, with its score and selection key.
__global__ void __launch_bounds__(256) k_moe_logits_finish(const MoeShape s, const MoeInputs in,
                                                           const MoeWorkspace w) {
    const uint64_t n = (uint64_t)s.tokens * s.experts, i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const double* part = ws_ptr<const double>(w, w.off_lgpart);
    double sum = part[i];
    // Slices in order; the loads of 32 slices go out before the first of them is added.
    constexpr uint32_t kBatch = 32;
    uint32_t z = 1;
    for (; z + kBatch <= w.lg_slices; z += kBatch) {
        double v[kBatch];
#pragma unroll
        for (uint32_t k = 0; k < kBatch; ++k) v[k] = part[(uint64_t)(z + k) * n + i];
#pragma unroll
        for (uint32_t k = 0; k < kBatch; ++k) sum += v[k];
    }
    for (; z < w.lg_slices; ++z) sum += part[(uint64_t)z * n + i];
    router_logit_store(s, in, w, (uint32_t)(i % s.experts), (uint32_t)(i / s.experts), sum);
}

// Grouped layers with many column slices (few tokens): one wave per logit. Lane l adds slices
// l, l + 64, ... in order and the wave adds its 64 sums in a fixed butterfly order (lane 0's
// result is kept), rounded to f32, with its score and selection key.
__global__ void __launch_bounds__(256) k_moe_logits_finish_wave(const MoeShape s, const MoeInputs in,
                                                                const MoeWorkspace w) {
    const uint64_t n = (uint64_t)s.tokens * s.experts, i = (uint64_t)blockIdx.x * 4u + (threadIdx.x >> 6);
    if (i >= n) return;  // whole waves
    const uint32_t lane = threadIdx.x & 63u;
    const double* part = ws_ptr<const double>(w, w.off_lgpart);
    double sum = 0.0;
    for (uint32_t z = lane; z < w.lg_slices; z += 64u) sum += part[(uint64_t)z * n + i];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if (lane == 0) router_logit_store(s, in, w, (uint32_t)(i % s.experts), (uint32_t)(i / s.experts), sum);
}

// The router product's finishing launch: a wave per logit when there are 64 or more slices.
static hipError_t launch_logits_finish(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                                       hipStream_t st) {
    const uint64_t n = (uint64_t)s.tokens * s.experts;
    if (w.lg_slices >= 64u)
        hipLaunchKernelGGL(k_moe_logits_finish_wave, dim3((uint32_t)((n + 3u) / 4u)), dim3(256), 0, st, s, in, w);
    else
        hipLaunchKernelGGL(k_moe_logits_finish, dim3((uint32_t)((n + 255u) / 256u)), dim3(256), 0, st, s, in, w);
    return hipGetLastError();
}

// Blocks b < R (R = experts, or 0 for caller-given routes): expert row b's logits for the tokens
// of group g (tokens 8g .. 8g + 7). Blocks R + c: the limbs of column block c of the group's
// tokens, in blocks of their own so that no routing block waits for them. Block (0, 0) zeroes the
// status word; all blocks together zero the handoff counters.
__global__ void __launch_bounds__(256) k_moe_router(const MoeShape s, const MoeInputs in,
                                                    const MoeWorkspace w) {
    __shared__ double red[kMoeMaxTokens][4];
    const uint32_t b = blockIdx.x;
    const uint32_t t0 = blockIdx.y * kMoeMaxTokens;
    const uint32_t t1 = t0 + kMoeMaxTokens < s.tokens ? t0 + kMoeMaxTokens : s.tokens;
    // The row's weights are requested first; zeroing and the activation limbs overlap their
    // latency.
    RouterRow rr;
    const uint32_t R = s.routing != kRouteGiven ? s.experts : 0u;
    const bool routes = b < R;
    if (routes) router_row_load(s, in, b, t0, rr);
    if (b == 0 && blockIdx.y == 0 && threadIdx.x < 2) {
        MoeHeader* h = ws_ptr<MoeHeader>(w, w.off_header);
        (&h->status)[threadIdx.x] = 0;
    }
    {
        uint32_t* cnt = ws_ptr<uint32_t>(w, w.off_counters);
        const uint32_t nb = gridDim.x * gridDim.y, lb = blockIdx.y * gridDim.x + b;
        for (uint32_t i = lb * blockDim.x + threadIdx.x; i < w.counters; i += nb * blockDim.x) cnt[i] = 0;
    }
    if (!routes) {
        if (b - R < w.xblocks)
            prep_x_block(in.x, s.width, s.width, t0, t1, w.xslots, w.estride, b - R,
                         ws_ptr<int8_t>(w, w.off_xlimbs), ws_ptr<int>(w, w.off_xexp),
                         ws_ptr<uint32_t>(w, w.off_xflags));
        return;
    }
    router_row_partials(s, in, b, t0, t1, red, rr);
    __syncthreads();
    if (threadIdx.x < t1 - t0) router_logit_finish(s, in, w, b, t0 + threadIdx.x, red[threadIdx.x]);
}

// ------------------------------------------------------------------------------------------
// Routing (run by every gate/up block; block 0 publishes the result).
// ------------------------------------------------------------------------------------------

// Per-token selection scratch in LDS.
struct TopKLds {
    uint32_t id[kMoeMaxTopK];
    float val[kMoeMaxTopK];
    double p[kMoeMaxTopK];
};

// Top-k of one token by one wave (all lanes active). Lane l holds experts l, l + 64, ... (PER of
// them) with the selection keys of the router kernel, and first sorts them by key, descending,
// equal keys keeping ascending ids. Round k then takes the largest remaining key, ties to the
// lowest id: a DPP wave maximum over the lanes' heads, the head's lane (a wave minimum of ids
// only when several heads tie), and that lane drops its head. The experts thus come out in the
// reference's rank order; lanes k < K then form the weights with the reference's float64
// arithmetic, summing in rank order. Returns true when the token cannot be routed (non-finite
// logits or a non-positive weight sum).
template <int PER>
__device__ bool route_topk(const float* lg, const float* scr, const uint32_t* keys, uint32_t E,
                           uint32_t K, bool softmax, const MoeShape& s, TopKLds& tk,
                           uint32_t* out_idx, float* out_w, bool coherent) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t key[PER];
    float lv[PER], sv[PER];
    bool bad = false;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const uint32_t e = lane + 64u * i;
        key[i] = 0;
        lv[i] = sv[i] = 0.0f;
        if (e < E) {
            key[i] = coherent ? load_shared_u32(keys + e) : *gp(keys + e);
            lv[i] = coherent ? load_shared(lg + e) : *gp(lg + e);
            sv[i] = coherent ? load_shared(scr + e) : *gp(scr + e);
            // A non-finite logit or selection bias refuses the token (require_finite of the
            // logits and the bias, deepseek_v4_reference.cpp:235-238, :161).
            bad |= !isfinite(lv[i]) || key[i] <= 1u;
        }
    }
    // key[] is sorted in place; hid[] follows it. Values are read from lv/sv by id.
    uint32_t hid[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) hid[i] = lane + 64u * i;
#pragma unroll
    for (int i = 1; i < PER; ++i)
#pragma unroll
        for (int j = i; j > 0; --j)
            if (key[j] > key[j - 1]) {
                const uint32_t tk_ = key[j], ti = hid[j];
                key[j] = key[j - 1];
                hid[j] = hid[j - 1];
                key[j - 1] = tk_;
                hid[j - 1] = ti;
            }
    double sel = 0.0;  // the taken values, added in rank order
    for (uint32_t k = 0; k < K; ++k) {
        const uint32_t m = wave_max_u32(key[0]);
        const bool top = key[0] == m && m != 0;
        const uint64_t hit = __ballot(top);
        uint32_t wl = 0;
        if (hit == 0) {
            bad = true;
        } else if ((hit & (hit - 1)) == 0) {
            wl = (uint32_t)__builtin_ctzll(hit);
        } else {
            const uint32_t mid = wave_min_u32(top ? hid[0] : 0xffffffffu);
            wl = (uint32_t)__builtin_ctzll(__ballot(top && hid[0] == mid));
        }
        const uint32_t id = hit ? (uint32_t)__builtin_amdgcn_readlane((int)hid[0], wl) : 0u;
        const uint32_t wi = id >> 6;
        float l = lv[0], sc = sv[0];
#pragma unroll
        for (int i = 1; i < PER; ++i)
            if (wi == (uint32_t)i) {
                l = lv[i];
                sc = sv[i];
            }
        const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(softmax ? l : sc), id & 63u));
        sel += (double)v;
        if (lane == 0) {
            tk.id[k] = id;
            tk.val[k] = v;
        }
        if (lane == wl) {
#pragma unroll
            for (int i = 0; i + 1 < PER; ++i) {
                key[i] = key[i + 1];
                hid[i] = hid[i + 1];
            }
            key[PER - 1] = 0;
        }
    }
    if (!softmax) {
        // Weights are the taken scores over their sum (sel, added in rank order as taken).
        __builtin_amdgcn_wave_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (lane < K) {
            bad |= !(sel > 0.0) || isinf(sel);
            out_idx[lane] = tk.id[lane];
            out_w[lane] = (float)((double)tk.val[lane] / sel * (double)s.route_scale);
        }
        return __any(bad);
    }
    double sum_all = 0.0, mx = 0.0;
    {
        // The largest key is the largest logit: the first selected expert's.
        mx = (double)__int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(tk.val[0])));
#pragma unroll
        for (int i = 0; i < PER; ++i)
            if (lane + 64u * i < E) sum_all += exp((double)lv[i] - mx);
        sum_all = wave_sum_f64(sum_all);
    }
    __builtin_amdgcn_wave_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    double pk = 0.0;
    float vk = 0.0f;
    if (lane < K) {
        vk = tk.val[lane];
        pk = exp((double)vk - mx) * (sum_all > 0.0 ? 1.0 / sum_all : 0.0);
        tk.p[lane] = pk;
    }
    __builtin_amdgcn_wave_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (lane < K) {
        double sel_sum = 0.0;
#pragma unroll 8
        for (uint32_t q = 0; q < K; ++q) sel_sum += tk.p[q];
        float wk = (float)pk;
        if (s.renormalize && sel_sum > 0.0) wk = (float)((double)wk * (1.0 / sel_sum));
        out_idx[lane] = tk.id[lane];
        out_w[lane] = wk;
    }
    return __any(bad);
}

struct RouteLds {
    TopKLds topk[kMoeMaxTokens];
    uint32_t idx[kMoeMaxTokens * kMoeMaxTopK];
    float wt[kMoeMaxTokens * kMoeMaxTopK];
    uint32_t first[kMoeMaxTokens * kMoeMaxTopK];
    uint32_t bad[kMoeMaxTokens];
    uint32_t n_active;
    ActiveExpert act[kMaxActive];
};


// Routing of token t by one wave: its K ids and weights into idx/wt (LDS, in the token's rank
// order); returns true in every lane when the token is refused.
__device__ __forceinline__ bool route_token(const MoeShape& s, const MoeInputs& in,
                                            const MoeWorkspace& w, uint32_t t, TopKLds& tk,
                                            uint32_t* idx, float* wt, bool coherent = false) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t K = s.top_k, E = s.experts;
    const uint64_t base = (uint64_t)t * E;
    bool bad = false;
    if (s.routing == kRouteGiven || s.routing == kRouteTable) {
        for (uint32_t k = lane; k < K; k += 64) {
            uint32_t id = 0;
            if (s.routing == kRouteGiven) id = in.given_ids ? *gp(in.given_ids + t * K + k) : 0u;
            else id = *gp(in.table_ids + t * K + k);
            if (id >= E) { bad = true; id = 0; }
            idx[k] = id;
        }
        __builtin_amdgcn_wave_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        // Duplicate experts within one token are refused.
        for (uint32_t k = lane; k < K; k += 64)
            for (uint32_t j = 0; j < k; ++j)
                if (idx[j] == idx[k]) bad = true;
        if (s.routing == kRouteGiven) {
            for (uint32_t k = lane; k < K; k += 64)
                wt[k] = in.given_weights ? *gp(in.given_weights + t * K + k) : 1.0f;
        } else {
            // Every logit of the token must be finite, selected or not (activate_gate_logits,
            // deepseek_v4_reference.cpp:161).
            const float* lg = ws_ptr<const float>(w, w.off_logits) + base;
            for (uint32_t e = lane; e < E; e += 64u) bad |= !isfinite(coherent ? load_shared(lg + e) : *gp(lg + e));
            if (lane == 0) {
                const float* scr = ws_ptr<const float>(w, w.off_scores) + base;
                double sum = 0.0;
                float sc[kMoeMaxTopK];
                for (uint32_t k = 0; k < K; ++k) {
                    sc[k] = coherent ? load_shared(scr + idx[k]) : *gp(scr + idx[k]);
                    sum += (double)sc[k];
                }
                if (!(sum > 0.0) || isinf(sum)) bad = true;
                for (uint32_t k = 0; k < K; ++k)
                    wt[k] = (float)((double)sc[k] / sum * (double)s.route_scale);
            }
        }
    } else {
        const float* lg = ws_ptr<const float>(w, w.off_logits) + base;
        const float* scr = ws_ptr<const float>(w, w.off_scores) + base;
        const uint32_t* keys = ws_ptr<const uint32_t>(w, w.off_keys) + base;
        const bool softmax = s.routing == kRouteSoftmax;
        if (E <= 64) bad = route_topk<1>(lg, scr, keys, E, K, softmax, s, tk, idx, wt, coherent);
        else if (E <= 128) bad = route_topk<2>(lg, scr, keys, E, K, softmax, s, tk, idx, wt, coherent);
        else if (E <= 256) bad = route_topk<4>(lg, scr, keys, E, K, softmax, s, tk, idx, wt, coherent);
        else if (E <= 512) bad = route_topk<8>(lg, scr, keys, E, K, softmax, s, tk, idx, wt, coherent);
        else bad = route_topk<16>(lg, scr, keys, E, K, softmax, s, tk, idx, wt, coherent);
    }
    return __any(bad);
}

// Routing of token t by one wave of a gate/up block: ids and weights into rt.idx/wt, refusal into
// rt.bad[t].
__device__ __forceinline__ void route_token_wave(const MoeShape& s, const MoeInputs& in,
                                                 const MoeWorkspace& w, uint32_t t, RouteLds& rt,
                                                 bool coherent = false) {
    const uint32_t K = s.top_k;
    const bool bad = route_token(s, in, w, t, rt.topk[t], rt.idx + t * K, rt.wt + t * K, coherent);
    if ((threadIdx.x & 63u) == 0) rt.bad[t] = bad ? 1u : 0u;
}

// After route_token_wave for every token (and a barrier), the whole block builds the active-expert
// list: distinct experts in ascending id, each with its tokens in ascending order, and every
// token's combine order. publish also writes them (and the routes) to the workspace, and raises
// the status bits of refused routes and of non-finite activations (x_nonfinite).
__device__ __forceinline__ void build_active(const MoeShape& s, const MoeWorkspace& w, bool publish,
                                            bool x_nonfinite, RouteLds& rt,
                                            CombineEntry* comb_lds = nullptr) {
    const uint32_t K = s.top_k, E = s.experts, P = s.tokens * K;
    const uint32_t p = threadIdx.x;
    CombineEntry* comb = ws_ptr<CombineEntry>(w, w.off_combine);
    if (s.tokens == 1 && rt.bad[0] == 0) {
        // One routed token: its K experts are distinct, so expert p's active index and combine
        // position are its rank by id, with one token in slot 0 (what the general pass below
        // computes for this case, without its first-occurrence pass and barrier).
        if (p < K) {
            const uint32_t e = rt.idx[p];
            const float wt = rt.wt[p];
            if (publish) {
                *gp(ws_ptr<uint32_t>(w, w.off_route_idx) + p) = e;
                *gp(ws_ptr<float>(w, w.off_route_w) + p) = wt;
            }
            uint32_t a = 0;
#pragma unroll 8
            for (uint32_t q = 0; q < K; ++q) a += rt.idx[q] < e ? 1u : 0u;
            rt.act[a].tok[0] = 0;
            rt.act[a].route_w[0] = wt;
            rt.act[a].expert = e;
            rt.act[a].ntok = 1;
            rt.act[a].apply_w = s.semantics == kSemDeepseek ? 1u : 0u;
            rt.act[a].limit = s.routed_limit;
            const uint32_t at = s.semantics == kSemDeepseek ? a : p;
            const CombineEntry entry{a << 3, s.semantics == kSemQwen ? wt : 1.0f};
            if (publish) {
                uint32_t* ce = reinterpret_cast<uint32_t*>(comb + at);
                *gp(ce) = entry.src;
                *gp(ce + 1) = __float_as_uint(entry.w);
            }
            if (comb_lds) comb_lds[at] = entry;
        }
        if (threadIdx.x == 0) {
            if (s.has_shared) {
                ActiveExpert& sh = rt.act[K];
                sh.expert = E;
                sh.ntok = 1;
                sh.apply_w = 0;
                sh.limit = s.shared_limit;
                sh.tok[0] = 0;
                sh.route_w[0] = 1.0f;
                if (publish) {
                    uint32_t* ce = reinterpret_cast<uint32_t*>(comb + K);
                    *gp(ce) = K << 3;
                    *gp(ce + 1) = __float_as_uint(1.0f);
                }
                if (comb_lds) comb_lds[K] = CombineEntry{K << 3, 1.0f};
            }
            rt.n_active = K + (s.has_shared ? 1u : 0u);
            if (publish) {
                MoeHeader* hdr = ws_ptr<MoeHeader>(w, w.off_header);
                *gp(&hdr->n_active) = rt.n_active;
                if (x_nonfinite) or_bits(&hdr->status, kStatusNonFiniteInput);
            }
        }
    } else {
        // The loops below read LDS words whose loads are independent; unrolling lets several be in
        // flight at once instead of one latency per word.
        if (p < P) {
            uint32_t first = 1;
            const uint32_t ep = rt.idx[p];
#pragma unroll 8
            for (uint32_t q = 0; q < p; ++q) first &= rt.idx[q] != ep ? 1u : 0u;
            rt.first[p] = first;
        }
        __syncthreads();
        bool bad = false;
#pragma unroll 8
        for (uint32_t t = 0; t < s.tokens; ++t) bad |= rt.bad[t] != 0;
        if (p < P) {
            const uint32_t e = rt.idx[p], t = p / K, k = p % K;
            const float wt = rt.wt[p];
            if (publish) {
                *gp(ws_ptr<uint32_t>(w, w.off_route_idx) + p) = e;
                *gp(ws_ptr<float>(w, w.off_route_w) + p) = wt;
            }
            uint32_t a = 0, slot = 0, ntok = 0, pos = 0;
#pragma unroll 8
            for (uint32_t q = 0; q < P; ++q) {
                const uint32_t eq = rt.idx[q];
                a += (rt.first[q] && eq < e) ? 1u : 0u;
                ntok += eq == e ? 1u : 0u;
                slot += (eq == e && q < p) ? 1u : 0u;
            }
#pragma unroll 8
            for (uint32_t j = 0; j < K; ++j) pos += rt.idx[t * K + j] < e ? 1u : 0u;
            rt.act[a].tok[slot] = t;
            rt.act[a].route_w[slot] = wt;
            if (slot == 0) {
                rt.act[a].expert = e;
                rt.act[a].ntok = ntok;
                rt.act[a].apply_w = s.semantics == kSemDeepseek ? 1u : 0u;
                rt.act[a].limit = s.routed_limit;
            }
            const uint32_t at = s.semantics == kSemDeepseek ? pos : k;
            const CombineEntry entry{(a << 3) | slot, s.semantics == kSemQwen ? wt : 1.0f};
            if (publish) {
                uint32_t* ce = reinterpret_cast<uint32_t*>(comb + t * (K + 1) + at);
                *gp(ce) = entry.src;
                *gp(ce + 1) = __float_as_uint(entry.w);
            }
            if (comb_lds) comb_lds[t * (K + 1) + at] = entry;
        }
        if (threadIdx.x == 0) {
            uint32_t n_routed = 0;
#pragma unroll 8
            for (uint32_t q = 0; q < P; ++q) n_routed += rt.first[q];
            if (s.has_shared) {
                ActiveExpert& sh = rt.act[n_routed];
                sh.expert = E;
                sh.ntok = s.tokens;
                sh.apply_w = 0;
                sh.limit = s.shared_limit;
                for (uint32_t t = 0; t < s.tokens; ++t) {
                    sh.tok[t] = t;
                    sh.route_w[t] = 1.0f;
                    if (publish) {
                        uint32_t* ce = reinterpret_cast<uint32_t*>(comb + t * (K + 1) + K);
                        *gp(ce) = (n_routed << 3) | t;
                        *gp(ce + 1) = __float_as_uint(1.0f);
                    }
                    if (comb_lds) comb_lds[t * (K + 1) + K] = CombineEntry{(n_routed << 3) | t, 1.0f};
                }
            }
            rt.n_active = bad ? 0u : n_routed + (s.has_shared ? 1u : 0u);
            if (publish) {
                MoeHeader* hdr = ws_ptr<MoeHeader>(w, w.off_header);
                *gp(&hdr->n_active) = rt.n_active;
                const uint32_t bits = (bad ? kStatusBadRoute : 0u) | (x_nonfinite ? kStatusNonFiniteInput : 0u);
                if (bits) or_bits(&hdr->status, bits);
            }
        }
    }
    __syncthreads();
    if (publish) {
        const uint32_t words = rt.n_active * (uint32_t)(sizeof(ActiveExpert) / 4u);
        const uint32_t* src = reinterpret_cast<const uint32_t*>(rt.act);
        uint32_t* dst = ws_ptr<uint32_t>(w, w.off_active);
        for (uint32_t i = threadIdx.x; i < words; i += blockDim.x) *gp(dst + i) = src[i];
    }
}

// ------------------------------------------------------------------------------------------
// SwiGLU.
// ------------------------------------------------------------------------------------------

// ------------------------------------------------------------------------------------------
// Stream policies.
// ------------------------------------------------------------------------------------------

// Tile epilogues run out of line: they are rare, and inlined into the streaming loop their
// float64 code would compete with the in-flight weight buffers for registers. Their arguments are
// plain scalars (a structure argument would be passed through scratch memory).

// Last wave of gate/up tile job j: gate/up sums, SwiGLU, the tile's h rows ([A][NT][inter]), and
// the maxima of |h| per 256-row block and slot (hmax [A][hblocks][8], the down kernel's limb
// exponents). The active-expert list is the RouteLds at LDS byte route_off.
// With entries == nullptr the active list is the RouteLds at LDS byte route_off (per-block
// routing); otherwise it is the grouped path's list in global memory.
template <int NT>
__device__ __attribute__((noinline)) void gateup_fixup(const float* rec, float* hout, uint32_t* hmax,
                                                       uint32_t* status, uint32_t j, uint32_t first,
                                                       uint32_t last, uint32_t tiles, uint32_t hblocks,
                                                       uint32_t inter, uint32_t semantics,
                                                       uint32_t route_off, const ActiveExpert* entries) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t a = j / tiles, t = j - a * tiles;
    const ActiveExpert& ae =
        entries ? entries[a] : reinterpret_cast<const RouteLds*>(lds + route_off)->act[a];
    const uint32_t lane = threadIdx.x & 63u, n = lane & 31u, hh = lane >> 5;
    const uint32_t row = t * 32u + n, sb = t / 8u, F = inter;
    const uint32_t nt = uni(ae.ntok);
    bool bad = false;
#pragma unroll
    for (int i = 0; i < (NT + 1) / 2; ++i) {
        const uint32_t sl = 2u * i + hh;
        float hmag = 0.0f;
        if (sl < nt) {
            float gu[2];
            sum_records<NT, 2>(rec, 2u * NT * 64u, j, first, last, sl, n, gu);
            if (row < F) {
                const float h = swiglu(semantics, gu[0], gu[1], ae.limit, ae.apply_w != 0, ae.route_w[sl]);
                bad |= !isfinite(gu[0]) || !isfinite(gu[1]) || !isfinite(h);
                store_shared(hout + ((uint64_t)a * NT + sl) * F + row, h);
                hmag = isfinite(h) ? fabsf(h) : 0.0f;
            }
        }
        for (int o = 16; o > 0; o >>= 1) hmag = fmaxf(hmag, __shfl_xor(hmag, o));
        if (n == 0 && sl < nt)
            __hip_atomic_fetch_max(gp(hmax + ((uint64_t)a * hblocks + sb) * 8u + sl),
                                   __float_as_uint(hmag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (__any(bad) && lane == 0) or_bits(status, kStatusNonFiniteOutput);
}

// Gate and up projections: job j = (active expert a, tile t) = (j / tiles, j % tiles), two
// matrices per job.
template <uint32_t FMT, int NT, bool LDS>
struct GateUp {
    // wave loop interface
    uint32_t chunks, nmat, ng;
    ASrc<LDS, NT * 128u> as;
    float hscale;
    // context
    MoeShape s;
    MoeInputs in;
    MoeWorkspace w;
    vl_tiled_layout L;
    uint32_t tiles, UJ, TU, NW, wid;
    uint32_t stage_off, scale_off, route_off;
    const uint8_t* lds;
    const RouteLds* rt;
    const uint8_t* const* wptr;  // [a][2] gate, up
    uint32_t ntok;
    uint32_t tok[NT];

    __device__ TileRef tref(uint32_t j, uint32_t mat) const {
        const uint32_t a = j / tiles, t = j - a * tiles;
        return tile_ref<FMT>(L, uni_ptr(wptr[2u * a + mat]), t);
    }

    __device__ void job_begin(uint32_t j) {
        const uint32_t a = j / tiles;
        const ActiveExpert& ae = rt->act[a];
        ntok = uni(ae.ntok);
#pragma unroll
        for (int s2 = 0; s2 < NT; ++s2) tok[s2] = uni(ae.tok[(uint32_t)s2 < ntok ? s2 : 0]);
        const uint32_t m = threadIdx.x & 31u, kh = (threadIdx.x >> 5) & 1u;
        const uint32_t sl = a_slot(m), limb = a_limb(m);
        const uint32_t tk = ae.tok[sl < ntok ? sl : 0u];
        const uint32_t off = tk * 128u + limb * 32u + 16u * kh;
        if (LDS) as.off = stage_off + off;
        else as.ptr = ws_ptr<int8_t>(w, w.off_xlimbs) + off;
    }

    __device__ void scales(uint32_t, uint32_t c, float (&fs)[NT]) const {
        const uint32_t eb = FMT == VL_TYPE_Q8_0 ? c / 2u : c;
#pragma unroll
        for (int s2 = 0; s2 < NT; ++s2)
            fs[s2] = (uint32_t)s2 < ntok ? lds_load<float>(scale_off + 4u * (8u * eb + tok[s2])) : 0.0f;
    }

    static constexpr bool kPrefetch = false;

    __device__ uint32_t* store(uint32_t j, const float (&m0)[NT], const float (&m1)[NT], uint32_t& kc) const {
        const uint32_t lane = threadIdx.x & 63u;
        constexpr uint32_t RF = 2u * NT * 64u;
        float* r = ws_ptr<float>(w, w.off_rec_gu) + (uint64_t)(wid + j) * RF;
#pragma unroll
        for (int s2 = 0; s2 < NT; ++s2) {
            store_shared(r + s2 * 64u + lane, m0[s2]);
            store_shared(r + (NT + s2) * 64u + lane, m1[s2]);
        }
        kc = wave_of_unit(j * UJ + UJ - 1u, NW, TU) - wave_of_unit(j * UJ, NW, TU) + 1u;
        return counters_of(w).gu + j;
    }

    __device__ void fixup(uint32_t j) const {
        const float* rec = ws_ptr<const float>(w, w.off_rec_gu);
        const uint32_t first = wave_of_unit(j * UJ, NW, TU);
        const uint32_t last = wave_of_unit(j * UJ + UJ - 1u, NW, TU);
        const MoeCounters cn = counters_of(w);
        gateup_fixup<NT>(rec, ws_ptr<float>(w, w.off_h), cn.hmax,
                         &ws_ptr<MoeHeader>(w, w.off_header)->status, j, first, last, tiles,
                         w.hblocks, s.inter, s.semantics, route_off, nullptr);
    }
};

// Dynamic LDS of the gate/up kernel, from byte 0: decode tables, staged activation limbs (LDS
// path), the 2^-e scales of the activation blocks, per-wave flags, the routing state and the
// weight pointers.
// Layers with at most kPtrTabExperts routed experts keep every expert's gate and up pointers in
// LDS (loaded while the block routes), so the active experts' pointers cost no memory latency
// after routing.
constexpr uint32_t kPtrTabExperts = 256;
struct GateUpLds {
    uint32_t stage, scale, flags, route, wptr, ptab, bytes;
};
__host__ __device__ inline GateUpLds gateup_lds(uint32_t table_bytes, uint32_t stage_bytes,
                                                uint32_t xblocks) {
    GateUpLds l;
    l.stage = table_bytes;
    l.scale = l.stage + stage_bytes;
    l.flags = l.scale + xblocks * 8u * 4u;
    l.route = (l.flags + kStreamWaves * 4u + 15u) & ~15u;
    l.wptr = (l.route + (uint32_t)sizeof(RouteLds) + 15u) & ~15u;
    l.ptab = l.wptr + kMaxActive * 2u * 8u;
    l.bytes = l.ptab + (kPtrTabExperts + 1u) * 2u * 8u;
    return l;
}

template <uint32_t FMT, int NT, bool LDS>
__global__ void __launch_bounds__(stream_threads<NT>()) k_moe_gateup(const MoeShape s, const MoeInputs in,
                                                               const MoeWorkspace w) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr uint32_t TB = table_bytes<FMT>();
    const uint32_t stage_bytes = LDS ? (s.width / 32u) * NT * 128u : 0u;
    const GateUpLds lay = gateup_lds(TB, stage_bytes, w.xblocks);
    RouteLds& rt = *reinterpret_cast<RouteLds*>(lds + lay.route);
    const uint8_t** wptr = reinterpret_cast<const uint8_t**>(lds + lay.wptr);
    const uint32_t wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    int nonfinite = 0;
    // Waves 0..tokens-1 route; the others fill the decode tables and stage the activations, or,
    // when every wave routes, the whole block does so afterwards.
    const bool fillers = s.tokens < nwaves;
    if (wave < s.tokens) route_token_wave(s, in, w, wave, rt);
    if (!fillers) __syncthreads();
    if (!fillers || wave >= s.tokens) {
        const uint32_t first = fillers ? s.tokens : 0u;
        const uint32_t tid = threadIdx.x - 64u * first, nthr = blockDim.x - 64u * first;
        // The first batch of every copy below is loaded before anything is stored, so the phase
        // waits about one memory latency: decode tables, activation limbs, slot exponents and
        // flags, and the experts' gate/up pointers. Larger copies finish in plain loops.
        using TF = TableFill<FMT>;
        constexpr uint32_t XB = 4, SB = 2, PB = 2;
        TF tf;
        const bool one = TF::single(nthr);
        if (one) tf.load(tid, nthr);
        const uint4* xsrc = ws_ptr<const uint4>(w, w.off_xlimbs);
        uint4* xdst = reinterpret_cast<uint4*>(lds + lay.stage);
        const uint32_t xn = LDS ? stage_bytes / 16u : 0u;
        uint4 xv[XB];
#pragma unroll
        for (uint32_t j = 0; j < XB; ++j)
            if (tid + j * nthr < xn) xv[j] = ld_u4(xsrc + tid + j * nthr);
        const int* xe = ws_ptr<const int>(w, w.off_xexp);
        const uint32_t* xf = ws_ptr<const uint32_t>(w, w.off_xflags);
        float* sc = reinterpret_cast<float*>(lds + lay.scale);
        const uint32_t sn = w.xblocks * 8u;
        int ev[SB];
        uint32_t fv[SB];
#pragma unroll
        for (uint32_t j = 0; j < SB; ++j) {
            const uint32_t i = tid + j * nthr;
            ev[j] = 0;
            fv[j] = 0;
            if (i < sn && (i & 7u) < s.tokens) {
                ev[j] = *gp(xe + i);
                fv[j] = *gp(xf + i);
            }
        }
        uint64_t* pt = reinterpret_cast<uint64_t*>(lds + lay.ptab);
        const uint32_t pn = s.experts <= kPtrTabExperts ? 2u * (s.experts + (s.has_shared ? 1u : 0u)) : 0u;
        auto ptr_word = [&](uint32_t i) {
            const MoeExpert& ex = in.experts[i / 2u];
            return reinterpret_cast<uint64_t>((i % 2u) ? ex.up : ex.gate);
        };
        uint64_t pv[PB];
#pragma unroll
        for (uint32_t j = 0; j < PB; ++j)
            if (tid + j * nthr < pn) pv[j] = ptr_word(tid + j * nthr);
        if (one) tf.store(lds, tid, nthr);
        else fill_tables<FMT>(lds, tid, nthr);
#pragma unroll
        for (uint32_t j = 0; j < XB; ++j)
            if (tid + j * nthr < xn) xdst[tid + j * nthr] = xv[j];
        for (uint32_t i = tid + XB * nthr; i < xn; i += nthr) xdst[i] = ld_u4(xsrc + i);
#pragma unroll
        for (uint32_t j = 0; j < SB; ++j) {
            const uint32_t i = tid + j * nthr;
            if (i < sn) {
                const bool live = (i & 7u) < s.tokens;
                sc[i] = live ? __builtin_amdgcn_ldexpf(1.0f, -ev[j]) : 0.0f;
                if (live && fv[j]) nonfinite = 1;
            }
        }
        for (uint32_t i = tid + SB * nthr; i < sn; i += nthr) {
            const bool live = (i & 7u) < s.tokens;
            sc[i] = live ? __builtin_amdgcn_ldexpf(1.0f, -*gp(xe + i)) : 0.0f;
            if (live && *gp(xf + i)) nonfinite = 1;
        }
#pragma unroll
        for (uint32_t j = 0; j < PB; ++j)
            if (tid + j * nthr < pn) pt[tid + j * nthr] = pv[j];
        for (uint32_t i = tid + PB * nthr; i < pn; i += nthr) pt[i] = ptr_word(i);
    }
    const bool any_nonfinite = block_any(nonfinite != 0, reinterpret_cast<uint32_t*>(lds + lay.flags));
    build_active(s, w, blockIdx.x == 0, any_nonfinite, rt);
    const uint64_t* pt = reinterpret_cast<const uint64_t*>(lds + lay.ptab);
    for (uint32_t i = threadIdx.x; i < 2u * rt.n_active; i += blockDim.x) {
        const uint32_t e = rt.act[i / 2u].expert;
        if (s.experts <= kPtrTabExperts) {
            wptr[i] = reinterpret_cast<const uint8_t*>(pt[2u * e + i % 2u]);
        } else {
            const MoeExpert& ex = in.experts[e];
            wptr[i] = (i % 2u) ? ex.up : ex.gate;
        }
    }
    __syncthreads();
    GateUp<FMT, NT, LDS> pol;
    pol.s = s;
    pol.in = in;
    pol.w = w;
    vl_make_layout(FMT, s.inter, s.width, &pol.L);
    pol.chunks = units_per_row(FMT, s.width);
    pol.nmat = 2;
    pol.ng = pol.L.groups;
    pol.tiles = w.tiles_gu;
    pol.UJ = 2u * pol.chunks;
    pol.TU = uni(rt.n_active) * w.tiles_gu * pol.UJ;
    pol.NW = active_waves(gridDim.x * stream_waves<NT>(), pol.TU);
    pol.wid = blockIdx.x * stream_waves<NT>() + uni(threadIdx.x >> 6);
    pol.stage_off = lay.stage;
    pol.scale_off = lay.scale;
    pol.route_off = lay.route;
    pol.lds = lds;
    pol.rt = &rt;
    pol.wptr = wptr;
    pol.hscale = (threadIdx.x & 32u) ? 65536.0f : 1.0f;
    pol.ntok = 0;
    stream_range<FMT, NT, LDS>(pol, range_begin(pol.wid, pol.NW, pol.TU),
                               range_begin(pol.wid + 1u, pol.NW, pol.TU));
}

// Last wave of down job j: the expert's output rows of tile t (ypart [A][NT][width]); unless
// tile_cnt is null, the last expert of tile t then combines the layer output rows in each token's
// combine order (the CombineEntry table [tokens][top_k + 1] at LDS byte comb_off).
template <int NT>
__device__ __attribute__((noinline)) void down_fixup(const float* rec, float* ypart, float* out,
                                                     uint32_t* tile_cnt, uint32_t* status, uint32_t j,
                                                     uint32_t first, uint32_t last, uint32_t tiles,
                                                     uint32_t n_active, uint32_t width, uint32_t tokens,
                                                     uint32_t top_k, uint32_t has_shared,
                                                     uint32_t semantics, uint32_t ntok,
                                                     uint32_t comb_off) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t a = j / tiles, t = j - a * tiles;
    const uint32_t lane = threadIdx.x & 63u, n = lane & 31u, hh = lane >> 5;
    const uint32_t row = t * 32u + n, H = width;
#pragma unroll
    for (int i = 0; i < (NT + 1) / 2; ++i) {
        const uint32_t sl = 2u * i + hh;
        if (sl < ntok) {
            float y[1];
            sum_records<NT, 1>(rec, NT * 64u, j, first, last, sl, n, y);
            if (row < H) store_shared(ypart + ((uint64_t)a * NT + sl) * H + row, y[0]);
        }
    }
    if (!tile_cnt || !arrive(tile_cnt + t, n_active)) return;  // grouped path: combined later
    const CombineEntry* comb = reinterpret_cast<const CombineEntry*>(lds + comb_off);
    const uint32_t K = top_k, nent = K + (has_shared ? 1u : 0u);
    constexpr uint32_t kMaxEnt = kMoeMaxTopK + 1u;
    bool bad = false;
    for (uint32_t idx = lane; idx < tokens * 32u; idx += 64u) {
        const uint32_t tk = idx / 32u, r = t * 32u + idx % 32u;
        if (r >= H) continue;
        // All of the row's expert outputs are loaded before the first is added.
        float y[kMaxEnt];
#pragma unroll
        for (uint32_t k = 0; k < kMaxEnt; ++k) {
            y[k] = 0.0f;
            if (k < nent) {
                const uint32_t src = comb[tk * (K + 1u) + k].src;
                y[k] = load_shared(ypart + ((uint64_t)(src >> 3) * NT + (src & 7u)) * H + r);
            }
        }
        float acc = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < kMaxEnt; ++k) {
            if (k < nent) {
                const float wt = comb[tk * (K + 1u) + k].w;
                acc = (semantics == kSemQwen && k < K) ? __fadd_rn(acc, __fmul_rn(y[k], wt))
                                                       : __fadd_rn(acc, y[k]);
            }
        }
        bad |= !isfinite(acc);
        *gp(out + (uint64_t)tk * H + r) = acc;
    }
    if (__any(bad) && lane == 0) or_bits(status, kStatusNonFiniteOutput);
}

// Down projection: job j = (active expert a, tile t of the output rows). The block turns the h of
// the experts its units touch (a0 .. a0 + stage - 1) into limbs, in LDS when LDS is set and in
// the block's slab of the workspace otherwise, layout [expert][inter/32][NT][4][32].
template <uint32_t FMT, int NT, bool LDS>
struct Down {
    uint32_t chunks, nmat, ng;
    ASrc<LDS, NT * 128u> as;
    float hscale;
    MoeShape s;
    MoeInputs in;
    MoeWorkspace w;
    uint32_t n_active;
    vl_tiled_layout L;
    uint32_t tiles, UJ, TU, NW, wid;
    uint32_t a0, expert_bytes, stage_off, scale_off, comb_off;
    const int8_t* slab;
    const uint8_t* lds;
    const ActiveExpert* act;
    const uint8_t* const* wptr;
    uint32_t cur_a, ntok;

    __device__ TileRef tref(uint32_t j, uint32_t) const {
        const uint32_t a = j / tiles, t = j - a * tiles;
        return tile_ref<FMT>(L, uni_ptr(wptr[a]), t);
    }

    __device__ void job_begin(uint32_t j) {
        cur_a = j / tiles;
        ntok = uni(act[cur_a].ntok);
        const uint32_t m = threadIdx.x & 31u, kh = (threadIdx.x >> 5) & 1u;
        const uint32_t sl = a_slot(m), limb = a_limb(m);
        const uint32_t off = (cur_a - a0) * expert_bytes + (sl < ntok ? sl : 0u) * 128u + limb * 32u + 16u * kh;
        if (LDS) as.off = stage_off + off;
        else as.ptr = slab + off;
    }

    __device__ void scales(uint32_t, uint32_t c, float (&fs)[NT]) const {
        const uint32_t eb = FMT == VL_TYPE_Q8_0 ? c / 2u : c;
        const uint32_t sc = scale_off + 32u * ((cur_a - a0) * w.hblocks + eb);
#pragma unroll
        for (int s2 = 0; s2 < NT; ++s2) fs[s2] = (uint32_t)s2 < ntok ? lds_load<float>(sc + 4u * s2) : 0.0f;
    }

    static constexpr bool kPrefetch = false;

    __device__ uint32_t* store(uint32_t j, const float (&m0)[NT], const float (&)[NT], uint32_t& kc) const {
        const uint32_t lane = threadIdx.x & 63u;
        constexpr uint32_t RF = NT * 64u;
        float* r = ws_ptr<float>(w, w.off_rec_dn) + (uint64_t)(wid + j) * RF;
#pragma unroll
        for (int s2 = 0; s2 < NT; ++s2) store_shared(r + s2 * 64u + lane, m0[s2]);
        kc = wave_of_unit(j * UJ + UJ - 1u, NW, TU) - wave_of_unit(j * UJ, NW, TU) + 1u;
        return counters_of(w).dn + j;
    }

    __device__ void fixup(uint32_t j) const {
        const float* rec = ws_ptr<const float>(w, w.off_rec_dn);
        const uint32_t first = wave_of_unit(j * UJ, NW, TU);
        const uint32_t last = wave_of_unit(j * UJ + UJ - 1u, NW, TU);
        const MoeCounters cn = counters_of(w);
        down_fixup<NT>(rec, ws_ptr<float>(w, w.off_ypart), in.out, cn.tile,
                       &ws_ptr<MoeHeader>(w, w.off_header)->status, j, first, last, tiles, n_active,
                       s.width, s.tokens, s.top_k, s.has_shared, s.semantics,
                       uni(act[j / tiles].ntok), comb_off);
    }
};

// h of experts a0..a1 -> limbs (dst, [expert - a0][inter/32][NT][4][32]) with one exponent per
// 256-row block and slot from the gate/up kernel's maxima; scale[(a - a0)][block][8] = 2^-e.
// load() requests one batch of kB quads per thread (quads i0 + j * blockDim.x) and, with the
// first batch, this thread's scale maximum; store() converts and writes them, so a thread waits
// one memory latency per batch. ntok[a * stride] is expert a's token count.
template <int NT>
struct HConvert {
    static constexpr int kB = 8;
    const MoeWorkspace* w;
    const uint32_t* ntok;
    uint32_t inter, a0, stride, quads, total, nsc;
    float4 f4[kB];
    uint32_t mx[kB], sm;

    __device__ void init(const MoeWorkspace& ws, uint32_t inter_, uint32_t a0_, uint32_t a1,
                         const uint32_t* ntok_, uint32_t stride_) {
        w = &ws;
        ntok = ntok_;
        stride = stride_;
        inter = inter_;
        a0 = a0_;
        quads = inter / 4u;
        total = (a1 - a0 + 1u) * NT * quads;
        nsc = (a1 - a0 + 1u) * ws.hblocks * 8u;
    }
    __device__ uint32_t tokens(uint32_t a) const { return ntok[a * stride]; }
    __device__ bool live(uint32_t i) const {
        return i < total && (i / quads) % NT < tokens(a0 + i / (quads * NT));
    }
    __device__ void load(uint32_t i0) {
        const uint32_t* hmax = counters_of(*w).hmax;
        const float* h = ws_ptr<const float>(*w, w->off_h);
        if (i0 == threadIdx.x && threadIdx.x < nsc)
            sm = *gp(hmax + (uint64_t)a0 * w->hblocks * 8u + threadIdx.x);
#pragma unroll
        for (int j = 0; j < kB; ++j) {
            const uint32_t i = i0 + j * blockDim.x;
            const uint32_t q = i % quads, sl = (i / quads) % NT, a = a0 + i / (quads * NT), col = 4u * q;
            if (live(i)) {
                mx[j] = *gp(hmax + ((uint64_t)a * w->hblocks + col / 256u) * 8u + sl);
                f4[j] = ld_f4(h + ((uint64_t)a * NT + sl) * inter + col);
            }
        }
    }
    __device__ void store(uint32_t i0, int8_t* dst, float* scale) const {
        if (i0 == threadIdx.x) {
            const uint32_t* hmax = counters_of(*w).hmax;
            if (threadIdx.x < nsc) scale[threadIdx.x] = __builtin_amdgcn_ldexpf(1.0f, -limb_exponent(__uint_as_float(sm)));
            for (uint32_t i = threadIdx.x + blockDim.x; i < nsc; i += blockDim.x) {
                const uint32_t m = *gp(hmax + (uint64_t)a0 * w->hblocks * 8u + i);
                scale[i] = __builtin_amdgcn_ldexpf(1.0f, -limb_exponent(__uint_as_float(m)));
            }
        }
#pragma unroll
        for (int j = 0; j < kB; ++j) {
            const uint32_t i = i0 + j * blockDim.x;
            if (!live(i)) continue;
            const uint32_t q = i % quads, sl = (i / quads) % NT, al = i / (quads * NT), col = 4u * q;
            const float v[4] = {f4[j].x, f4[j].y, f4[j].z, f4[j].w};
            uint32_t packed[4];
            limbs4(v, limb_exponent(__uint_as_float(mx[j])), packed);
            int8_t* d = dst + (uint64_t)al * down_expert_bytes(inter, NT) +
                        ((uint64_t)(col / 32u) * NT + sl) * 128u + (col % 32u);
#pragma unroll
            for (int l = 0; l < 4; ++l) *reinterpret_cast<uint32_t*>(d + 32u * l) = packed[l];
        }
    }
};

// HConvert's halves over every batch; a thread with no quads still writes its scales.
template <int NT>
__device__ __forceinline__ void convert_h(const MoeWorkspace& w, uint32_t inter, uint32_t a0,
                                          uint32_t a1, const uint32_t* ntok, uint32_t ntok_stride,
                                          int8_t* dst, float* scale) {
    HConvert<NT> c;
    c.init(w, inter, a0, a1, ntok, ntok_stride);
    for (uint32_t i0 = threadIdx.x; i0 < c.total || i0 == threadIdx.x; i0 += HConvert<NT>::kB * blockDim.x) {
        c.load(i0);
        c.store(i0, dst, scale);
    }
}

// Dynamic LDS of the down kernel, from byte 0: decode tables, staged h limbs (LDS path), the 2^-e
// scales of the staged experts' h blocks, the active list, the down weight pointers and the
// combine table.
struct DownLds {
    uint32_t stage, scale, act, wptr, comb, dtab, bytes;
};
__host__ __device__ inline DownLds down_lds(uint32_t table_bytes, uint32_t stage_bytes,
                                            uint32_t stage, uint32_t hblocks) {
    DownLds l;
    l.stage = table_bytes;
    l.scale = l.stage + stage_bytes;
    l.act = (l.scale + stage * hblocks * 8u * 4u + 15u) & ~15u;
    l.wptr = l.act + kMaxActive * (uint32_t)sizeof(ActiveExpert);
    l.comb = l.wptr + kMaxActive * 8u;
    l.dtab = (l.comb + kMoeMaxTokens * (kMoeMaxTopK + 1u) * (uint32_t)sizeof(CombineEntry) + 7u) & ~7u;
    l.bytes = l.dtab + (kPtrTabExperts + 1u) * 8u;
    return l;
}

template <uint32_t FMT, int NT, bool LDS>
__global__ void __launch_bounds__(stream_threads<NT>()) k_moe_down(const MoeShape s, const MoeInputs in,
                                                             const MoeWorkspace w) {
    extern __shared__ __align__(16) uint8_t lds[];
    const MoeHeader* hdr = ws_ptr<const MoeHeader>(w, w.off_header);
    // The active count is loaded now but first used after the copies below have issued their
    // loads, so the kernel waits one memory latency for all of them.
    const uint32_t n_active_raw = *gp(&hdr->n_active);
    const uint32_t tiles = w.tiles_dn, UJ = units_per_row(FMT, s.inter);
    constexpr uint32_t WV = stream_waves<NT>();
    constexpr uint32_t TB = table_bytes<FMT>();
    const uint32_t eb = down_expert_bytes(s.inter, NT);
    const uint32_t stage_bytes = LDS ? w.stage * eb : 0u;
    const DownLds lay = down_lds(TB, stage_bytes, w.stage, w.hblocks);
    ActiveExpert* act = reinterpret_cast<ActiveExpert*>(lds + lay.act);
    const uint8_t** wptr = reinterpret_cast<const uint8_t**>(lds + lay.wptr);
    int8_t* slab = ws_ptr<int8_t>(w, w.off_hslab) + (uint64_t)blockIdx.x * w.stage * eb;
    // The decode tables' source words and every expert's down pointer (pools of up to
    // kPtrTabExperts) are requested before the active list and combine table are copied, so
    // the block waits one memory latency for all of them, and none for the weight pointers
    // after the barrier.
    TableFill<FMT> tf;
    const bool one = TableFill<FMT>::single(blockDim.x);
    if (one) tf.load(threadIdx.x, blockDim.x);
    static_assert(stream_threads<NT>() > kPtrTabExperts, "one down pointer per thread");
    uint64_t* dtab = reinterpret_cast<uint64_t*>(lds + lay.dtab);
    const uint32_t dn = s.experts <= kPtrTabExperts ? s.experts + (s.has_shared ? 1u : 0u) : 0u;
    uint64_t dv = 0;
    if (threadIdx.x < dn) dv = reinterpret_cast<uint64_t>(in.experts[threadIdx.x].down);
    {
        const uint32_t words = w.max_active * (uint32_t)(sizeof(ActiveExpert) / 4u);
        const uint32_t* src = ws_ptr<const uint32_t>(w, w.off_active);
        uint32_t* dst = reinterpret_cast<uint32_t*>(act);
        for (uint32_t i = threadIdx.x; i < words; i += blockDim.x) dst[i] = *gp(src + i);
        const uint32_t cwords = s.tokens * (s.top_k + 1u) * 2u;
        const uint32_t* csrc = ws_ptr<const uint32_t>(w, w.off_combine);
        uint32_t* cdst = reinterpret_cast<uint32_t*>(lds + lay.comb);
        for (uint32_t i = threadIdx.x; i < cwords; i += blockDim.x) cdst[i] = *gp(csrc + i);
    }
    if (one) tf.store(lds, threadIdx.x, blockDim.x);
    else fill_tables<FMT>(lds);
    if (threadIdx.x < dn) dtab[threadIdx.x] = dv;
    const uint32_t n_active = uni(n_active_raw);
    const uint32_t TU = n_active * tiles * UJ, NW = active_waves(gridDim.x * WV, TU);
    // Experts this block's units touch.
    const uint32_t ub0 = range_begin(blockIdx.x * WV, NW, TU);
    const uint32_t ub1 = range_begin((blockIdx.x + 1u) * WV, NW, TU);
    const uint32_t a0 = ub0 < ub1 ? (ub0 / UJ) / tiles : 0u;
    const uint32_t a1 = ub0 < ub1 ? ((ub1 - 1u) / UJ) / tiles : 0u;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n_active; i += blockDim.x)
        wptr[i] = dn ? reinterpret_cast<const uint8_t*>(dtab[act[i].expert]) : in.experts[act[i].expert].down;
    if (ub0 < ub1)
        convert_h<NT>(w, s.inter, a0, a1, &act[0].ntok, (uint32_t)(sizeof(ActiveExpert) / 4u),
                      LDS ? reinterpret_cast<int8_t*>(lds + lay.stage) : slab,
                      reinterpret_cast<float*>(lds + lay.scale));
    __syncthreads();
    if (n_active == 0) {
        if (blockIdx.x == 0)
            for (uint32_t i = threadIdx.x; i < s.tokens * s.width; i += blockDim.x) *gp(in.out + i) = 0.0f;
        return;
    }
    Down<FMT, NT, LDS> pol;
    pol.s = s;
    pol.in = in;
    pol.w = w;
    pol.n_active = n_active;
    vl_make_layout(FMT, s.width, s.inter, &pol.L);
    pol.chunks = UJ;
    pol.nmat = 1;
    pol.ng = pol.L.groups;
    pol.tiles = tiles;
    pol.UJ = UJ;
    pol.TU = TU;
    pol.NW = NW;
    pol.wid = blockIdx.x * WV + uni(threadIdx.x >> 6);
    pol.a0 = a0;
    pol.expert_bytes = eb;
    pol.stage_off = lay.stage;
    pol.scale_off = lay.scale;
    pol.comb_off = lay.comb;
    pol.slab = slab;
    pol.lds = lds;
    pol.act = act;
    pol.wptr = wptr;
    pol.hscale = (threadIdx.x & 32u) ? 65536.0f : 1.0f;
    pol.cur_a = 0;
    pol.ntok = 0;
    stream_range<FMT, NT, LDS>(pol, range_begin(pol.wid, NW, TU), range_begin(pol.wid + 1u, NW, TU));
}

// ------------------------------------------------------------------------------------------
// Grouped path: more than kMoeMaxTokens tokens.
//
// k_moe_route_many routes every token (one wave each) into the workspace's route arrays.
// k_moe_plan splits each selected expert's tokens, in ascending token order, into groups of up
// to kMoeMaxTokens (one job's MFMA token slots), appends the shared expert's groups (tokens in
// order) and writes every token's combine order. The gate/up and down kernels then stream the
// (group, tile) jobs of that list, and k_moe_combine adds each token's expert rows in its
// combine order. An expert's weights are read once per group of its tokens.
// ------------------------------------------------------------------------------------------

struct RouteWaveLds {
    TopKLds tk;
    uint32_t idx[kMoeMaxTopK];
    float wt[kMoeMaxTopK];
};

__global__ void __launch_bounds__(kStreamThreads) k_moe_route_many(const MoeShape s, const MoeInputs in,
                                                                   const MoeWorkspace w) {
    __shared__ RouteWaveLds r[kStreamWaves];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t t = blockIdx.x * kStreamWaves + wave;
    if (t >= s.tokens) return;
    RouteWaveLds& rw = r[wave];
    const bool bad = route_token(s, in, w, t, rw.tk, rw.idx, rw.wt);
    __builtin_amdgcn_wave_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const uint32_t K = s.top_k;
    if (lane < K) {
        *gp(ws_ptr<uint32_t>(w, w.off_route_idx) + (uint64_t)t * K + lane) = rw.idx[lane];
        *gp(ws_ptr<float>(w, w.off_route_w) + (uint64_t)t * K + lane) = rw.wt[lane];
    }
    if (bad && lane == 0) or_bits(&ws_ptr<MoeHeader>(w, w.off_header)->status, kStatusBadRoute);
}

// Dynamic LDS bytes of k_moe_plan: expert counts, group bases, the staged route ids, wave flags
// and one per-expert counter row per wave.
__host__ __device__ inline uint32_t plan_lds_bytes(const MoeShape& s) {
    return (2u * s.experts + 1u + s.tokens * s.top_k + kStreamWaves + kStreamWaves * s.experts) * 4u;
}

// One block: the grouped path's group list (ActiveExpert entries), their weight pointers, every
// token's combine entries, the group count and the status bits of refused routes and non-finite
// activations.
__global__ void __launch_bounds__(kStreamThreads) k_moe_plan(const MoeShape s, const MoeInputs in,
                                                             const MoeWorkspace w) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t T = s.tokens, K = s.top_k, E = s.experts, P = T * K;
    const uint32_t tid = threadIdx.x, nth = blockDim.x;
    uint32_t* cnt = reinterpret_cast<uint32_t*>(lds);
    uint32_t* base = cnt + E;
    uint32_t* ids = base + E + 1u;
    uint32_t* flags = ids + P;
    uint32_t* hist = flags + kStreamWaves;  // [wave][E]
    const uint32_t wave = tid >> 6, lane = tid & 63u, nw = nth >> 6;
    // Wave w takes tokens [tw0, tw1) in order.
    const uint32_t tw0 = (uint32_t)((uint64_t)wave * T / nw), tw1 = (uint32_t)((uint64_t)(wave + 1u) * T / nw);
    MoeHeader* hdr = ws_ptr<MoeHeader>(w, w.off_header);
    const uint32_t* ridx = ws_ptr<const uint32_t>(w, w.off_route_idx);
    const float* rwt = ws_ptr<const float>(w, w.off_route_w);
    for (uint32_t i = tid; i < P; i += nth) ids[i] = *gp(ridx + i);
    for (uint32_t i = tid; i < nw * E; i += nth) hist[i] = 0;
    bool nonfinite = false;
    const uint32_t* xf = ws_ptr<const uint32_t>(w, w.off_xflags);
    for (uint32_t i = tid; i < w.xblocks * w.estride; i += nth) nonfinite |= *gp(xf + i) != 0u;
    const bool any_nonfinite = block_any(nonfinite, flags);
    // 1. Per-wave counts of each expert over the wave's tokens (a token's experts are distinct;
    //    the duplicates of a refused token can only lose increments, which keeps ranks in range).
    //    Each assignment keeps its rank within the wave in the upper half of its id word.
    uint32_t* mine = hist + wave * E;
    for (uint32_t t = tw0; t < tw1; ++t)
        for (uint32_t k = lane; k < K; k += 64u) {
            const uint32_t e = ids[t * K + k];
            ids[t * K + k] = e | (mine[e]++ << 16);
        }
    __syncthreads();
    // 2. Per expert: the waves' counts become exclusive offsets; the total is the expert's count.
    for (uint32_t e = tid; e < E; e += nth) {
        uint32_t run = 0;
        for (uint32_t v = 0; v < nw; ++v) {
            const uint32_t h = hist[v * E + e];
            hist[v * E + e] = run;
            run += h;
        }
        cnt[e] = run;
    }
    __syncthreads();
    static_assert(kStreamThreads >= 1024u, "one expert per thread: layers have at most 1024");
    // Each expert's first group: an exclusive block scan of the group counts (one expert per
    // thread; the layer has at most as many experts as the block has threads), in the waves by
    // shuffles, then over the waves' totals.
    {
        const uint32_t g = tid < E ? (cnt[tid] + kMoeMaxTokens - 1u) / kMoeMaxTokens : 0u;
        uint32_t inc = g;
#pragma unroll
        for (uint32_t d = 1; d < 64u; d <<= 1) {
            const uint32_t v = (uint32_t)__shfl_up((int)inc, d);
            if (lane >= d) inc += v;
        }
        if (lane == 63u) flags[wave] = inc;
        __syncthreads();
        uint32_t before = 0, all = 0;
        for (uint32_t v = 0; v < nw; ++v) {
            const uint32_t f = flags[v];
            before += v < wave ? f : 0u;
            all += f;
        }
        if (tid < E) base[tid] = before + inc - g;
        if (tid == 0) base[E] = all;
    }
    __syncthreads();
    ActiveExpert* ent = ws_ptr<ActiveExpert>(w, w.off_active);
    MoeExpert* gw = ws_ptr<MoeExpert>(w, w.off_gweights);
    CombineEntry* comb = ws_ptr<CombineEntry>(w, w.off_combine);
    const bool deepseek = s.semantics == kSemDeepseek, qwen = s.semantics == kSemQwen;
    // 3. Every assignment in parallel: its rank among the expert's assignments is its wave's
    //    offset plus its rank within the wave, so an expert's ranks ascend with the tokens.
    for (uint32_t p = tid; p < P; p += nth) {
        const uint32_t t = p / K, k = p - t * K;
        const uint32_t e = ids[p] & 0xffffu;
        const uint32_t v = (uint32_t)((((uint64_t)t + 1u) * nw - 1u) / T);  // the wave holding t
        const uint32_t r = hist[v * E + e] + (ids[p] >> 16);
        const uint32_t a = base[e] + r / kMoeMaxTokens, sl = r % kMoeMaxTokens;
        ActiveExpert* A = ent + a;
        const float wt = *gp(rwt + p);
        *gp(&A->tok[sl]) = t;
        *gp(&A->route_w[sl]) = wt;
        if (sl == 0) {
            const uint32_t n = cnt[e];
            *gp(&A->expert) = e;
            *gp(&A->ntok) = n - r < kMoeMaxTokens ? n - r : kMoeMaxTokens;
            *gp(&A->apply_w) = deepseek ? 1u : 0u;
            *gp(&A->limit) = s.routed_limit;
            gw[a] = in.experts[e];
        }
        uint32_t at = k;
        if (deepseek) {
            at = 0;
            for (uint32_t k2 = 0; k2 < K; ++k2) at += (ids[t * K + k2] & 0xffffu) < e ? 1u : 0u;
        }
        uint32_t* ce = reinterpret_cast<uint32_t*>(comb + (uint64_t)t * (K + 1u) + at);
        *gp(ce) = (a << 3) | sl;
        *gp(ce + 1) = __float_as_uint(qwen ? wt : 1.0f);
    }
    const uint32_t routed_groups = base[E];
    if (s.has_shared) {
        const MoeExpert ex = in.experts[E];
        for (uint32_t t = tid; t < T; t += nth) {
            const uint32_t a = routed_groups + t / kMoeMaxTokens, sl = t % kMoeMaxTokens;
            ActiveExpert* A = ent + a;
            *gp(&A->tok[sl]) = t;
            *gp(&A->route_w[sl]) = 1.0f;
            if (sl == 0) {
                *gp(&A->expert) = E;
                *gp(&A->ntok) = T - t < kMoeMaxTokens ? T - t : kMoeMaxTokens;
                *gp(&A->apply_w) = 0u;
                *gp(&A->limit) = s.shared_limit;
                gw[a] = ex;
            }
            uint32_t* ce = reinterpret_cast<uint32_t*>(comb + (uint64_t)t * (K + 1u) + K);
            *gp(ce) = (a << 3) | sl;
            *gp(ce + 1) = __float_as_uint(1.0f);
        }
    }
    // The fp16 kernels' items: each expert's entries in runs of up to 2 * kWideGroups, in entry
    // order (an exclusive block scan of the run counts, as for the groups), then the shared
    // expert's.
    uint32_t nitems = 0;
    if (w.wide) {
        constexpr uint32_t RUN = 2u * kWideGroups;
        const uint32_t g = tid < E ? (cnt[tid] + kMoeMaxTokens - 1u) / kMoeMaxTokens : 0u;
        const uint32_t ni = (g + RUN - 1u) / RUN;
        uint32_t inc = ni;
#pragma unroll
        for (uint32_t d = 1; d < 64u; d <<= 1) {
            const uint32_t v = (uint32_t)__shfl_up((int)inc, d);
            if (lane >= d) inc += v;
        }
        if (lane == 63u) flags[wave] = inc;
        __syncthreads();
        uint32_t before = 0, all = 0;
        for (uint32_t v = 0; v < nw; ++v) {
            const uint32_t f = flags[v];
            before += v < wave ? f : 0u;
            all += f;
        }
        before += inc - ni;
        WideItem* items = ws_ptr<WideItem>(w, w.off_items);
        for (uint32_t i = 0; i < ni; ++i) {
            const uint32_t left = g - RUN * i;
            items[before + i] = WideItem{base[tid] + RUN * i, left < RUN ? left : RUN, {0u, 0u}};
        }
        nitems = all;
        if (s.has_shared) {
            const uint32_t gs = (T + kMoeMaxTokens - 1u) / kMoeMaxTokens, ns = (gs + RUN - 1u) / RUN;
            for (uint32_t i = tid; i < ns; i += nth) {
                const uint32_t left = gs - RUN * i;
                items[all + i] = WideItem{routed_groups + RUN * i, left < RUN ? left : RUN, {0u, 0u}};
            }
            nitems += ns;
        }
    }
    if (tid == 0) {
        const bool bad = (load_shared_u32(&hdr->status) & kStatusBadRoute) != 0;
        const uint32_t total = routed_groups + (s.has_shared ? (T + kMoeMaxTokens - 1u) / kMoeMaxTokens : 0u);
        *gp(&hdr->n_active) = bad ? 0u : total;
        *gp(&hdr->reserved[0]) = bad ? 0u : nitems;
        if (any_nonfinite) or_bits(&hdr->status, kStatusNonFiniteInput);
    }
}

// Dynamic LDS of the grouped stream kernels, from byte 0: decode tables, then per group the
// weight pointers (nptr of them), the token ids (u16 x kMoeMaxTokens) and the token count, then
// (down) the 2^-e scales of the staged groups' h blocks.
struct GroupLds {
    uint32_t wptr, tok, ntok, scale, bytes;
};
__host__ __device__ inline GroupLds group_lds(uint32_t table_bytes, uint32_t groups, uint32_t nptr,
                                              uint32_t scale_bytes) {
    GroupLds l;
    l.wptr = (table_bytes + 15u) & ~15u;
    l.tok = l.wptr + groups * nptr * 8u;
    l.ntok = l.tok + groups * kMoeMaxTokens * 2u;
    l.scale = (l.ntok + groups * 4u + 15u) & ~15u;
    l.bytes = l.scale + scale_bytes;
    return l;
}

// Copies the group list's pointers (gate/up or down), token ids and counts into LDS.
__device__ __forceinline__ void stage_groups(const MoeWorkspace& w, uint32_t n, const GroupLds& lay,
                                             bool down, uint8_t* lds) {
    const ActiveExpert* ent = ws_ptr<const ActiveExpert>(w, w.off_active);
    const MoeExpert* gw = ws_ptr<const MoeExpert>(w, w.off_gweights);
    uint64_t* wp = reinterpret_cast<uint64_t*>(lds + lay.wptr);
    uint16_t* tok = reinterpret_cast<uint16_t*>(lds + lay.tok);
    uint32_t* ntok = reinterpret_cast<uint32_t*>(lds + lay.ntok);
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const MoeExpert ex = gw[i];
        if (down) {
            wp[i] = reinterpret_cast<uint64_t>(ex.down);
        } else {
            wp[2u * i] = reinterpret_cast<uint64_t>(ex.gate);
            wp[2u * i + 1u] = reinterpret_cast<uint64_t>(ex.up);
        }
        const uint32_t nt = *gp(&ent[i].ntok);
        ntok[i] = nt;
        for (uint32_t k = 0; k < kMoeMaxTokens; ++k)
            tok[i * kMoeMaxTokens + k] = (uint16_t)(k < nt ? *gp(&ent[i].tok[k]) : 0u);
    }
}

template <uint32_t FMT>
struct GateUpGrouped {
    static constexpr int NT = kMoeMaxTokens;
    uint32_t chunks, nmat, ng;
    ASrc<false, 0> as;
    float hscale;
    MoeShape s;
    MoeWorkspace w;
    vl_tiled_layout L;
    uint32_t tiles, UJ, TU, NW, wid;
    uint32_t wptr_off, tok_off, ntok_off;
    uint32_t ntok;
    uint32_t tok[NT];

    __device__ TileRef tref(uint32_t j, uint32_t mat) const {
        const uint32_t a = j / tiles, t = j - a * tiles;
        const uint64_t p = lds_load<uint64_t>(wptr_off + (2u * a + mat) * 8u);
        return tile_ref<FMT>(L, uni_ptr(reinterpret_cast<const uint8_t*>(p)), t);
    }

    __device__ void job_begin(uint32_t j) {
        const uint32_t a = j / tiles;
        ntok = uni(lds_load<uint32_t>(ntok_off + 4u * a));
        const uint32_t tb = tok_off + 2u * NT * a;
#pragma unroll
        for (int s2 = 0; s2 < NT; ++s2) tok[s2] = uni(lds_load<uint16_t>(tb + 2u * s2));
        const uint32_t m = threadIdx.x & 31u, kh = (threadIdx.x >> 5) & 1u;
        const uint32_t sl = a_slot(m), limb = a_limb(m);
        const uint32_t tk = lds_load<uint16_t>(tb + 2u * (sl < ntok ? sl : 0u));
        as.ptr = ws_ptr<int8_t>(w, w.off_xlimbs) + (uint64_t)tk * 128u + limb * 32u + 16u * kh;
    }

    __device__ void scales(uint32_t, uint32_t c, float (&fs)[NT]) const {
        const uint32_t eb = FMT == VL_TYPE_Q8_0 ? c / 2u : c;
        const int* xe = ws_ptr<const int>(w, w.off_xexp) + (uint64_t)eb * w.estride;
#pragma unroll
        for (int s2 = 0; s2 < NT; ++s2)
            fs[s2] = (uint32_t)s2 < ntok ? __builtin_amdgcn_ldexpf(1.0f, -*gp(xe + tok[s2])) : 0.0f;
    }

    // Activations and exponents of up to 1024 tokens stay in global memory: a unit's eight A
    // fragments and slot scales are fetched one unit ahead.
    static constexpr bool kPrefetch = true;
    __device__ void load_ops(uint32_t j, uint32_t c, Operands<NT>& o) const {
        const uint32_t a = j / tiles;
        const uint32_t lane = threadIdx.x & 63u, m = lane & 31u, kh = lane >> 5;
        const uint32_t nt = lds_load<uint32_t>(ntok_off + 4u * a);
        const uint32_t tb = tok_off + 2u * NT * a;
        const uint32_t sl = a_slot(m), limb = a_limb(m);
        const uint32_t tk = lds_load<uint16_t>(tb + 2u * (sl < nt ? sl : 0u));
        const int8_t* p = ws_ptr<const int8_t>(w, w.off_xlimbs) + (uint64_t)tk * 128u + limb * 32u + 16u * kh;
        constexpr uint32_t NF = FMT == VL_TYPE_Q8_0 ? 4u : 8u;
#pragma unroll
        for (uint32_t g = 0; g < NF; ++g) {
            const uint32_t G = NF * c + g < ng ? NF * c + g : ng - 1u;  // past the row end: unused
            o.a[g] = *gp(reinterpret_cast<const i32x4*>(p + (uint64_t)G * as.stride));
        }
        // Lane s (< NT) fetches slot s's exponent; unused slots read token 0's and are masked
        // when the scales are formed.
        const uint32_t eb = FMT == VL_TYPE_Q8_0 ? c / 2u : c;
        const uint32_t ts = lds_load<uint16_t>(tb + 2u * (lane & (NT - 1u)));
        o.ev = (uint32_t)*gp(ws_ptr<const int>(w, w.off_xexp) + (uint64_t)eb * w.estride + ts);
    }

    __device__ void ops_scales(const Operands<NT>& o, uint32_t j, uint32_t, float (&fs)[NT]) const {
        const uint32_t nt = uni(lds_load<uint32_t>(ntok_off + 4u * (j / tiles)));
#pragma unroll
        for (int s2 = 0; s2 < NT; ++s2)
            fs[s2] = (uint32_t)s2 < nt
                         ? __builtin_amdgcn_ldexpf(1.0f, -(int)__builtin_amdgcn_readlane((int)o.ev, s2))
                         : 0.0f;
    }


    __device__ uint32_t* store(uint32_t j, const float (&m0)[NT], const float (&m1)[NT], uint32_t& kc) const {
        const uint32_t lane = threadIdx.x & 63u;
        constexpr uint32_t RF = 2u * NT * 64u;
        float* r = ws_ptr<float>(w, w.off_rec_gu) + (uint64_t)(wid + j) * RF;
#pragma unroll
        for (int s2 = 0; s2 < NT; ++s2) {
            store_shared(r + s2 * 64u + lane, m0[s2]);
            store_shared(r + (NT + s2) * 64u + lane, m1[s2]);
        }
        kc = wave_of_unit(j * UJ + UJ - 1u, NW, TU) - wave_of_unit(j * UJ, NW, TU) + 1u;
        return counters_of(w).gu + j;
    }

    __device__ void fixup(uint32_t j) const {
        const float* rec = ws_ptr<const float>(w, w.off_rec_gu);
        const uint32_t first = wave_of_unit(j * UJ, NW, TU);
        const uint32_t last = wave_of_unit(j * UJ + UJ - 1u, NW, TU);
        const MoeCounters cn = counters_of(w);
        gateup_fixup<NT>(rec, ws_ptr<float>(w, w.off_h), cn.hmax,
                         &ws_ptr<MoeHeader>(w, w.off_header)->status, j, first, last, tiles,
                         w.hblocks, s.inter, s.semantics, 0u, ws_ptr<const ActiveExpert>(w, w.off_active));
    }
};

// Waves per block of the grouped gate/up kernel: 12 (three per SIMD, 170 registers each) where
// the eight-slot loop fits that budget without spilling (IQ2_XXS, Q8_0), else 8.
template <uint32_t FMT>
__host__ __device__ constexpr uint32_t gateup_grouped_waves() {
    return FMT == VL_TYPE_IQ2_XXS || FMT == VL_TYPE_Q8_0 ? 12u : 8u;
}

template <uint32_t FMT>
__global__ void __launch_bounds__(gateup_grouped_waves<FMT>() * 64u) k_moe_gateup_grouped(const MoeShape s, const MoeInputs in,
                                                                       const MoeWorkspace w) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int NT = kMoeMaxTokens;
    const uint32_t n = uni(*gp(&ws_ptr<const MoeHeader>(w, w.off_header)->n_active));
    const GroupLds lay = group_lds(table_bytes<FMT>(), w.max_active, 2u, 0u);
    fill_tables<FMT>(lds);
    stage_groups(w, n, lay, false, lds);
    __syncthreads();
    if (n == 0) return;
    GateUpGrouped<FMT> pol;
    pol.s = s;
    pol.w = w;
    vl_make_layout(FMT, s.inter, s.width, &pol.L);
    pol.chunks = units_per_row(FMT, s.width);
    pol.nmat = 2;
    pol.ng = pol.L.groups;
    pol.tiles = w.tiles_gu;
    pol.UJ = 2u * pol.chunks;
    pol.TU = n * w.tiles_gu * pol.UJ;
    pol.NW = active_waves(gridDim.x * gateup_grouped_waves<FMT>(), pol.TU);
    pol.wid = blockIdx.x * gateup_grouped_waves<FMT>() + uni(threadIdx.x >> 6);
    pol.wptr_off = lay.wptr;
    pol.tok_off = lay.tok;
    pol.ntok_off = lay.ntok;
    pol.as.stride = w.xslots * 128u;
    pol.hscale = (threadIdx.x & 32u) ? 65536.0f : 1.0f;
    pol.ntok = 0;
    stream_range<FMT, NT, false>(pol, range_begin(pol.wid, pol.NW, pol.TU),
                                 range_begin(pol.wid + 1u, pol.NW, pol.TU));
}

template <uint32_t FMT>
struct DownGrouped {
    static constexpr int NT = kMoeMaxTokens;
    uint32_t chunks, nmat, ng;
    ASrc<false, NT * 128u> as;
    float hscale;
    MoeShape s;
    MoeInputs in;
    MoeWorkspace w;
    uint32_t n_active;
    vl_tiled_layout L;
    uint32_t tiles, UJ, TU, NW, wid;
    uint32_t a0, expert_bytes, scale_off, wptr_off, ntok_off;
    const int8_t* slab;
    uint32_t cur_a, ntok;

    __device__ TileRef tref(uint32_t j, uint32_t) const {
        const uint32_t a = j / tiles, t = j - a * tiles;
        const uint64_t p = lds_load<uint64_t>(wptr_off + 8u * a);
        return tile_ref<FMT>(L, uni_ptr(reinterpret_cast<const uint8_t*>(p)), t);
    }

    __device__ void job_begin(uint32_t j) {
        cur_a = j / tiles;
        ntok = uni(lds_load<uint32_t>(ntok_off + 4u * cur_a));
        const uint32_t m = threadIdx.x & 31u, kh = (threadIdx.x >> 5) & 1u;
        const uint32_t sl = a_slot(m), limb = a_limb(m);
        as.ptr = slab + (uint64_t)(cur_a - a0) * expert_bytes + (sl < ntok ? sl : 0u) * 128u + limb * 32u + 16u * kh;
    }

    __device__ void scales(uint32_t, uint32_t c, float (&fs)[NT]) const {
        const uint32_t eb = FMT == VL_TYPE_Q8_0 ? c / 2u : c;
        const uint32_t sc = scale_off + 32u * ((cur_a - a0) * w.hblocks + eb);
#pragma unroll
        for (int s2 = 0; s2 < NT; ++s2) fs[s2] = (uint32_t)s2 < ntok ? lds_load<float>(sc + 4u * s2) : 0.0f;
    }

    // The staged h limbs are L2-resident (written by this block's prologue) and jobs are eight
    // units long: loading a unit's A fragments one unit ahead measured slower than in place.
    static constexpr bool kPrefetch = false;

    __device__ uint32_t* store(uint32_t j, const float (&m0)[NT], const float (&)[NT], uint32_t& kc) const {
        const uint32_t lane = threadIdx.x & 63u;
        constexpr uint32_t RF = NT * 64u;
        float* r = ws_ptr<float>(w, w.off_rec_dn) + (uint64_t)(wid + j) * RF;
#pragma unroll
        for (int s2 = 0; s2 < NT; ++s2) store_shared(r + s2 * 64u + lane, m0[s2]);
        kc = wave_of_unit(j * UJ + UJ - 1u, NW, TU) - wave_of_unit(j * UJ, NW, TU) + 1u;
        return counters_of(w).dn + j;
    }

    __device__ void fixup(uint32_t j) const {
        const float* rec = ws_ptr<const float>(w, w.off_rec_dn);
        const uint32_t first = wave_of_unit(j * UJ, NW, TU);
        const uint32_t last = wave_of_unit(j * UJ + UJ - 1u, NW, TU);
        down_fixup<NT>(rec, ws_ptr<float>(w, w.off_ypart), in.out, nullptr,
                       &ws_ptr<MoeHeader>(w, w.off_header)->status, j, first, last, tiles, n_active,
                       s.width, s.tokens, s.top_k, s.has_shared, s.semantics,
                       uni(lds_load<uint32_t>(ntok_off + 4u * (j / tiles))), 0u);
    }
};

template <uint32_t FMT>
__global__ void __launch_bounds__(stream_threads<kMoeMaxTokens>()) k_moe_down_grouped(const MoeShape s, const MoeInputs in,
                                                                     const MoeWorkspace w) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int NT = kMoeMaxTokens;
    const uint32_t n_active = uni(*gp(&ws_ptr<const MoeHeader>(w, w.off_header)->n_active));
    const uint32_t tiles = w.tiles_dn, UJ = units_per_row(FMT, s.inter);
    constexpr uint32_t WV = stream_waves<NT>();
    const uint32_t TU = n_active * tiles * UJ, NW = active_waves(gridDim.x * WV, TU);
    const uint32_t ub0 = range_begin(blockIdx.x * WV, NW, TU);
    const uint32_t ub1 = range_begin((blockIdx.x + 1u) * WV, NW, TU);
    const uint32_t a0 = ub0 < ub1 ? (ub0 / UJ) / tiles : 0u;
    const uint32_t a1 = ub0 < ub1 ? ((ub1 - 1u) / UJ) / tiles : 0u;
    const uint32_t eb = down_expert_bytes(s.inter, NT);
    const GroupLds lay = group_lds(table_bytes<FMT>(), w.max_active, 1u, w.stage * w.hblocks * 32u);
    int8_t* slab = ws_ptr<int8_t>(w, w.off_hslab) + (uint64_t)blockIdx.x * w.stage * eb;
    fill_tables<FMT>(lds);
    stage_groups(w, n_active, lay, true, lds);
    __syncthreads();
    if (ub0 < ub1)
        convert_h<NT>(w, s.inter, a0, a1, reinterpret_cast<const uint32_t*>(lds + lay.ntok), 1u, slab,
                      reinterpret_cast<float*>(lds + lay.scale));
    __syncthreads();
    if (n_active == 0) return;
    DownGrouped<FMT> pol;
    pol.s = s;
    pol.in = in;
    pol.w = w;
    pol.n_active = n_active;
    vl_make_layout(FMT, s.width, s.inter, &pol.L);
    pol.chunks = UJ;
    pol.nmat = 1;
    pol.ng = pol.L.groups;
    pol.tiles = tiles;
    pol.UJ = UJ;
    pol.TU = TU;
    pol.NW = NW;
    pol.wid = blockIdx.x * WV + uni(threadIdx.x >> 6);
    pol.a0 = a0;
    pol.expert_bytes = eb;
    pol.scale_off = lay.scale;
    pol.wptr_off = lay.wptr;
    pol.ntok_off = lay.ntok;
    pol.slab = slab;
    pol.hscale = (threadIdx.x & 32u) ? 65536.0f : 1.0f;
    pol.cur_a = 0;
    pol.ntok = 0;
    stream_range<FMT, NT, false>(pol, range_begin(pol.wid, NW, TU), range_begin(pol.wid + 1u, NW, TU));
}

// out[t][r]: token t's expert rows added in its combine order (zero when the layer was refused).
__global__ void __launch_bounds__(256) k_moe_combine(const MoeShape s, const MoeInputs in,
                                                     const MoeWorkspace w) {
    constexpr uint32_t NT = kMoeMaxTokens, kMaxEnt = kMoeMaxTopK + 1u;
    const uint32_t H = s.width, K = s.top_k, nent = K + (s.has_shared ? 1u : 0u);
    // Four consecutive columns per thread (the width is a multiple of 32). Every entry's source
    // and row values are requested before the first is added; the sum keeps the combine order.
    const uint64_t i = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4u;
    const MoeHeader* hdr = ws_ptr<const MoeHeader>(w, w.off_header);
    const uint32_t n_active = *gp(&hdr->n_active);
    bool bad = false;
    if (i < (uint64_t)s.tokens * H) {
        const uint32_t t = (uint32_t)(i / H), r = (uint32_t)(i - (uint64_t)t * H);
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (n_active) {
            const CombineEntry* ce = ws_ptr<const CombineEntry>(w, w.off_combine) + (uint64_t)t * (K + 1u);
            const float* yp = ws_ptr<const float>(w, w.off_ypart);
            uint32_t src[kMaxEnt];
            float wt[kMaxEnt];
#pragma unroll
            for (uint32_t k = 0; k < kMaxEnt; ++k) {
                src[k] = k < nent ? *gp(&ce[k].src) : 0u;
                wt[k] = k < nent ? *gp(&ce[k].w) : 0.0f;
            }
            float4 y[kMaxEnt];
#pragma unroll
            for (uint32_t k = 0; k < kMaxEnt; ++k)
                if (k < nent) y[k] = ld_f4(yp + ((uint64_t)(src[k] >> 3) * NT + (src[k] & 7u)) * H + r);
#pragma unroll
            for (uint32_t k = 0; k < kMaxEnt; ++k) {
                if (k >= nent) continue;
                const float v[4] = {y[k].x, y[k].y, y[k].z, y[k].w};
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    acc[c] = (s.semantics == kSemQwen && k < K) ? __fadd_rn(acc[c], __fmul_rn(v[c], wt[k]))
                                                                : __fadd_rn(acc[c], v[c]);
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) bad |= !isfinite(acc[c]);
        const f32x4 o = {acc[0], acc[1], acc[2], acc[3]};
        *gp(reinterpret_cast<f32x4*>(in.out + i)) = o;
    }
    if (__any(bad) && (threadIdx.x & 63u) == 0)
        or_bits(&ws_ptr<MoeHeader>(w, w.off_header)->status, kStatusNonFiniteOutput);
}

// ------------------------------------------------------------------------------------------
// Launch sequence.
// ------------------------------------------------------------------------------------------

// LDS of one workgroup on gfx950; the stream kernels keep all their LDS in the dynamic part.
constexpr uint32_t kLdsBudget = 160u * 1024u;

// Events that the launch records around one kernel's execution (profiled layers), or none.
struct KernelEvents {
    hipEvent_t start, stop;
};

template <typename K, typename... Args>
static hipError_t launch_timed(const KernelEvents* ke, K kernel, dim3 grid, dim3 block, uint32_t shm,
                               hipStream_t st, Args... args) {
    if (ke) hipExtLaunchKernelGGL(kernel, grid, block, shm, st, ke->start, ke->stop, 0u, args...);
    else hipLaunchKernelGGL(kernel, grid, block, shm, st, args...);
    return hipGetLastError();
}

template <typename K, typename... Args>
static hipError_t launch_stream_ev(const KernelEvents* ke, K kernel, uint32_t blocks, uint32_t threads,
                                   uint32_t shm, hipStream_t st, Args... args) {
    const hipError_t e = ensure_dynamic_lds((const void*)kernel, shm);
    if (e != hipSuccess) return e;
    return launch_timed(ke, kernel, dim3(blocks), dim3(threads), shm, st, args...);
}

template <typename K, typename... Args>
static hipError_t launch_stream(K kernel, uint32_t blocks, uint32_t threads, uint32_t shm,
                                hipStream_t st, Args... args) {
    return launch_stream_ev(static_cast<const KernelEvents*>(nullptr), kernel, blocks, threads, shm, st, args...);
}

template <uint32_t FMT, int NT>
static hipError_t launch_gateup_nt(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                                   hipStream_t st, const KernelEvents* ke) {
    const uint32_t stage = (s.width / 32u) * NT * 128u;
    const GateUpLds staged = gateup_lds(table_bytes<FMT>(), stage, w.xblocks);
    if (staged.bytes <= kLdsBudget)
        return launch_stream_ev(ke, k_moe_gateup<FMT, NT, true>, w.blocks, stream_threads<NT>(), staged.bytes, st, s, in, w);
    const GateUpLds plain = gateup_lds(table_bytes<FMT>(), 0u, w.xblocks);
    return launch_stream_ev(ke, k_moe_gateup<FMT, NT, false>, w.blocks, stream_threads<NT>(), plain.bytes, st, s, in, w);
}

template <uint32_t FMT>
static hipError_t launch_gateup_fmt(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                                    hipStream_t st, const KernelEvents* ke = nullptr) {
    switch (w.slots) {
        case 1: return launch_gateup_nt<FMT, 1>(s, in, w, st, ke);
        case 2: return launch_gateup_nt<FMT, 2>(s, in, w, st, ke);
        case 4: return launch_gateup_nt<FMT, 4>(s, in, w, st, ke);
        default: return launch_gateup_nt<FMT, 8>(s, in, w, st, ke);
    }
}

template <uint32_t FMT, int NT>
static hipError_t launch_down_nt(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                                 hipStream_t st, const KernelEvents* ke) {
    const DownLds staged = down_lds(table_bytes<FMT>(), w.stage * down_expert_bytes(s.inter, NT),
                                    w.stage, w.hblocks);
    if (staged.bytes <= kLdsBudget)
        return launch_stream_ev(ke, k_moe_down<FMT, NT, true>, w.blocks, stream_threads<NT>(), staged.bytes, st, s, in, w);
    const DownLds plain = down_lds(table_bytes<FMT>(), 0u, w.stage, w.hblocks);
    return launch_stream_ev(ke, k_moe_down<FMT, NT, false>, w.blocks, stream_threads<NT>(), plain.bytes, st, s, in, w);
}

template <uint32_t FMT>
static hipError_t launch_down_fmt(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                                  hipStream_t st, const KernelEvents* ke = nullptr) {
    switch (w.slots) {
        case 1: return launch_down_nt<FMT, 1>(s, in, w, st, ke);
        case 2: return launch_down_nt<FMT, 2>(s, in, w, st, ke);
        case 4: return launch_down_nt<FMT, 4>(s, in, w, st, ke);
        default: return launch_down_nt<FMT, 8>(s, in, w, st, ke);
    }
}

template <uint32_t FMT>
static hipError_t launch_gateup_grouped(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                                        hipStream_t st) {
    const GroupLds lay = group_lds(table_bytes<FMT>(), w.max_active, 2u, 0u);
    if (lay.bytes > kLdsBudget) return hipErrorInvalidValue;
    return launch_stream(k_moe_gateup_grouped<FMT>, w.blocks, gateup_grouped_waves<FMT>() * 64u, lay.bytes, st, s, in, w);
}

template <uint32_t FMT>
static hipError_t launch_down_grouped(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                                      hipStream_t st) {
    const GroupLds lay = group_lds(table_bytes<FMT>(), w.max_active, 1u, w.stage * w.hblocks * 32u);
    if (lay.bytes > kLdsBudget) return hipErrorInvalidValue;
    return launch_stream(k_moe_down_grouped<FMT>, w.blocks, stream_threads<kMoeMaxTokens>(), lay.bytes, st, s, in, w);
}

// Routing, planning, gate/up, down and combine of the grouped path.
static hipError_t launch_moe_grouped(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                                     hipStream_t st, hipEvent_t* ev, hipEvent_t* kev) {
    // Stages of several kernels: each stage's kernel bracket is recorded at its boundaries.
    auto mark = [&](uint32_t stage) {
        if (kev && stage > 0) (void)hipEventRecord(kev[2u * stage - 1u], st);  // previous stop
        if (ev) (void)hipEventRecord(ev[stage], st);
        if (kev && stage < kStageCount) (void)hipEventRecord(kev[2u * stage], st);  // start
    };
    mark(kStageRouter);
    // The router kernel zeroes the counters and forms the activation limbs (the fp16 kernels'
    // activations come from k_wide_prep); the logits come from the tiled product.
    const uint32_t groups = (s.tokens + kMoeMaxTokens - 1u) / kMoeMaxTokens;
    MoeShape sx = s;
    sx.routing = kRouteGiven;
    hipError_t e;
    if (w.wide) {
        if ((e = launch_wide_prep(s, in, w, st)) != hipSuccess) return e;
    } else {
        hipLaunchKernelGGL(k_moe_router, dim3(w.xblocks, groups), dim3(256), 0, st, sx, in, w);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (s.routing != kRouteGiven) {
        hipLaunchKernelGGL(k_moe_logits_part,
                           dim3((s.experts + kLgE - 1u) / kLgE, (s.tokens + kLgT - 1u) / kLgT, w.lg_slices),
                           dim3(256), 0, st, s, in, w);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if ((e = launch_logits_finish(s, in, w, st)) != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k_moe_route_many, dim3((s.tokens + kStreamWaves - 1u) / kStreamWaves),
                       dim3(kStreamThreads), 0, st, s, in, w);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const uint32_t plan_shm = plan_lds_bytes(s);
    if ((e = ensure_dynamic_lds((const void*)k_moe_plan, plan_shm)) != hipSuccess) return e;
    hipLaunchKernelGGL(k_moe_plan, dim3(1), dim3(kStreamThreads), plan_shm, st, s, in, w);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    mark(kStageGateUp);
    if (w.wide) {
        if ((e = launch_wide_gateup(s, in, w, st)) != hipSuccess) return e;
        mark(kStageDown);
        if ((e = launch_wide_down(s, in, w, st)) != hipSuccess) return e;
        const uint64_t outs = (uint64_t)s.tokens * s.width;
        hipLaunchKernelGGL(k_moe_combine, dim3((uint32_t)((outs / 4u + 255u) / 256u)), dim3(256), 0, st, s, in, w);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        mark(kStageCount);
        return hipSuccess;
    }
    switch (s.gate_type) {
        case VL_TYPE_IQ2_XXS: e = launch_gateup_grouped<VL_TYPE_IQ2_XXS>(s, in, w, st); break;
        case VL_TYPE_IQ3_XXS: e = launch_gateup_grouped<VL_TYPE_IQ3_XXS>(s, in, w, st); break;
        case VL_TYPE_IQ1_S: e = launch_gateup_grouped<VL_TYPE_IQ1_S>(s, in, w, st); break;
        case VL_TYPE_Q8_0: e = launch_gateup_grouped<VL_TYPE_Q8_0>(s, in, w, st); break;
        default: e = launch_gguf_moe_gateup(s, in, w, st); break;
    }
    if (e != hipSuccess) return e;
    mark(kStageDown);
    switch (s.down_type) {
        case VL_TYPE_IQ2_XXS: e = launch_down_grouped<VL_TYPE_IQ2_XXS>(s, in, w, st); break;
        case VL_TYPE_IQ3_XXS: e = launch_down_grouped<VL_TYPE_IQ3_XXS>(s, in, w, st); break;
        case VL_TYPE_IQ1_S: e = launch_down_grouped<VL_TYPE_IQ1_S>(s, in, w, st); break;
        case VL_TYPE_Q8_0: e = launch_down_grouped<VL_TYPE_Q8_0>(s, in, w, st); break;
        default: e = launch_gguf_moe_down(s, in, w, st); break;
    }
    if (e != hipSuccess) return e;
    const uint64_t outs = (uint64_t)s.tokens * s.width;
    hipLaunchKernelGGL(k_moe_combine, dim3((uint32_t)((outs / 4u + 255u) / 256u)), dim3(256), 0, st, s, in, w);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    mark(kStageCount);
    return hipSuccess;
}

hipError_t launch_moe_route(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w, hipStream_t st) {
    if (!moe_shape_ok(s) || w.blocks == 0 || s.routing == kRouteGiven) return hipErrorInvalidValue;
    hipError_t e;
    if (w.grouped) {
        // As the grouped layer: the router kernel zeroes the status and counters and forms the
        // activation limbs; the logits come from the tiled product.
        MoeShape sx = s;
        sx.routing = kRouteGiven;
        if (w.wide) {
            if ((e = launch_wide_prep(s, in, w, st)) != hipSuccess) return e;
        } else {
            hipLaunchKernelGGL(k_moe_router, dim3(w.xblocks, (s.tokens + kMoeMaxTokens - 1u) / kMoeMaxTokens),
                               dim3(256), 0, st, sx, in, w);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        hipLaunchKernelGGL(k_moe_logits_part,
                           dim3((s.experts + kLgE - 1u) / kLgE, (s.tokens + kLgT - 1u) / kLgT, w.lg_slices),
                           dim3(256), 0, st, s, in, w);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if ((e = launch_logits_finish(s, in, w, st)) != hipSuccess) return e;
    } else {
        hipLaunchKernelGGL(k_moe_router, dim3(s.experts + w.xblocks), dim3(256), 0, st, s, in, w);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_moe_route_many, dim3((s.tokens + kStreamWaves - 1u) / kStreamWaves), dim3(kStreamThreads),
                       0, st, s, in, w);
    return hipGetLastError();
}

hipError_t launch_moe(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                      hipStream_t st, hipEvent_t* ev, hipEvent_t* kev) {
    if (!moe_shape_ok(s) || w.blocks == 0) return hipErrorInvalidValue;
    if (w.grouped) return launch_moe_grouped(s, in, w, st, ev, kev);
    // Stage kernel brackets: start and stop of each stage's kernel.
    KernelEvents ke[kStageCount];
    for (uint32_t i = 0; kev && i < kStageCount; ++i) ke[i] = KernelEvents{kev[2u * i], kev[2u * i + 1u]};
    auto rec = [&](hipEvent_t e) { (void)hipEventRecord(e, st); };
    auto mark = [&](uint32_t stage) {
        if (ev) rec(ev[stage]);
    };
    mark(kStageRouter);
    const uint32_t router_blocks = (s.routing == kRouteGiven ? 0u : s.experts) + w.xblocks;
    hipError_t e = launch_timed(kev ? &ke[kStageRouter] : nullptr, k_moe_router, dim3(router_blocks),
                                dim3(256), 0u, st, s, in, w);
    if (e != hipSuccess) return e;
    mark(kStageGateUp);
    if (tok_applies(s, w.blocks)) {
        e = launch_tok_gateup(s, in, w, st, kev ? kev + 2u * kStageGateUp : nullptr);
        if (e != hipSuccess) return e;
        mark(kStageDown);
        e = launch_tok_down(s, in, w, st, kev ? kev + 2u * kStageDown : nullptr);
        mark(kStageCount);
        return e;
    }
    const KernelEvents* kg = kev ? &ke[kStageGateUp] : nullptr;
    switch (s.gate_type) {
        case VL_TYPE_IQ2_XXS: e = launch_gateup_fmt<VL_TYPE_IQ2_XXS>(s, in, w, st, kg); break;
        case VL_TYPE_IQ3_XXS: e = launch_gateup_fmt<VL_TYPE_IQ3_XXS>(s, in, w, st, kg); break;
        case VL_TYPE_IQ1_S: e = launch_gateup_fmt<VL_TYPE_IQ1_S>(s, in, w, st, kg); break;
        case VL_TYPE_Q8_0: e = launch_gateup_fmt<VL_TYPE_Q8_0>(s, in, w, st, kg); break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    mark(kStageDown);
    const KernelEvents* kd = kev ? &ke[kStageDown] : nullptr;
    switch (s.down_type) {
        case VL_TYPE_IQ2_XXS: e = launch_down_fmt<VL_TYPE_IQ2_XXS>(s, in, w, st, kd); break;
        case VL_TYPE_IQ3_XXS: e = launch_down_fmt<VL_TYPE_IQ3_XXS>(s, in, w, st, kd); break;
        case VL_TYPE_IQ1_S: e = launch_down_fmt<VL_TYPE_IQ1_S>(s, in, w, st, kd); break;
        case VL_TYPE_Q8_0: e = launch_down_fmt<VL_TYPE_Q8_0>(s, in, w, st, kd); break;
        default: return hipErrorInvalidValue;
    }
    mark(kStageCount);
    return e;
}

// ------------------------------------------------------------------------------------------
// Workspace for callers that cannot allocate: one array per device, in the code object's own
// device memory, shared by every call on that device.
// ------------------------------------------------------------------------------------------

static __device__ __align__(256) uint8_t scratch[kStaticWorkspaceBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

// The address of the current device's scratch array, looked up once per device (the array's name
// is a host-side stand-in, not a device address).
hipError_t static_workspace(void** ptr) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return hipSuccess;
}

}  // namespace vl
