// Host-side interface of the MoE-layer kernels (vl_moe.hip).
#ifndef VL_MOE_H
#define VL_MOE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vl {

// Resident (tiled) weights of one expert.
struct MoeExpert {
    const uint8_t* gate;
    const uint8_t* up;
    const uint8_t* down;
};

// How the expert's activation is formed and how expert outputs are combined.
enum MoeSemantics : uint32_t {
    // execute_expert + moe_forward (deepseek_v4_graph.cpp:1826-1894, :2129-2266): float64 SwiGLU
    // with optional clamp, route weight applied before the down projection, outputs added in
    // ascending expert id, shared expert last.
    kSemDeepseek = 0,
    // qwen38_expert_mlp_q8 + qwen38_moe_block (qwen3_8_flash_next_reference.cpp:1317-1421):
    // silu_f(g) * u in float, route weight applied to the expert output in slot order.
    kSemQwen = 1,
    // routed_expert_iq1_s_iq3_xxs_f32 (ggml_quantization.cpp:1678-1745): g / (1 + expf(-g)) * u
    // in float, no clamp, no route weight.
    kSemPlain = 2,
};

enum MoeRouting : uint32_t {
    kRouteLearned = 0,  // top-k of score(logit) + bias (deepseek_v4_reference.cpp:223-255)
    kRouteTable = 1,    // ids from a per-token table, weights from scores (:275-307)
    kRouteSoftmax = 2,  // float64 softmax top-k (qwen3_8_flash_next_reference.cpp:1186-1240)
    kRouteGiven = 3,    // ids and weights supplied by the caller (one expert FFN call)
};

enum MoeScore : uint32_t { kScoreSqrtSoftplus = 0, kScoreSigmoid = 1 };

// Token slots of one MFMA job; more tokens take the grouped path (up to kMoeMaxTokensGrouped
// tokens, with at most kMoeMaxGroupAssign token-expert assignments and kMoeMaxGroups groups).
constexpr uint32_t kMoeMaxTokens = 8;
constexpr uint32_t kMoeMaxTopK = 16;
constexpr uint32_t kMoeMaxTokensGrouped = 1024;
constexpr uint32_t kMoeMaxGroupAssign = 16384;
constexpr uint32_t kMoeMaxGroups = 1792;

struct MoeShape {
    uint32_t tokens, width, inter, experts, top_k;
    uint32_t gate_type, down_type;
    uint32_t semantics, routing, score_fn, has_shared, renormalize;
    float route_scale, routed_limit, shared_limit;
};

// Inputs of one layer call. Router and bias are float32; table ids [tokens][top_k]; given ids
// and weights [tokens][top_k] for kRouteGiven (weights may be null: no route weight).
struct MoeInputs {
    const MoeExpert* experts;  // device array: experts entries, then the shared expert
    const float* router;       // [experts][width]
    const float* bias;         // [experts] or null
    const uint32_t* table_ids;
    const uint32_t* given_ids;
    const float* given_weights;
    const float* x;            // [tokens][width]
    float* out;                // [tokens][width]
};

// Device workspace of one layer call, carved by moe_workspace_layout. The first word is the
// status word. Sizes depend on the persistent grid (waves) of the device the call runs on.
struct MoeWorkspace {
    uint8_t* base;
    uint64_t bytes;
    uint64_t off_header, off_logits, off_scores, off_keys, off_route_idx, off_route_w, off_active, off_combine,
        off_xexp, off_xflags, off_xlimbs, off_counters, off_rec_gu, off_rec_dn, off_h,
        off_hslab, off_ypart, off_gweights, off_lgpart, off_trec;
    // Grouped layers on the fp16 kernels: activations and h as hi/lo fp16 [row][2][cols], with one
    // scale per token (x) and per row and 256-column block (h), and the item list.
    uint64_t off_x16, off_xsc, off_h16, off_hsc, off_items;
    uint32_t grouped;                                 // more than kMoeMaxTokens tokens
    uint32_t wide;                                    // grouped, on the fp16 kernels
    uint32_t max_items;
    uint32_t lg_slices;                               // column slices of the grouped router product
    uint32_t max_active, slots, waves, blocks;        // slots: MFMA token slots of a job
    uint32_t xslots, estride;                         // token strides of the limb and exponent arrays
    uint32_t tiles_gu, tiles_dn, hblocks, xblocks;  // gate/up and down tiles, h and x exponent blocks
    uint32_t counters;                                // u32 words at off_counters
    uint32_t stage;                                   // experts one down block converts h for
};

bool moe_shape_ok(const MoeShape& s);
// blocks: persistent blocks of the matvec kernels (one per CU).
uint64_t moe_workspace_bytes(const MoeShape& s, uint32_t blocks);
MoeWorkspace moe_workspace_layout(const MoeShape& s, uint32_t blocks, void* base);

// Stages of one layer call, in launch order; a profiled call records an event before each
// stage and one after the last.
enum MoeStage : uint32_t { kStageRouter = 0, kStageGateUp, kStageDown, kStageCount };

// Issues the whole layer on the stream. When events is non-null it holds kStageCount + 1 events
// recorded between the stages; when kernel_events is non-null, a start and a stop event per stage
// that bracket the stage's kernel itself (recorded by the launch; stages of several kernels and
// single-launch layers record them at the stage boundaries). Bracketed launches lengthen the gaps
// between kernels, so the two are meant for separate calls.
hipError_t launch_moe(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& ws,
                      hipStream_t stream, hipEvent_t* events = nullptr,
                      hipEvent_t* kernel_events = nullptr);

// Routes every token without running the experts: the router stage and the per-token routing of
// the layer, leaving the routes (and the refusal bits of the status word) in the workspace. For
// callers that must know the selected experts before their weights are on the device.
hipError_t launch_moe_route(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& ws, hipStream_t stream);

// Gate/up and down stages of a grouped layer whose gate/up or down matrices are of a GGUF-layout
// type (vl_gguf.hip): they read the plan, the active groups and their weight pointers, and write
// h and the per-slot down outputs as the tiled grouped stages do.
hipError_t launch_gguf_moe_gateup(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& ws,
                                  hipStream_t stream);
hipError_t launch_gguf_moe_down(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& ws,
                                hipStream_t stream);
// Bytes of the per-device workspace that vl_moe_layer_noalloc uses instead of a caller's buffer.
constexpr uint64_t kStaticWorkspaceBytes = 64ull << 20;

// Device address of the current device's static workspace (kStaticWorkspaceBytes), looked up on
// the first call for each device; nothing is allocated.
hipError_t static_workspace(void** ptr);

}  // namespace vl

#endif  // VL_MOE_H
