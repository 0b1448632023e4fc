/* vastloom_hip.h - C ABI of the MI355X (gfx950) quantized routed-expert path.
 *
 * This library takes the place of the reference's CUDA device boundary (src/cuda: the
 * CudaDriver/CudaDriverBackend launch entries and the CudaMatvecAccelerator seam) for the
 * GGUF storage types Q8_0, IQ2_XXS, IQ3_XXS and IQ1_S. Every entry point takes plain pointers
 * and sizes; device pointers are HIP device addresses, streams are hipStream_t passed as void*
 * (NULL = the default stream). Nothing here allocates behind the caller's back except the
 * governed entry points (vl_device_alloc, the accelerator), which reserve with the Safety
 * Governor first.
 *
 * Status codes: 0 is success, 1..10 are 1 + the reference's vastloom::ErrorCode
 * (include/vastloom/core/status.hpp:10-21), and VL_DECLINED is the accelerator seam's
 * "Ok(false)": the call was refused, outputs are untouched, and the caller runs its CPU path
 * (include/vastloom/inference/deepseek_v4_reference.hpp:437-451). vl_last_error() returns the
 * calling thread's message for the last failure.
 */
#ifndef VASTLOOM_HIP_H
#define VASTLOOM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum vl_status {
    VL_OK = 0,
    VL_INVALID_ARGUMENT = 1,
    VL_INVALID_FORMAT = 2,
    VL_NOT_FOUND = 3,
    VL_PERMISSION_DENIED = 4,
    VL_IO_ERROR = 5,
    VL_INTEGRITY_ERROR = 6,
    VL_UNSAFE_PATH = 7,
    VL_UNSUPPORTED = 8,
    VL_RESOURCE_EXHAUSTED = 9,
    VL_INTERNAL_ERROR = 10,
    VL_DECLINED = 100
} vl_status;

/* GGUF storage type ids (include/vastloom/inference/ggml_quantization.hpp:35-46). */
#define VL_GGML_F32 0u
#define VL_GGML_Q8_0 8u
#define VL_GGML_IQ2_XXS 16u
#define VL_GGML_IQ3_XXS 18u
#define VL_GGML_IQ1_S 19u

/* Bits of the device status word that the kernels raise (read with vl_read_status). */
#define VL_STATUS_NONFINITE_INPUT 1u
#define VL_STATUS_NONFINITE_OUTPUT 2u
#define VL_STATUS_BAD_ROUTE 4u

/* Thread-local message describing the last non-zero status returned on this thread. */
const char* vl_last_error(void);

/* Number of visible HIP devices. Replaces the reference's driver probe for device presence
 * (src/cuda/cuda_driver.cpp:1573-1576). */
int vl_device_count(int* count);

/* Bytes of a GGUF matrix and of its resident (tiled) device form. The tiled form holds the same
 * block bytes rearranged for aligned loads, plus zero rows up to a multiple of 32 rows.
 * Mirrors ggml_storage_bytes (include/vastloom/inference/ggml_quantization.hpp:93-97). */
int vl_matrix_layout(uint32_t ggml_type, uint64_t rows, uint64_t cols, uint64_t* gguf_bytes,
                     uint64_t* device_bytes);

/* GGUF bytes already on the device -> tiled device form (vl_matrix_layout's device_bytes).
 * Replaces the weight upload of CudaMatvecAccelerator::ensure_resident
 * (src/cuda/cuda_matvec_accelerator.cpp:211-218); the tiled form stays resident. */
int vl_pack_matrix(uint32_t ggml_type, uint64_t rows, uint64_t cols, const void* gguf_device,
                   void* tiled_device, void* stream);

/* Decode a tiled matrix to float32 rows [rows][cols], bit-identical to the reference decoders
 * (dequantize_q8_0 / _iq2_xxs / _iq3_xxs / _iq1_s, ggml_quantization.hpp:99-215). */
int vl_dequantize(uint32_t ggml_type, uint64_t rows, uint64_t cols, const void* tiled_device,
                  float* out_device, void* stream);

/* Workspace bytes vl_matvec needs for this shape and token count (1..8) on the current device
 * (the size grows with the device's compute-unit count). */
int vl_matvec_workspace(uint32_t ggml_type, uint64_t rows, uint64_t cols, uint32_t tokens,
                        uint64_t* bytes);

/* y[t][r] = sum_c W[r][c] * x[t][c] for t < tokens (1..8); x is [tokens][cols] float32, y is
 * [tokens][rows] float32, both on the device. The device-resident counterpart of the reference
 * matvecs (matvec_q8_0_f32 / _iq2_xxs_f32 / _iq3_xxs_f32 / _iq1_s_f32,
 * ggml_quantization.hpp:119-215) and of the CudaDriver *_with_transfer launches
 * (src/cuda/cuda_driver.cpp:2083-2180) without their per-call transfers. Asynchronous on the
 * stream; the workspace's status word (vl_read_status) reports non-finite inputs or outputs,
 * which the reference refuses (ggml_quantization.cpp:591-599, :808-813). */
int vl_matvec(uint32_t ggml_type, uint64_t rows, uint64_t cols, const void* tiled_device,
              const float* x_device, uint32_t tokens, float* y_device, void* workspace,
              uint64_t workspace_bytes, void* stream);

/* Synchronizes the stream and returns the status bits recorded in a workspace by the calls
 * issued on it since the workspace was last handed to an entry point. */
int vl_read_status(const void* workspace, void* stream, uint32_t* bits);

/* ---- Expert FFN and MoE layer ------------------------------------------------------------ */

/* Tiled device weights of one expert: gate (w1), up (w3), down (w2). */
typedef struct vl_expert_weights {
    const void* gate;
    const void* up;
    const void* down;
} vl_expert_weights;

/* SwiGLU and combine conventions.
 * VL_SEM_DEEPSEEK: execute_expert + moe_forward (src/inference/deepseek_v4_graph.cpp:1826-1894,
 *   :2129-2266): float64 SwiGLU, gate capped and up clamped at the limit when it is > 0, route
 *   weight applied before the down projection, outputs added in ascending expert id, then the
 *   shared expert (no route weight).
 * VL_SEM_QWEN: qwen38_expert_mlp_q8 + qwen38_moe_block
 *   (src/inference/qwen3_8_flash_next_reference.cpp:1317-1421): silu_f(g) * u in float, expert
 *   outputs scaled by the route weight and added in route-slot order, then the shared expert.
 * VL_SEM_PLAIN: routed_expert_iq1_s_iq3_xxs_f32 (src/inference/ggml_quantization.cpp:1678-1745):
 *   g / (1 + expf(-g)) * u in float, no clamp, no route weight. */
#define VL_SEM_DEEPSEEK 0u
#define VL_SEM_QWEN 1u
#define VL_SEM_PLAIN 2u

/* Routing.
 * VL_ROUTE_LEARNED: top-k of score(logit) + bias, ties to the lower id; weights = selected
 *   scores / their float64 sum * route_scale (deepseek_v4_route_learned_logits,
 *   src/inference/deepseek_v4_reference.cpp:223-255; route_from_indices :80-121).
 * VL_ROUTE_TABLE: expert ids from table_ids[token][slot], weights as above
 *   (deepseek_v4_route_hash_logits, :275-307).
 * VL_ROUTE_SOFTMAX: float64 softmax over the logits, top-k by probability, optional
 *   renormalisation (qwen38_moe_route, src/inference/qwen3_8_flash_next_reference.cpp:1186-1240).
 * VL_ROUTE_GIVEN: ids and weights supplied in given_ids / given_weights (null ids = expert 0,
 *   null weights = 1). */
#define VL_ROUTE_LEARNED 0u
#define VL_ROUTE_TABLE 1u
#define VL_ROUTE_SOFTMAX 2u
#define VL_ROUTE_GIVEN 3u

/* Score of a gate logit: sqrt(softplus(x)) (deepseek_v4_reference.cpp:65-69) or the float64
 * logistic (:71-78). */
#define VL_SCORE_SQRT_SOFTPLUS 0u
#define VL_SCORE_SIGMOID 1u

typedef struct vl_moe_config {
    uint32_t tokens;        /* 1..8 */
    uint32_t width;         /* model width H (multiple of 256) */
    uint32_t intermediate;  /* expert width F */
    uint32_t experts;       /* routed experts E (<= 1024) */
    uint32_t top_k;         /* 1..16 */
    uint32_t gate_type;     /* storage type of gate and up */
    uint32_t down_type;     /* storage type of down */
    uint32_t semantics;
    uint32_t routing;
    uint32_t score_fn;
    uint32_t has_shared;    /* the shared expert is entry E of the expert array */
    uint32_t renormalize;   /* softmax routing only */
    float route_scale;
    float routed_limit;     /* SwiGLU clamp of routed experts, 0 = none */
    float shared_limit;     /* SwiGLU clamp of the shared expert, 0 = none */
} vl_moe_config;

typedef struct vl_moe_inputs {
    const vl_expert_weights* experts;  /* DEVICE array of E (+1 shared) entries */
    const float* router;               /* [E][width] float32, device */
    const float* bias;                 /* [E] selection bias or null (learned routing) */
    const uint32_t* table_ids;         /* [tokens][top_k] (table routing) */
    const uint32_t* given_ids;         /* [tokens][top_k] (given routing) or null */
    const float* given_weights;        /* [tokens][top_k] (given routing) or null */
    const float* x;                    /* [tokens][width] float32, device */
    float* out;                        /* [tokens][width] float32, device */
} vl_moe_inputs;

/* Workspace bytes vl_moe_layer needs for this configuration on the current device. */
int vl_moe_workspace(const vl_moe_config* config, uint64_t* bytes);

/* One MoE layer: router logits (float64 accumulation), routing, the selected experts' SwiGLU
 * FFNs and the combine, all on the stream with no host synchronisation. The status word of the
 * workspace (vl_read_status) reports non-finite values and invalid routes (an out-of-range or
 * repeated expert id); the output is then not meaningful, as the reference would have refused
 * the layer. Replaces the per-matvec device calls of moe_forward / qwen38_moe_block. */
int vl_moe_layer(const vl_moe_config* config, const vl_moe_inputs* inputs, void* workspace,
                 uint64_t workspace_bytes, void* stream);

/* Routing chosen by the last vl_moe_layer on this workspace: ids and weights [tokens][top_k]
 * copied to host memory (synchronizes the stream). */
int vl_moe_read_routes(const vl_moe_config* config, const void* workspace, void* stream,
                       uint32_t* ids_host, float* weights_host);

/* ---- Stage timing (replaces the reference's steady_clock kernel_ms, which timed a whole
 * synchronous call: src/cuda/cuda_matvec_accelerator.cpp:258-311) ---------------------------- */

/* Stages of one vl_moe_layer call, in launch order: router logits and activation limbs;
 * routing with the gate/up projections and SwiGLU; the down projections with the combine. */
#define VL_STAGE_ROUTER 0u
#define VL_STAGE_GATE_UP 1u
#define VL_STAGE_DOWN 2u
#define VL_STAGE_COUNT 3u

typedef struct vl_timeline vl_timeline;

/* A set of HIP events for up to `calls` profiled layer calls. */
int vl_timeline_create(uint32_t calls, vl_timeline** out);
void vl_timeline_destroy(vl_timeline* timeline);

/* vl_moe_layer that also records events around each stage into slot `call` of the timeline. */
int vl_moe_layer_profiled(const vl_moe_config* config, const vl_moe_inputs* inputs,
                          void* workspace, uint64_t workspace_bytes, void* stream,
                          vl_timeline* timeline, uint32_t call);

/* Milliseconds of each stage of a recorded call (the events must have completed). */
int vl_timeline_stage_ms(vl_timeline* timeline, uint32_t call, float* ms /* [VL_STAGE_COUNT] */);

#ifdef __cplusplus
}
#endif

#endif /* VASTLOOM_HIP_H */
