/* vastloom_hip.h - C ABI of the MI355X (gfx950) quantized routed-expert path.
 *
 * This library takes the place of the reference's CUDA device boundary (src/cuda: the
 * CudaDriver/CudaDriverBackend launch entries and the CudaMatvecAccelerator seam) for the
 * GGUF storage types Q8_0, IQ2_XXS, IQ3_XXS and IQ1_S. Every entry point takes plain pointers
 * and sizes; device pointers are HIP device addresses, streams are hipStream_t passed as void*
 * (NULL = the default stream). Nothing here allocates device or pinned memory behind the
 * caller's back: the governed entry points (vl_buffer_alloc, the accelerator) reserve every
 * byte with a Safety Governor before allocating it.
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

/* GGUF storage type ids (include/vastloom/inference/ggml_quantization.hpp:34-45). Q8_0 and the
 * three IQ types are rearranged ("tiled") when they become resident; Q4_K, Q5_K, Q6_K, IQ2_S,
 * MXFP4, BF16 and F32 stay in their GGUF bytes. Every one of them has device dequantize and
 * matvec through the matrix entry points. The MoE layer entry points take any of them for gate/up
 * and down, except a GGUF-layout gate/up with a tiled down (refused as invalid_argument). */
#define VL_GGML_F32 0u
#define VL_GGML_Q8_0 8u
#define VL_GGML_Q4_K 12u
#define VL_GGML_Q5_K 13u
#define VL_GGML_Q6_K 14u
#define VL_GGML_IQ2_XXS 16u
#define VL_GGML_IQ3_XXS 18u
#define VL_GGML_IQ1_S 19u
#define VL_GGML_IQ2_S 22u
#define VL_GGML_BF16 30u
#define VL_GGML_MXFP4 39u

/* Bits of the device status word that the kernels raise (read with vl_read_status). */
#define VL_STATUS_NONFINITE_INPUT 1u
#define VL_STATUS_NONFINITE_OUTPUT 2u
#define VL_STATUS_BAD_ROUTE 4u
#define VL_STATUS_INTERNAL 8u /* reserved: a bounded device-side wait gave up; the output is not valid */

/* Thread-local message describing the last non-zero status returned on this thread. */
const char* vl_last_error(void);

/* Number of visible HIP devices. Replaces the reference's driver probe for device presence
 * (src/cuda/cuda_driver.cpp:1573-1576). */
int vl_device_count(int* count);

/* One visible GPU, as the reference's GpuInfo (include/vastloom/hardware/hardware_probe.hpp:27-35),
 * read from the HIP runtime where the reference runs nvidia-smi (src/hardware/hardware_probe.cpp:
 * 304-311). Temperature and power limit are not reported by the runtime: has_temperature and
 * has_power_limit are 0, as the reference's empty optionals. */
typedef struct vl_gpu_info {
    char backend[16];        /* "hip" */
    char name[128];          /* marketing name */
    char arch[64];           /* e.g. "gfx950:sramecc+:xnack-" */
    char driver_version[32]; /* hipDriverGetVersion, decimal */
    uint64_t total_vram_bytes;
    uint64_t free_vram_bytes; /* hipMemGetInfo on the device, at the call */
    uint32_t compute_units;
    uint32_t has_temperature;
    uint32_t has_power_limit;
    uint32_t reserved;
} vl_gpu_info;
int vl_gpu_probe(int device, vl_gpu_info* out);

/* The runtime policy's VRAM hard limit from a probed GPU (src/safety/runtime_policy.cpp:137-141):
 * min(80 % of total, free - 1 GiB) when more than 1 GiB is free, else 0 (no VRAM budget). The 80 %
 * is the reference's percentage() (src/core/bytes.cpp:99-107): a long double product, truncated. */
int vl_vram_hard_limit(uint64_t total_vram_bytes, uint64_t free_vram_bytes, uint64_t* limit);

/* Bytes of a GGUF matrix and of its resident (tiled) device form. The tiled form holds the same
 * block bytes rearranged for aligned loads, plus zero rows up to a multiple of 32 rows; for the
 * GGUF-layout types it is the GGUF matrix itself (device_bytes == gguf_bytes).
 * Mirrors ggml_storage_bytes (include/vastloom/inference/ggml_quantization.hpp:93-97). */
int vl_matrix_layout(uint32_t ggml_type, uint64_t rows, uint64_t cols, uint64_t* gguf_bytes,
                     uint64_t* device_bytes);

/* GGUF bytes already on the device -> tiled device form (vl_matrix_layout's device_bytes).
 * Replaces the weight upload of CudaMatvecAccelerator::ensure_resident
 * (src/cuda/cuda_matvec_accelerator.cpp:211-218); the tiled form stays resident. */
int vl_pack_matrix(uint32_t ggml_type, uint64_t rows, uint64_t cols, const void* gguf_device,
                   void* tiled_device, void* stream);

/* Decode a tiled matrix to float32 rows [rows][cols], bit-identical to the reference decoders
 * (dequantize_q8_0 / _q4_k / _q5_k / _q6_k / _iq2_xxs / _iq2_s / _iq3_xxs / _iq1_s / _mxfp4 / _bf16 /
 * _f32_le, ggml_quantization.hpp:99-266). */
int vl_dequantize(uint32_t ggml_type, uint64_t rows, uint64_t cols, const void* tiled_device,
                  float* out_device, void* stream);

/* Workspace bytes vl_matvec needs for this shape and token count (1..8) on the current device
 * (the size grows with the device's compute-unit count). */
int vl_matvec_workspace(uint32_t ggml_type, uint64_t rows, uint64_t cols, uint32_t tokens,
                        uint64_t* bytes);

/* y[t][r] = sum_c W[r][c] * x[t][c] for t < tokens (1..8); x is [tokens][cols] float32, y is
 * [tokens][rows] float32, both on the device. The device-resident counterpart of the reference
 * matvecs (matvec_q8_0_f32 / _iq2_xxs_f32 / _iq3_xxs_f32 / _iq1_s_f32 and, for the GGUF-layout
 * types, matvec_q4_k_f32 / _q5_k / _q6_k / _iq2_s / _mxfp4 / _bf16 / _f32_le_f32,
 * ggml_quantization.hpp:99-266) and of the CudaDriver *_with_transfer launches
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
 *   null weights = 1).
 * Refused (VL_STATUS_BAD_ROUTE): an expert id out of range; a non-finite logit or selection bias
 * (require_finite, deepseek_v4_reference.cpp:161, :235-238); selected weights that cannot be
 * normalised. Divergence: a token whose table or given ids repeat an expert is refused here,
 * while the reference's route_from_indices accepts it and adds each slot's output
 * (deepseek_v4_graph.cpp:2211-2228); every route the reference's own routers produce has
 * distinct experts. */
#define VL_ROUTE_LEARNED 0u
#define VL_ROUTE_TABLE 1u
#define VL_ROUTE_SOFTMAX 2u
#define VL_ROUTE_GIVEN 3u

/* Score of a gate logit: sqrt(softplus(x)) (deepseek_v4_reference.cpp:65-69) or the float64
 * logistic (:71-78). */
#define VL_SCORE_SQRT_SOFTPLUS 0u
#define VL_SCORE_SIGMOID 1u

typedef struct vl_moe_config {
    uint32_t tokens;        /* 1..1024; above 8 the grouped path (at most 16384 token-expert
                             * assignments and 1792 groups of up to 8 tokens) */
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
 * FFNs and the combine, all on the stream with no host synchronisation. Up to 8 tokens share
 * each expert's weight pass; more tokens take the grouped path, which splits each selected
 * expert's tokens, in ascending order, into groups and streams the expert's weights once per run
 * of up to 32 tokens for IQ2_XXS (up to 8 for the other types) (moe_forward's per-expert token
 * batches, deepseek_v4_graph.cpp:2211-2229). The status word of the workspace (vl_read_status)
 * reports non-finite values and refused routes (see Routing); the output is then not
 * meaningful, as the reference would have refused
 * the layer. Replaces the per-matvec device calls of moe_forward / qwen38_moe_block. */
int vl_moe_layer(const vl_moe_config* config, const vl_moe_inputs* inputs, void* workspace,
                 uint64_t workspace_bytes, void* stream);

/* Routes every token of a layer without running its experts: the router logits, scores and
 * selection (learned, table or softmax routing; not VL_ROUTE_GIVEN) of vl_moe_layer, with the routes
 * left in the workspace for vl_moe_read_routes and refused tokens in its status word
 * (vl_read_status). inputs->experts is not read (may be NULL); out is not written. The reference
 * routes a layer before its provider acquires the selected experts (moe_forward's router-first
 * batch, src/inference/deepseek_v4_graph.cpp:1971-2029): a caller whose experts live in host memory
 * routes first, makes the selected experts resident, then runs vl_moe_layer with
 * VL_ROUTE_GIVEN and these routes. */
int vl_moe_route(const vl_moe_config* config, const vl_moe_inputs* inputs, void* workspace,
                 uint64_t workspace_bytes, void* stream);

/* vl_moe_layer without a caller-owned workspace, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. The workspace is a fixed 64 MiB array in the library's device
 * memory, one per device, looked up (never allocated) on the first call on that device; layers
 * whose workspace would exceed it are refused with VL_RESOURCE_EXHAUSTED before anything is
 * launched (single-token and small multi-token layers fit; large prefill batches do not). Every
 * call on one device shares that device's array, so calls that overlap on one device (on
 * different streams or from different threads without ordering) race and give undefined results.
 * Each call clears what it needs zeroed itself, on the stream. */
int vl_moe_layer_noalloc(const vl_moe_config* config, const vl_moe_inputs* inputs, void* stream);

/* Synchronizes the stream and returns the status bits of the last vl_moe_layer_noalloc on the
 * current device (as vl_read_status does for a caller's workspace). No counterpart in the
 * reference; for the same callers. */
int vl_moe_noalloc_status(void* stream, uint32_t* bits);

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

/* With enabled, later profiled calls record, instead of stage marks, events that the launch
 * places around each stage's kernel execution (such launches lengthen the gaps between kernels,
 * so the two are recorded in separate calls). */
int vl_timeline_set_kernel_brackets(vl_timeline* timeline, int enabled);

/* Milliseconds of each stage's kernel of a call recorded with kernel brackets: the kernel's own
 * execution, without the gaps between launches. Stages of several kernels (layers of more than 8
 * tokens) and single-launch layers report their stage time. Like the stage times, this replaces
 * the steady-clock kernel_ms of cuda_matvec_accelerator.cpp:258-311. */
int vl_timeline_kernel_ms(vl_timeline* timeline, uint32_t call, float* ms /* [VL_STAGE_COUNT] */);

/* ---- Safety Governor ------------------------------------------------------------------------
 * A native counterpart of safety::ResourceGovernor (src/safety/resource_governor.cpp:19-214,
 * include/vastloom/safety/resource_governor.hpp:15-117): per-kind hard budgets, an optional
 * aggregate host-memory budget, and a safety state that refuses new reservations when critical
 * or emergency. The allocating entry points below see a Governor only through vl_governor_ops,
 * so a caller that owns its own ResourceGovernor passes that instead (INTEGRATION.md shows the
 * adapter). */

#define VL_KIND_RAM 0u      /* ResourceKind::ram */
#define VL_KIND_VRAM 1u     /* ResourceKind::vram: device memory */
#define VL_KIND_STAGING 2u  /* ResourceKind::staging: pinned host memory */
#define VL_KIND_SCRATCH 3u  /* ResourceKind::scratch */

#define VL_STATE_NORMAL 0u
#define VL_STATE_PRESSURE 1u
#define VL_STATE_CRITICAL 2u
#define VL_STATE_EMERGENCY 3u

typedef struct vl_resource_limits { /* ResourceLimits (resource_governor.hpp:29-42) */
    uint64_t host_memory_hard_limit;  /* 0 = per-kind budgets only */
    uint64_t ram_hard_limit;
    uint64_t vram_hard_limit;
    uint64_t staging_hard_limit;
    uint64_t scratch_hard_limit;
    uint64_t minimum_system_ram_available;
    uint64_t minimum_storage_available;
    double pressure_ratio;  /* clamped to [0.10, 0.99] */
    double critical_ratio;  /* clamped to [pressure_ratio + 0.01, 1.0] */
    uint32_t recovery_samples;
} vl_resource_limits;

typedef struct vl_runtime_pressure { /* RuntimePressure (resource_governor.hpp:44-48) */
    uint64_t system_ram_available;
    uint64_t gpu_vram_available;
    uint64_t storage_available;
} vl_runtime_pressure;

typedef struct vl_governor_snapshot {
    uint32_t state;
    uint32_t recovery_counter;
    uint64_t reserved[4]; /* by VL_KIND_* */
} vl_governor_snapshot;

typedef struct vl_governor vl_governor;

/* The reference's ResourceLimits defaults (2 GiB RAM and 20 GiB storage reserves, ratios 0.82 and
 * 0.93, 3 recovery samples) with every hard budget 0, i.e. nothing may be reserved yet. */
void vl_resource_limits_default(vl_resource_limits* limits);
int vl_governor_create(const vl_resource_limits* limits, vl_governor** out);
void vl_governor_destroy(vl_governor* governor);
/* ResourceGovernor::try_reserve (resource_governor.cpp:64-105): zero bytes is invalid_argument;
 * the critical and emergency states, a zero or exceeded kind budget and an exceeded aggregate
 * host budget are resource_exhausted. On success *reservation is a non-zero id. */
int vl_governor_try_reserve(vl_governor* governor, uint32_t kind, uint64_t bytes, const char* tag,
                            uint64_t* reservation);
/* Reservation::release: the bytes return to the budget. */
int vl_governor_release(vl_governor* governor, uint64_t reservation);
/* Reservation::abandon_accounting_on_external_release_failure: the id is dropped and its bytes
 * stay charged (memory that could not be freed must not be handed out again). */
int vl_governor_abandon(vl_governor* governor, uint64_t reservation);
/* ResourceGovernor::update_pressure (resource_governor.cpp:107-196). */
int vl_governor_update_pressure(vl_governor* governor, const vl_runtime_pressure* pressure,
                                uint32_t* state);
int vl_governor_snapshot_get(const vl_governor* governor, vl_governor_snapshot* out);

/* A Governor as the allocating entry points see it. */
typedef struct vl_governor_ops {
    void* ctx;
    /* Returns a vl_status; on VL_OK *reservation is a non-zero id. */
    int (*try_reserve)(void* ctx, uint32_t kind, uint64_t bytes, const char* tag,
                       uint64_t* reservation);
    void (*release)(void* ctx, uint64_t reservation);
    void (*abandon)(void* ctx, uint64_t reservation);
} vl_governor_ops;

/* The ops of a native Governor (valid while the Governor lives). */
vl_governor_ops vl_governor_as_ops(vl_governor* governor);

/* ---- Governed allocations -------------------------------------------------------------------
 * CudaDriver::allocate / CudaAllocation (src/cuda/cuda_driver.cpp:2881-3010): reserve with the
 * Governor, check that the device keeps min_free_after bytes free after the allocation, then
 * allocate; release frees and returns the bytes, and a failed free keeps the bytes charged and
 * quarantines the handle. */

typedef struct vl_buffer vl_buffer;

/* kind VL_KIND_VRAM: device memory on `device`; VL_KIND_STAGING: pinned host memory (hipHostMalloc).
 * Refusals (the Governor's, or too little free device memory) return VL_RESOURCE_EXHAUSTED. */
int vl_buffer_alloc(const vl_governor_ops* governor, uint32_t kind, int device, uint64_t bytes,
                    uint64_t min_free_after, const char* tag, vl_buffer** out);
void* vl_buffer_ptr(const vl_buffer* buffer);
uint64_t vl_buffer_bytes(const vl_buffer* buffer);
int vl_buffer_free(vl_buffer* buffer);

/* ---- Matvec accelerator with device residency -------------------------------------------------
 * The DeepseekV4MatvecAccelerator seam (include/vastloom/inference/deepseek_v4_reference.hpp:
 * 437-451) as CudaMatvecAccelerator implements it (src/cuda/cuda_matvec_accelerator.cpp:102-314,
 * include/vastloom/cuda/cuda_matvec_accelerator.hpp:17-113): matrices become resident on first
 * use, keyed by cache identity; matrices that will not recur are evicted first, then the least
 * recently used; anything this cannot take is declined (VL_DECLINED, output untouched). Uploads
 * go through Governor-reserved pinned staging and hipMemcpyAsync on a copy stream, in row
 * ranges, each range packed into the resident tiled form on the compute stream. */

typedef struct vl_packed_matrix { /* DeepseekV4PackedMatrix (deepseek_v4_reference.hpp:104-141) */
    uint32_t ggml_type;
    uint32_t recurring;           /* the next pass asks for these weights again */
    uint64_t rows;
    uint64_t logical_columns;
    uint64_t storage_columns;
    const void* encoded;          /* host GGUF bytes (the descriptor's payload) */
    uint64_t encoded_bytes;
    uint64_t cache_identity;      /* 0 = do not cache: declined */
} vl_packed_matrix;

typedef struct vl_accel_options { /* CudaMatvecAcceleratorOptions (.hpp:17-30) */
    int device_ordinal;
    uint32_t experts_only;            /* decline recurring matrices */
    uint64_t minimum_free_vram_after; /* default 1 GiB */
    uint64_t maximum_resident_bytes;  /* default 6 GiB */
    uint64_t maximum_matrices;        /* default 512 */
    uint64_t staging_bytes;           /* pinned staging for uploads, two slots; default 64 MiB */
} vl_accel_options;

#define VL_ACCEL_TYPE_SLOTS 8u

typedef struct vl_accel_stats { /* CudaMatvecAcceleratorStats (.hpp:32-54) */
    uint64_t offered, accelerated, declined, evicted, declined_recurring;
    uint64_t resident_matrices, resident_bytes, uploaded_bytes;
    uint32_t declined_type[VL_ACCEL_TYPE_SLOTS];     /* storage types declined for having no kernel */
    uint64_t declined_by_type[VL_ACCEL_TYPE_SLOTS];  /* ... and how often (first 8 types seen) */
    double kernel_ms, upload_ms;
} vl_accel_stats;

/* Device operations of an accelerator: the default is HIP on options->device_ordinal. A test can
 * pass its own (CudaDriver::from_backend_for_testing, src/cuda/cuda_driver.cpp:2909-2916). Every
 * function returns a vl_status. */
typedef struct vl_accel_backend {
    void* ctx;
    int (*free_memory)(void* ctx, int device, uint64_t* free_bytes);
    int (*allocate)(void* ctx, uint32_t kind, int device, uint64_t bytes, void** ptr);
    int (*release)(void* ctx, uint32_t kind, void* ptr);
    /* GGUF host bytes -> tiled resident form at `tiled`, through `staging` (pinned, two slots of
     * staging_bytes / 2) and `scratch` (device, two slots of the same size). */
    int (*upload)(void* ctx, uint32_t type, uint64_t rows, uint64_t cols, const void* gguf,
                  void* tiled, void* staging, void* scratch, uint64_t staging_bytes);
    /* Device bytes matvec needs for x, y and its workspace at this shape. */
    int (*io_bytes)(void* ctx, uint32_t type, uint64_t rows, uint64_t cols, uint64_t* bytes);
    /* y = W x with host x and y, through the device buffer io (io_bytes long); synchronous. A
     * non-finite x or y is VL_INVALID_ARGUMENT, as the reference's matvec refuses it. */
    int (*matvec)(void* ctx, uint32_t type, uint64_t rows, uint64_t cols, const void* tiled,
                  const float* x, float* y, void* io, uint64_t io_bytes);
} vl_accel_backend;

typedef struct vl_accel vl_accel;

void vl_accel_options_default(vl_accel_options* options);
/* backend may be NULL (HIP). Reserves and allocates the staging buffers. */
int vl_accel_create(const vl_accel_options* options, const vl_governor_ops* governor,
                    const vl_accel_backend* backend, vl_accel** out);
/* Releases every resident matrix and the staging buffers. */
int vl_accel_destroy(vl_accel* accel);
/* DeepseekV4MatvecAccelerator::matvec: input has storage_columns floats, output rows floats,
 * both host memory. VL_OK: output written; VL_DECLINED: output untouched; else an error. */
int vl_accel_matvec(vl_accel* accel, const vl_packed_matrix* matrix, const float* input,
                    uint64_t input_len, float* output, uint64_t output_len);
/* Makes the matrix resident without multiplying (upload on first sight). VL_OK or VL_DECLINED.
 * On VL_OK the resident form is complete: the upload has finished on the device. */
int vl_accel_prefetch(vl_accel* accel, const vl_packed_matrix* matrix);
/* 1 when these weights are resident now, else 0 (CudaMatvecAccelerator::holds). */
int vl_accel_holds(const vl_accel* accel, uint64_t cache_identity);
/* Device address of a resident matrix's tiled form (for vl_expert_weights), or VL_NOT_FOUND. The
 * address stays valid until the accelerator drops the matrix: a later vl_accel_matvec or
 * vl_accel_prefetch that needs room may evict it, and vl_accel_destroy releases it. Work that
 * reads it must have completed before such a call. */
int vl_accel_resident_matrix(const vl_accel* accel, uint64_t cache_identity, const void** tiled);
int vl_accel_stats_get(const vl_accel* accel, vl_accel_stats* out);

#ifdef __cplusplus
}
#endif

#endif /* VASTLOOM_HIP_H */
