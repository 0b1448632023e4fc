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

/* Workspace bytes vl_matvec needs for this shape and token count (1..8). */
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

#ifdef __cplusplus
}
#endif

#endif /* VASTLOOM_HIP_H */
