// Internal host-side interface of the HIP kernels (C++). The public C ABI in include/vastloom_hip.h
// is implemented on top of these in vl_capi.cpp.
#ifndef VL_KERNELS_H
#define VL_KERNELS_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vl_layout.h"

namespace vl {

// Status bits a kernel may raise in the caller's device status word.
constexpr uint32_t kStatusNonFiniteInput = 1u;
constexpr uint32_t kStatusNonFiniteOutput = 2u;
constexpr uint32_t kStatusBadRoute = 4u;

// Int8 limb encoding of float activations: per token, x * 2^e rounded to an int32 of at most
// 2^30 in magnitude, split into four signed base-256 digits. Stored [group][token slot][limb][32
// columns] so that one 16-byte load is one lane's MFMA A fragment. Token slots are padded to a
// power of two no larger than 8.
__host__ __device__ inline uint32_t limb_slots(uint32_t tokens) {
    return tokens <= 1 ? 1u : tokens <= 2 ? 2u : tokens <= 4 ? 4u : 8u;
}
__host__ __device__ inline uint64_t limb_bytes(uint32_t cols, uint32_t tokens) {
    return (uint64_t)(cols / 32u) * limb_slots(tokens) * 128u;
}

// One quantized matvec of a batch: y[token][row] = W x[token] for up to eight tokens.
struct QmvJob {
    const uint8_t* w;    // tiled matrix
    const int8_t* xl;    // limbs of the input tokens
    const int* xe;       // per-token exponents
    float* y;            // output, token-major with stride y_stride
    uint32_t rows, cols, tokens, y_stride;
};

// Jobs reach the kernel either inline in its arguments (host-built batches of up to
// kInlineJobs) or through a device array (batches built on the device, e.g. by routing).
constexpr uint32_t kInlineJobs = 16;
struct QmvBatch {
    QmvJob inline_jobs[kInlineJobs];
    const QmvJob* device_jobs;  // used when non-null
};

hipError_t launch_pack(const vl_tiled_layout& L, const uint8_t* gguf, uint8_t* tiled,
                       hipStream_t stream);
hipError_t launch_dequant(const vl_tiled_layout& L, const uint8_t* tiled, float* out,
                          hipStream_t stream);
// x: [sets][tokens][cols] with token stride x_stride and set stride set_stride (floats); limbs
// of set s at xl + s * limb_bytes(cols, tokens), exponents at xe + s * 8.
hipError_t launch_prep_limbs(const float* x, uint32_t sets, uint32_t tokens, uint32_t cols,
                             uint64_t x_stride, uint64_t set_stride, int8_t* xl, int* xe,
                             uint32_t* status, hipStream_t stream);
// Every job has the given type, at most max_tiles tiles and at most max_cols columns; njobs jobs
// are read from the batch.
hipError_t launch_qmv(uint32_t type, uint32_t token_slots, const QmvBatch& batch, uint32_t njobs,
                      uint32_t max_tiles, uint32_t max_cols, uint32_t* status, hipStream_t stream);
hipError_t launch_fill_u32(uint32_t* dst, uint32_t count, uint32_t value, hipStream_t stream);

}  // namespace vl

#endif  // VL_KERNELS_H
