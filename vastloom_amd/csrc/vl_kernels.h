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
constexpr uint32_t kStatusInternal = 8u;  // reserved: a bounded wait inside a layer kernel gave up

// Int8 limb encoding of float activations: per token and 256-column block, x * 2^e rounded to
// an int32 of at most 2^30 in magnitude, split into four signed base-256 digits. Stored
// [group of 32 columns][token slot][limb][32 columns] so that one 16-byte load is one lane's
// MFMA A fragment. Token slots are padded to a power of two no larger than 8.
__host__ __device__ inline uint32_t limb_slots(uint32_t tokens) {
    return tokens <= 1 ? 1u : tokens <= 2 ? 2u : tokens <= 4 ? 4u : 8u;
}
__host__ __device__ inline uint64_t limb_bytes(uint32_t cols, uint32_t tokens) {
    return (uint64_t)(cols / 32u) * limb_slots(tokens) * 128u;
}

// Persistent blocks of the stream kernels on the current device (one per CU), or 0.
uint32_t stream_blocks();
// Raises a kernel's dynamic LDS limit once per process.
hipError_t ensure_dynamic_lds(const void* kernel, uint32_t bytes);

hipError_t launch_pack(const vl_tiled_layout& L, const uint8_t* gguf, uint8_t* tiled,
                       hipStream_t stream);
// Rows [row0, row1) of the padded matrix (row1 <= rows_padded); gguf_row0 holds the GGUF bytes
// of rows row0 .. min(row1, rows) - 1.
hipError_t launch_pack_rows(const vl_tiled_layout& L, const uint8_t* gguf_row0, uint8_t* tiled,
                            uint32_t row0, uint32_t row1, hipStream_t stream);
hipError_t launch_dequant(const vl_tiled_layout& L, const uint8_t* tiled, float* out,
                          hipStream_t stream);

// One quantized matvec call, y[token][row] = W x[token] for up to eight tokens. The workspace
// (matvec_workspace_bytes) starts with the status word; its handoff counters are cleared by
// the call itself.
uint64_t matvec_workspace_bytes(uint32_t type, uint32_t rows, uint32_t cols, uint32_t tokens,
                                uint32_t blocks);
hipError_t launch_matvec(const vl_tiled_layout& L, const uint8_t* w, const float* x,
                         uint32_t tokens, float* y, uint8_t* workspace, uint32_t blocks,
                         hipStream_t stream);

// The GGUF-layout types (vl_type_tiled() false), in vl_gguf.hip; launch_pack_rows,
// launch_dequant and launch_matvec hand these types on to them.
hipError_t launch_gguf_copy_rows(const vl_tiled_layout& L, const uint8_t* gguf_row0, uint8_t* dst,
                                 uint32_t row0, uint32_t row1, hipStream_t stream);
hipError_t launch_gguf_dequant(const vl_tiled_layout& L, const uint8_t* w, float* out,
                               hipStream_t stream);
hipError_t launch_gguf_matvec(const vl_tiled_layout& L, const uint8_t* w, const float* x,
                              uint32_t tokens, float* y, uint8_t* workspace, hipStream_t stream);

}  // namespace vl

#endif  // VL_KERNELS_H
