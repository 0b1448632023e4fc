/* CPU oracle for the quantized routed-expert path. TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU arithmetic for the path, used as the checker
 * for the HIP product (tests, smoke, and the CPU-baseline leg of the benchmark). Nothing in the
 * product links, loads or calls this library. Every function names the reference code it
 * follows; paths are relative to the reference tree.
 *
 * Status codes: 0 = ok, otherwise 1 + vastloom::ErrorCode (include/vastloom/core/status.hpp:10-21).
 *
 * Parity pins (see tests/test_oracle_*.py): every decoder and matvec is pinned by the reference's
 * committed known-answer vectors (tests/test_main.cpp:863-973, :1295-1460, :1832-1907) and, where
 * the reference sources build in the container, by bit-equality against oracle/_ref. Routing and
 * the clamped SwiGLU are pinned by tests/fixtures/deepseek_v4_operators.json; softmax top-k by
 * tests/test_main.cpp:3966-3990; fp16 decode exhaustively against numpy. The sigmoid scoring
 * option and the MoE combine loops have no reference vector: they are pinned against closed
 * forms and a float64 numpy restatement (tests/test_oracle_layers.py).
 */
#ifndef VL_ORACLE_H
#define VL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    VLO_OK = 0,
    VLO_E_INVALID_ARGUMENT = 1,
    VLO_E_INVALID_FORMAT = 2,
    VLO_E_UNSUPPORTED = 8,
    VLO_E_RESOURCE_EXHAUSTED = 9,
    VLO_E_INTERNAL = 10,
};

/* GGML storage type ids (include/vastloom/inference/ggml_quantization.hpp:34-45). */
enum {
    VLO_F32 = 0, VLO_Q8_0 = 8, VLO_Q4_K = 12, VLO_Q5_K = 13, VLO_Q6_K = 14, VLO_IQ2_XXS = 16,
    VLO_IQ3_XXS = 18, VLO_IQ1_S = 19, VLO_IQ2_S = 22, VLO_BF16 = 30, VLO_MXFP4 = 39
};

enum { VLO_SCORE_SQRT_SOFTPLUS = 0, VLO_SCORE_SIGMOID = 1 };

/* Default element ceiling of QuantizedKernelLimits (ggml_quantization.hpp:49). */
#define VLO_DEFAULT_MAX_ELEMENTS 64000000u

typedef struct vlo_matrix {
    uint32_t type;
    const uint8_t* data;
    size_t bytes;
} vlo_matrix;

int vlo_codebooks_ok(void);
float vlo_fp16_to_f32(uint16_t value);
int vlo_block_layout(uint32_t type, size_t* block_elements, size_t* block_bytes);
int vlo_storage_bytes(uint32_t type, size_t rows, size_t cols, size_t max_elements, size_t* bytes);

int vlo_dequantize(uint32_t type, const uint8_t* encoded, size_t encoded_bytes, float* out,
                   size_t out_elements, size_t max_elements);
int vlo_dequantize_row(uint32_t type, const uint8_t* encoded, size_t encoded_bytes, size_t rows,
                       size_t cols, size_t row, float* out, size_t out_elements);
int vlo_matvec(uint32_t type, const uint8_t* encoded, size_t encoded_bytes, size_t rows,
               size_t cols, const float* x, size_t x_len, float* y, size_t y_len,
               size_t max_elements, unsigned max_threads);

int vlo_routed_expert_iq1s_iq3xxs(const vlo_matrix* gate, const vlo_matrix* up,
                                  const vlo_matrix* down, size_t width, size_t expert_width,
                                  const float* x, float* y);
int vlo_expert_deepseek(const vlo_matrix* w1, const vlo_matrix* w3, const vlo_matrix* w2,
                        size_t width, size_t intermediate, const float* x, size_t tokens,
                        const float* routing, float swiglu_limit, float* y, unsigned threads);
int vlo_expert_qwen(const vlo_matrix* gate, const vlo_matrix* up, const vlo_matrix* down,
                    size_t width, size_t intermediate, const float* x, float* y,
                    unsigned threads);

float vlo_sqrt_softplus(float value);
float vlo_sigmoid(float value);
float vlo_silu_f(float value);
int vlo_linear_f64(const float* weight, const float* x, size_t tokens, size_t in_width,
                   size_t out_width, float* out);
int vlo_route_learned(const float* logits, const float* bias, size_t tokens, size_t experts,
                      size_t top_k, float route_scale, int score_fn, uint32_t* indices,
                      float* weights);
int vlo_route_hash(const float* logits, const uint32_t* token_ids, const uint32_t* table,
                   size_t tokens, size_t vocabulary, size_t experts, size_t top_k,
                   float route_scale, int score_fn, uint32_t* indices, float* weights);
int vlo_route_softmax(const float* logits, size_t experts, size_t top_k, int renormalize,
                      uint32_t* indices, float* weights);

int vlo_moe_deepseek(const float* x, size_t tokens, size_t width, size_t intermediate,
                     size_t experts, size_t top_k, const uint32_t* indices,
                     const float* weights, const vlo_matrix* expert_matrices,
                     const vlo_matrix* shared, float routed_limit, float shared_limit,
                     float* out, unsigned threads);
int vlo_moe_qwen(const float* x, size_t width, size_t intermediate, size_t experts,
                 size_t top_k, const uint32_t* indices, const float* weights,
                 const vlo_matrix* expert_matrices, const vlo_matrix* shared, float* out,
                 unsigned threads);

#ifdef __cplusplus
}
#endif

#endif /* VL_ORACLE_H */
