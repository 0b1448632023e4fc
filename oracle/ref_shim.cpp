// C entry points over the reference's own CPU implementation. TEST INFRASTRUCTURE ONLY.
//
// Compiled by oracle/Makefile together with the reference sources where they lie in the
// reference tree (never copied into this repository) into oracle/_ref/libvlref.so. Tests use
// it to pin the C restatement in vl_oracle.c; the benchmark may time it as the CPU baseline.
// Each wrapper forwards to one public reference function and maps its Result to the oracle's
// status codes (0 = ok, else 1 + ErrorCode).
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <span>
#include <vector>

#include "vastloom/inference/deepseek_v4_reference.hpp"
#include "vastloom/inference/ggml_quantization.hpp"
#include "vastloom/inference/qwen3_8_flash_next_reference.hpp"

#define VLR_EXPORT extern "C" __attribute__((visibility("default")))

namespace vi = vastloom::inference;

namespace {

template <typename R>
int status(const R& result) {
    return result ? 0 : 1 + static_cast<int>(result.error().code);
}

std::span<const std::byte> bytes(const std::uint8_t* p, std::size_t n) {
    return {reinterpret_cast<const std::byte*>(p), n};
}

}  // namespace

VLR_EXPORT int vlr_dequantize(std::uint32_t type, const std::uint8_t* enc, std::size_t enc_bytes,
                              float* out, std::size_t out_elements, std::size_t max_elements) {
    vi::QuantizedKernelLimits limits;
    limits.max_elements = max_elements;
    std::span<float> o(out, out_elements);
    switch (type) {
        case vi::kGgmlTypeQ8_0: return status(vi::dequantize_q8_0(bytes(enc, enc_bytes), o, limits));
        case vi::kGgmlTypeIq2Xxs:
            return status(vi::dequantize_iq2_xxs(bytes(enc, enc_bytes), o, limits));
        case vi::kGgmlTypeIq3Xxs:
            return status(vi::dequantize_iq3_xxs(bytes(enc, enc_bytes), o, limits));
        case vi::kGgmlTypeIq1S: return status(vi::dequantize_iq1_s(bytes(enc, enc_bytes), o, limits));
        case vi::kGgmlTypeQ4K: return status(vi::dequantize_q4_k(bytes(enc, enc_bytes), o, limits));
        case vi::kGgmlTypeQ5K: return status(vi::dequantize_q5_k(bytes(enc, enc_bytes), o, limits));
        case vi::kGgmlTypeQ6K: return status(vi::dequantize_q6_k(bytes(enc, enc_bytes), o, limits));
        case vi::kGgmlTypeMxfp4: return status(vi::dequantize_mxfp4(bytes(enc, enc_bytes), o, limits));
        case vi::kGgmlTypeBf16: return status(vi::dequantize_bf16(bytes(enc, enc_bytes), o, limits));
        case vi::kGgmlTypeIq2S: return status(vi::dequantize_iq2_s(bytes(enc, enc_bytes), o, limits));
        default: return 1 + static_cast<int>(vastloom::ErrorCode::unsupported);
    }
}

VLR_EXPORT int vlr_matvec(std::uint32_t type, const std::uint8_t* enc, std::size_t enc_bytes,
                          std::size_t rows, std::size_t cols, const float* x, float* y,
                          std::size_t max_elements, unsigned threads) {
    vi::QuantizedKernelLimits limits;
    limits.max_elements = max_elements;
    limits.max_threads = threads;
    std::vector<float> scratch(rows);
    return status(vi::matvec_ggml_f32_transactional(type, bytes(enc, enc_bytes), rows, cols,
                                                    std::span<const float>(x, cols), scratch,
                                                    std::span<float>(y, rows), limits));
}

VLR_EXPORT int vlr_routed_expert_iq1s_iq3xxs(const std::uint8_t* gate, const std::uint8_t* up,
                                             const std::uint8_t* down, std::size_t width,
                                             std::size_t expert_width, const float* x, float* y) {
    const std::size_t gate_bytes = expert_width * width / 256 * 50;
    const std::size_t down_bytes = width * expert_width / 256 * 98;
    std::vector<float> g(expert_width), u(expert_width), d(width);
    return status(vi::routed_expert_iq1_s_iq3_xxs_f32(
        bytes(gate, gate_bytes), bytes(up, gate_bytes), bytes(down, down_bytes),
        std::span<const float>(x, width), vi::RoutedExpertScratch{g, u, d},
        std::span<float>(y, width)));
}

VLR_EXPORT int vlr_route_learned(const float* logits, const float* bias, std::size_t tokens,
                                 std::size_t experts, std::size_t top_k, float route_scale,
                                 std::uint32_t* indices, float* weights) {
    auto r = vi::deepseek_v4_route_learned_logits(
        std::span<const float>(logits, tokens * experts), std::span<const float>(bias, experts),
        tokens, experts, top_k, route_scale);
    if (!r) return status(r);
    std::memcpy(indices, r.value().indices.data(), tokens * top_k * sizeof(std::uint32_t));
    std::memcpy(weights, r.value().weights.data(), tokens * top_k * sizeof(float));
    return 0;
}

VLR_EXPORT int vlr_route_hash(const float* logits, const std::uint32_t* token_ids,
                              const std::uint32_t* table, std::size_t tokens,
                              std::size_t vocabulary, std::size_t experts, std::size_t top_k,
                              float route_scale, std::uint32_t* indices, float* weights) {
    auto r = vi::deepseek_v4_route_hash_logits(
        std::span<const float>(logits, tokens * experts),
        std::span<const std::uint32_t>(token_ids, tokens),
        std::span<const std::uint32_t>(table, vocabulary * top_k), tokens, vocabulary, experts,
        top_k, route_scale);
    if (!r) return status(r);
    std::memcpy(indices, r.value().indices.data(), tokens * top_k * sizeof(std::uint32_t));
    std::memcpy(weights, r.value().weights.data(), tokens * top_k * sizeof(float));
    return 0;
}

VLR_EXPORT int vlr_expert_swiglu_f32(const float* x, const float* gate_w, const float* down_w,
                                     const float* up_w, const float* routing,
                                     std::size_t tokens, std::size_t width,
                                     std::size_t intermediate, float limit, float* y) {
    auto r = vi::deepseek_v4_expert_swiglu(
        std::span<const float>(x, tokens * width),
        std::span<const float>(gate_w, intermediate * width),
        std::span<const float>(down_w, width * intermediate),
        std::span<const float>(up_w, intermediate * width),
        routing ? std::span<const float>(routing, tokens) : std::span<const float>(), tokens,
        width, intermediate, limit);
    if (!r) return status(r);
    std::memcpy(y, r.value().data(), tokens * width * sizeof(float));
    return 0;
}

VLR_EXPORT int vlr_qwen_route(const float* hidden, const float* router, std::size_t width,
                              std::uint32_t experts, std::uint32_t top_k, int renormalize,
                              std::uint32_t* indices, float* weights, float* logits) {
    auto r = vi::qwen38_moe_route(std::span<const float>(hidden, width),
                                  std::span<const float>(router, width * experts), experts,
                                  top_k, renormalize != 0);
    if (!r) return status(r);
    std::memcpy(indices, r.value().indices.data(), top_k * sizeof(std::uint32_t));
    std::memcpy(weights, r.value().weights.data(), top_k * sizeof(float));
    std::memcpy(logits, r.value().logits.data(), experts * sizeof(float));
    return 0;
}

VLR_EXPORT int vlr_qwen_expert_mlp_q8(const std::uint8_t* gate, const std::uint8_t* up,
                                      const std::uint8_t* down, std::uint32_t width,
                                      std::uint32_t intermediate, const float* x, float* y) {
    const std::size_t n = static_cast<std::size_t>(width) * intermediate / 32 * 34;
    vi::Qwen38OwnedExpertQ8 expert;
    expert.gate.assign(reinterpret_cast<const std::byte*>(gate),
                       reinterpret_cast<const std::byte*>(gate) + n);
    expert.up.assign(reinterpret_cast<const std::byte*>(up),
                     reinterpret_cast<const std::byte*>(up) + n);
    expert.down.assign(reinterpret_cast<const std::byte*>(down),
                       reinterpret_cast<const std::byte*>(down) + n);
    auto r = vi::qwen38_expert_mlp_q8(std::span<const float>(x, width), expert, width,
                                      intermediate);
    if (!r) return status(r);
    std::memcpy(y, r.value().data(), width * sizeof(float));
    return 0;
}
