// The reference-side binding of the MI355X path: vastloom::hip::HipMatvecAccelerator implements
// the graph's accelerator seam, inference::DeepseekV4MatvecAccelerator
// (include/vastloom/inference/deepseek_v4_reference.hpp:437-451), over the C ABI of
// libvastloom_hip.so (vastloom_hip.h), the way CudaMatvecAccelerator
// (src/cuda/cuda_matvec_accelerator.cpp:102-314) does over the CUDA driver. In the reference tree it
// is src/hip/hip_matvec_accelerator.hpp: it includes the reference's headers, links against its
// ResourceGovernor and deepseek_v4_packed_matrix_payload, and loads libvastloom_hip.so at run time.
//
// The reference keeps its own ResourceGovernor. Every byte the library reserves (pinned staging when
// the accelerator is created, device memory for each resident matrix) is a safety::Reservation
// taken from that Governor through vl_governor_ops and held here under an id until the library
// releases it, or abandons it after a failed device free (the bytes then stay charged, as
// CudaAllocation::release_for_destruction does, src/cuda/cuda_driver.cpp:2881-2893).
//
// Outcomes map onto the seam's contract: VL_OK is Ok(true) with the output written; VL_DECLINED is
// Ok(false) with the output untouched, and the graph runs its CPU kernel; any other status is an
// error carrying the library's message, never a silent CPU recompute
// (qwen3_8_flash_next_reference.cpp:1300-1303).
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <span>
#include <string>
#include <string_view>
#include <utility>

#include "vastloom/core/status.hpp"
#include "vastloom/inference/deepseek_v4_reference.hpp"
#include "vastloom/safety/resource_governor.hpp"
#include "vastloom_hip.h"

namespace vastloom::hip {

// A C ABI status (1 + ErrorCode, include/vastloom/core/status.hpp:10-21) as the reference's Error.
inline Error to_error(int code, std::string_view what) {
    const int ec = code - 1;
    const ErrorCode c = ec >= 0 && ec <= static_cast<int>(ErrorCode::internal_error) ? static_cast<ErrorCode>(ec)
                                                                                     : ErrorCode::internal_error;
    return make_error(c, vl_last_error(), std::string(what));
}

// The seam's three outcomes: accelerated, declined (output untouched), error.
inline Result<bool> to_offer(int code, std::string_view what) {
    if (code == VL_OK) return true;
    if (code == VL_DECLINED) return false;
    return to_error(code, what);
}

class HipMatvecAccelerator final : public inference::DeepseekV4MatvecAccelerator {
public:
    // backend: nullptr for the HIP device options.device_ordinal; a test passes its own device
    // operations (the seam CudaDriver::from_backend_for_testing gives the CUDA accelerator,
    // include/vastloom/cuda/cuda_driver.hpp:217).
    [[nodiscard]] static Result<std::unique_ptr<HipMatvecAccelerator>> create(
        safety::ResourceGovernor& governor, const vl_accel_options& options,
        const vl_accel_backend* backend = nullptr) {
        std::unique_ptr<HipMatvecAccelerator> self(new HipMatvecAccelerator(governor));
        const int rc = vl_accel_create(&options, &self->ops_, backend, &self->accel_);
        if (rc != VL_OK) return to_error(rc, "hip-matvec-accelerator");
        return self;
    }

    ~HipMatvecAccelerator() override {
        if (accel_ != nullptr) (void)vl_accel_destroy(accel_);
    }

    [[nodiscard]] Result<bool> matvec(const inference::DeepseekV4PackedMatrix& matrix, std::span<const float> input,
                                      std::span<float> output) override {
        auto payload = inference::deepseek_v4_packed_matrix_payload(matrix, "hip-matvec");
        if (!payload) return payload.error();
        const std::span<const std::byte> bytes = payload.value();
        const vl_packed_matrix pm{matrix.ggml_type,
                                  matrix.recurring ? 1U : 0U,
                                  static_cast<std::uint64_t>(matrix.rows),
                                  static_cast<std::uint64_t>(matrix.logical_columns),
                                  static_cast<std::uint64_t>(matrix.storage_columns),
                                  bytes.data(),
                                  static_cast<std::uint64_t>(bytes.size()),
                                  matrix.cache_identity};
        return to_offer(vl_accel_matvec(accel_, &pm, input.data(), input.size(), output.data(), output.size()),
                        "hip-matvec");
    }

    // CudaMatvecAccelerator::holds: whether these weights are resident now.
    [[nodiscard]] bool holds(std::uint64_t cache_identity) const { return vl_accel_holds(accel_, cache_identity) == 1; }

    [[nodiscard]] Result<vl_accel_stats> stats() const {
        vl_accel_stats s{};
        const int rc = vl_accel_stats_get(accel_, &s);
        if (rc != VL_OK) return to_error(rc, "hip-matvec-stats");
        return s;
    }

    // Reservations the library holds through this accelerator right now.
    [[nodiscard]] std::size_t reservations() const { return held_.size(); }

private:
    explicit HipMatvecAccelerator(safety::ResourceGovernor& governor) : governor_(governor) {
        ops_.ctx = this;
        ops_.try_reserve = &try_reserve;
        ops_.release = &release;
        ops_.abandon = &abandon;
    }

    static int try_reserve(void* ctx, std::uint32_t kind, std::uint64_t bytes, const char* tag, std::uint64_t* id) {
        auto* self = static_cast<HipMatvecAccelerator*>(ctx);
        auto r = self->governor_.try_reserve(static_cast<safety::ResourceKind>(kind), bytes, tag ? tag : "");
        if (!r) return 1 + static_cast<int>(r.error().code);
        *id = ++self->next_;
        self->held_.emplace(*id, r.take_value());
        return VL_OK;
    }
    static void release(void* ctx, std::uint64_t id) { static_cast<HipMatvecAccelerator*>(ctx)->held_.erase(id); }
    static void abandon(void* ctx, std::uint64_t id) {
        auto& held = static_cast<HipMatvecAccelerator*>(ctx)->held_;
        if (auto it = held.find(id); it != held.end()) {
            it->second.abandon_accounting_on_external_release_failure();
            held.erase(it);
        }
    }

    safety::ResourceGovernor& governor_;
    vl_governor_ops ops_{};
    vl_accel* accel_{nullptr};
    std::uint64_t next_{0};
    std::map<std::uint64_t, safety::Reservation> held_;
};

}  // namespace vastloom::hip
