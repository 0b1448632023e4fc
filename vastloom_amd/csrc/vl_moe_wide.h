// Host-side interface of the grouped layer's fp16-MFMA projection kernels (vl_moe_wide.hip) and
// the item records that k_moe_plan writes for them.
#ifndef VL_MOE_WIDE_H
#define VL_MOE_WIDE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vl_moe.h"

namespace vl {

// MFMA groups of sixteen tokens per item, waves per block (gate/up: one 32-row tile of each
// matrix per wave, 256 rows; down: two tiles per wave, 512 rows), and output slabs of 512 rows
// per down block.
constexpr uint32_t kWideGroups = 2;
constexpr uint32_t kWideWaves = 8;
constexpr uint32_t kWideDownSlabs = 2;

// One item of the group list: a run of up to 2 * kWideGroups consecutive entries of one expert.
struct WideItem {
    uint32_t first;    // first entry
    uint32_t entries;  // entries in the run
    uint32_t reserved[2];
};

// Whether a grouped layer of this shape runs on the fp16 kernels: IQ2_XXS gate, up and down,
// widths that are whole 256-column blocks.
bool wide_shape_ok(const MoeShape& s);
uint32_t wide_lds_bytes();

hipError_t launch_wide_prep(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w, hipStream_t st);
hipError_t launch_wide_gateup(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w, hipStream_t st);
hipError_t launch_wide_down(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w, hipStream_t st);

}  // namespace vl

#endif  // VL_MOE_WIDE_H
