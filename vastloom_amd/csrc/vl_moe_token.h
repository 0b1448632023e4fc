// Single-token MoE layers: the gate/up and down kernels of a layer whose one token is routed to
// top-k experts (plus an optional shared expert), and the work partition they share.
//
// Partition. A kernel's work is a list of jobs: a gate/up job is one 32-row tile of one active
// expert's gate and up matrices (2C units, C = units per matrix row); a down job is one 32-row
// tile of the layer output, over every active expert's down matrix (A*C units). Blocks own jobs:
//   D   data-parallel: block b owns q whole jobs, reduced and finished inside the block;
//   S   (gate/up only) the shared expert's jobs, split evenly over all blocks (stream-K);
//   R   the jobs that do not divide evenly among the blocks, split the same way.
// A block processes its S and R units first, so that the hand-off of those split jobs between
// blocks (a record per block, a counter, the last contributor finishing the job) happens while
// the block still streams its D jobs. The S region needs no routing: blocks stream the shared
// expert while the routing is formed.
//
// Inside a block, units are taken in chunks of kTokChunkUnits (never straddling a matrix or an
// expert) by the waves through an LDS counter, so the waves of a block finish together. Each
// chunk's partial sums go to its own LDS slot and are added in chunk order, which keeps the
// results deterministic whichever wave took which chunk.
#ifndef VL_MOE_TOKEN_H
#define VL_MOE_TOKEN_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vl_moe.h"

namespace vl {

constexpr uint32_t kTokWaves = 16;

// Units per chunk: two, except one for IQ3_XXS, whose units are the widest to hold in registers.
__host__ __device__ constexpr uint32_t tok_chunk_units(uint32_t) { return 1u; }
constexpr uint32_t kTokMaxSeg = 4;       // jobs one block's piece of a stream-K region may touch
constexpr uint32_t kTokMaxActive = 17;   // top_k <= 16 plus the shared expert
constexpr uint32_t kTokMaxExperts = 1024;

// A stream-K region: `total` units of consecutive jobs from job0 on, split into equal contiguous
// pieces over the first `blocks` blocks (every one of them gets at least one unit).
struct TokRegion {
    uint32_t total, blocks, job0;
};

struct TokPlan {
    uint32_t grid;        // blocks launched
    uint32_t tiles;       // 32-row tiles of one matrix (gate/up: inter/32; down: width/32)
    uint32_t C;           // units per matrix row
    uint32_t UJ;          // units per job
    uint32_t CU;          // units per chunk
    uint32_t q;           // data-parallel jobs per block (jobs b*q .. b*q + q - 1)
    uint32_t A;           // active experts
    uint32_t max_chunks;  // chunks of the busiest block
    TokRegion S, R;
};

// Whether a layer takes the single-token kernels, and their plans for a grid of `blocks`.
bool tok_applies(const MoeShape& s, uint32_t blocks);
TokPlan tok_plan_gateup(const MoeShape& s, uint32_t blocks);
TokPlan tok_plan_down(const MoeShape& s, uint32_t blocks);

// Workspace bytes of the single-token kernels' hand-off records (0 when they do not apply).
uint64_t tok_record_bytes(const MoeShape& s, uint32_t blocks);

// Gate/up (with routing) and down launches of a single-token layer. `events`, when given, is a
// start and a stop event around each kernel's own execution.
hipError_t launch_tok_gateup(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                             hipStream_t st, hipEvent_t* events);
hipError_t launch_tok_down(const MoeShape& s, const MoeInputs& in, const MoeWorkspace& w,
                           hipStream_t st, hipEvent_t* events);

}  // namespace vl

#endif  // VL_MOE_TOKEN_H
