// gemm_core.hpp -- what the 256x256 GEMM kernels (dense bf16, fp8, general)
// share besides the pipelined tile itself (gemm_pipe.hpp): the tile order
// and launch plan (tile_plan.hpp) and the choice of epilogue.
#pragma once

#include "common.hpp"
#include "tile_plan.hpp"

namespace gemm_core {

// The workgroup-to-tile order and the tail-quarter mapping (tile_plan.hpp).
using tile_plan::tail_quarter;
using tile_plan::xcd_tile_order;

// Host: whether a 256x256-tile launch whose operands (A and B together) take
// `operand_bytes` stores C through LDS (gemm_pipe::store_bf16_staged).  C
// written straight from the accumulators lands in the caches in part-lines;
// once the operands alone nearly fill the 256 MiB last-level cache, that C
// evicts operand panels that later tiles re-read, and the staged nontemporal
// store is faster (measured: +9% bf16 8192^3, +15% 1024x28672x4096).  With
// smaller operands the staging only adds ~1 us per tile (-1% to -8% on eight
// shapes from 4096^3 to 8192x8192x1024, bf16 and fp8).
constexpr uint64_t kStagedOperandBytes = 192ull << 20;
inline bool staged_epilogue(uint64_t operand_bytes) {
  return operand_bytes >= kStagedOperandBytes;
}

}  // namespace gemm_core
