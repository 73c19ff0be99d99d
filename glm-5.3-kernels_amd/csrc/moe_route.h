// Stable small-batch MoE route alignment inside one wavefront, shared by the
// aligner kernel and the W4A16 expert kernels.
//
// Layout of kernels/titan_moe_align.py:12-46 (the stable baseline of
// benchmarks/moe_align.py:23-31): routes grouped by expert in ascending
// expert order, stable within an expert, each expert padded to a multiple of
// 8; routes outside [0, 288) are dropped.  Lane j = route j (up to 64):
//   * the 9-bit expert key gives, per lane, the masks of lanes with an equal
//     key (eq) and with a smaller key (lt) after 9 ballots, MSB first;
//   * rank = popcount(eq & valid lanes below me)   (stable position in the expert)
//   * a lane with rank % 8 == 0 starts an 8-block of its expert, so the
//     expert's first sorted position is 8 * popcount(lt & block starts).
#pragma once

#include "glm53_common.h"

namespace glm53 {

constexpr int kAlignExperts = 288;
constexpr int kAlignMaxRoutes = 64;

struct RoutePos {
  int key;          // expert id, kAlignExperts for a dropped route
  bool valid;       // in range and routed to an expert in [0, 288)
  int pos;          // sorted position of a valid route
  uint64_t starts;  // lanes whose route starts an 8-block
};

__device__ __forceinline__ int64_t load_route_id(const void* ids, int ids_i64, int i) {
  return ids_i64 ? static_cast<const int64_t*>(ids)[i]
                 : static_cast<int64_t>(static_cast<const int32_t*>(ids)[i]);
}

// raw: this lane's expert id (any value when !in_range); in_range: lane < R.
__device__ __forceinline__ RoutePos align_routes(int64_t raw, bool in_range) {
  const int lane = threadIdx.x & 63;
  const bool valid = in_range && raw >= 0 && raw < kAlignExperts;
  const int key = valid ? static_cast<int>(raw) : kAlignExperts;  // 9 bits
  uint64_t eq = ~0ull, lt = 0ull;
#pragma unroll
  for (int b = 8; b >= 0; b--) {
    const bool bit = (key >> b) & 1;
    const uint64_t ones = __ballot(bit);
    lt |= bit ? (eq & ~ones) : 0ull;
    eq &= bit ? ones : ~ones;
  }
  const uint64_t valid_mask = __ballot(valid);
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int rank = __popcll(eq & valid_mask & below);
  const bool starts_block = valid && (rank & 7) == 0;
  const uint64_t starts = __ballot(starts_block);
  const int offset = 8 * __popcll(lt & valid_mask & starts);
  return RoutePos{key, valid, offset + rank, starts};
}

}  // namespace glm53
