// Stable small-batch MoE route alignment for gfx950 (top-8, 288 experts,
// block 8, up to 64 routes).
//
// Behaviour of kernels/titan_moe_align.py:12-46 (equal to the stable baseline
// of benchmarks/moe_align.py:23-31): routes grouped by expert in ascending
// expert order, stable within an expert, each expert padded to a multiple of
// 8 with the value R; expert_ids holds the expert of every 8-block then -1;
// postpad = sum of padded sizes.  Routes outside [0, 288) are dropped.
//
// One wavefront, lane j = route j.  Everything is derived from wave ballots
// instead of an R x R compare or a histogram pass:
//   * the 9-bit expert key gives, per lane, the masks of lanes with an equal
//     key (eq) and with a smaller key (lt) after 9 ballots, MSB first;
//   * rank  = popcount(eq & lanes below me)   (stable position in the expert)
//   * a lane with rank % 8 == 0 starts an 8-block of its expert, so
//     offset = 8 * popcount(lt & block_starts) and
//     postpad = 8 * popcount(block_starts).
// The outputs are assembled in LDS (padding first, then the scatter) and
// copied out once, so every output word is written exactly once.
#include "glm53_common.h"

namespace glm53 {
namespace {

constexpr int kExperts = 288;
constexpr int kMaxRoutes = 64;

__global__ __launch_bounds__(64) void moe_align_small_kernel(const void* __restrict__ ids,
                                                             int ids_i64, int R,
                                                             int32_t* __restrict__ sorted_ids,
                                                             int32_t* __restrict__ expert_ids,
                                                             int32_t* __restrict__ postpad) {
  __shared__ int32_t s_sorted[kMaxRoutes * 8];
  __shared__ int32_t s_experts[kMaxRoutes];
  const int lane = threadIdx.x;

  int64_t raw = kExperts;
  if (lane < R)
    raw = ids_i64 ? static_cast<const int64_t*>(ids)[lane]
                  : static_cast<int64_t>(static_cast<const int32_t*>(ids)[lane]);
  const bool valid = lane < R && raw >= 0 && raw < kExperts;
  const int key = valid ? static_cast<int>(raw) : kExperts;  // 9 bits

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

  for (int i = lane; i < R * 8; i += 64) s_sorted[i] = R;
  s_experts[lane] = -1;
  __syncthreads();
  if (valid) s_sorted[offset + rank] = lane;
  if (starts_block) s_experts[(offset + rank) >> 3] = key;
  __syncthreads();
  for (int i = lane; i < R * 8; i += 64) sorted_ids[i] = s_sorted[i];
  if (lane < R) expert_ids[lane] = s_experts[lane];
  if (lane == 0) postpad[0] = 8 * __popcll(starts);
}

}  // namespace
}  // namespace glm53

using namespace glm53;

extern "C" int glm53_moe_align_small(const void* topk_ids, int ids_is_i64, int64_t num_routes,
                                     int32_t* sorted_ids, int32_t* expert_ids,
                                     int32_t* num_tokens_post_padded, void* stream) {
  if (num_routes < 1 || num_routes > kMaxRoutes) return GLM53_ERR_BAD_SHAPE;
  if (!topk_ids || !sorted_ids || !expert_ids || !num_tokens_post_padded)
    return GLM53_ERR_NULL_POINTER;
  (void)hipGetLastError();
  hipLaunchKernelGGL(moe_align_small_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream),
                     topk_ids, ids_is_i64, static_cast<int>(num_routes), sorted_ids, expert_ids,
                     num_tokens_post_padded);
  return static_cast<int>(hipGetLastError());
}
