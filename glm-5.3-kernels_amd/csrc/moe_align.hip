// Stable small-batch MoE route alignment for gfx950 (top-8, 288 experts,
// block 8, up to 64 routes).
//
// Behaviour of kernels/titan_moe_align.py:12-46 (equal to the stable baseline
// of benchmarks/moe_align.py:23-31): routes grouped by expert in ascending
// expert order, stable within an expert, each expert padded to a multiple of
// 8 with the value R; expert_ids holds the expert of every 8-block then -1;
// postpad = sum of padded sizes.  Routes outside [0, 288) are dropped.
//
// One wavefront, lane j = route j; the sorted positions come from wave
// ballots (align_routes, moe_route.h) instead of an R x R compare or a
// histogram pass.  The outputs are assembled in LDS (padding first, then the
// scatter) and copied out once, so every output word is written exactly once.
#include "moe_route.h"

namespace glm53 {
namespace {

__global__ __launch_bounds__(64) void moe_align_small_kernel(const void* __restrict__ ids,
                                                             int ids_i64, int R,
                                                             int32_t* __restrict__ sorted_ids,
                                                             int32_t* __restrict__ expert_ids,
                                                             int32_t* __restrict__ postpad) {
  __shared__ int32_t s_sorted[kAlignMaxRoutes * 8];
  __shared__ int32_t s_experts[kAlignMaxRoutes];
  const int lane = threadIdx.x;
  const RoutePos rp = align_routes(lane < R ? load_route_id(ids, ids_i64, lane) : -1, lane < R);

  for (int i = lane; i < R * 8; i += 64) s_sorted[i] = R;
  s_experts[lane] = -1;
  __syncthreads();
  if (rp.valid) s_sorted[rp.pos] = lane;
  if (rp.valid && (rp.starts >> lane) & 1) s_experts[rp.pos >> 3] = rp.key;
  __syncthreads();
  for (int i = lane; i < R * 8; i += 64) sorted_ids[i] = s_sorted[i];
  if (lane < R) expert_ids[lane] = s_experts[lane];
  if (lane == 0) postpad[0] = 8 * __popcll(rp.starts);
}

}  // namespace
}  // namespace glm53

using namespace glm53;

extern "C" int glm53_moe_align_small(const void* topk_ids, int ids_is_i64, int64_t num_routes,
                                     int32_t* sorted_ids, int32_t* expert_ids,
                                     int32_t* num_tokens_post_padded, void* stream) {
  if (num_routes < 1 || num_routes > kAlignMaxRoutes) return GLM53_ERR_BAD_SHAPE;
  if (!topk_ids || !sorted_ids || !expert_ids || !num_tokens_post_padded)
    return GLM53_ERR_NULL_POINTER;
  (void)hipGetLastError();
  hipLaunchKernelGGL(moe_align_small_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream),
                     topk_ids, ids_is_i64, static_cast<int>(num_routes), sorted_ids, expert_ids,
                     num_tokens_post_padded);
  return static_cast<int>(hipGetLastError());
}
