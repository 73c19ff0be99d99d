// Sparse indexer decode scoring for gfx950: FP8 paged MQA logits and the
// top-k pool selection that feeds the kpool expansion and the attention.
//
// The reference's decode indexer (integration/patch_decode_indexer.py:34-44)
// calls vLLM's fp8_paged_mqa_logits_triton over the pool-granular context
// (max_model_len / index_kpool columns), then a top-512 per row whose pool
// ids are expanded to token positions (patch_indexer_sharding.py:92-99).
// Both live in vLLM (not in the reference); the logits follow the published
// semantics of DeepGEMM's fp8_paged_mqa_logits, which that Triton kernel
// reproduces:
//   logits[t, j] = sum_h w[t, h] * max(0, s_j * (q[t, h, :] . k_j))
// for pool positions j < context_len[t] (-inf where the block table points
// outside the cache, and past the context when clean_logits is set), with q
// and k in FP8 E4M3 (OCP), k_j
// and its fp32 scale s_j read through the request's block table from the
// fused cache layout [num_blocks][block_size * 128 key bytes][block_size * 4
// scale bytes].
//
// Logits kernel: workgroup = (token, run of keys); 4 wavefronts, each takes
// 16 keys at a time.  Per 16 keys: the 16 keys' 128 bytes (one contiguous
// 2 KB block when the keys share a page) and scales, then 4 x (H/16)
// v_mfma_f32_16x16x32_fp8_fp8 with A = q (16 heads x 32 dims), B = k^T
// (32 dims x 16 keys).  Lane (g, c) of D holds key c for heads 4g + [0, 4)
// of each head tile, so the relu-weighted head sum is 4 FMAs per tile and
// two cross-row swaps.  Each lane's B operand is dims [32g, 32g + 32) of key
// c (32 contiguous bytes) and the A operand the same dims of its head, so
// k-slot 8g + e of MFMA m is dim 32g + 8m + e on both sides.  A wave issues
// the loads of all its groups before the first MFMA.
//
// Top-k kernel: one 1024-thread workgroup per row; radix select on the
// order-preserving 32-bit keys of the logits (12, 12 and 8 bits, a 4096-bin
// LDS histogram per pass) finds the k-th largest key, then one ordered
// compaction writes the selected positions in ascending order (ties at the
// threshold resolved by position): deterministic.
#include "glm53_common.h"

namespace glm53 {
namespace {

constexpr int kHeadDim = 128;
constexpr int kMaxHeads = 64;
constexpr int kLogitWaves = 4;
constexpr int kLogitThreads = 64 * kLogitWaves;

typedef float f32x4v __attribute__((ext_vector_type(4)));

struct LogitsArgs {
  const uint8_t* q;         // fp8 [T][H][128], strides in bytes
  int64_t sq_t, sq_h;
  const uint8_t* kv;        // fused pages
  int64_t page_bytes;       // byte stride between pages (>= block_size * 132)
  int block_size;
  int num_blocks;
  const float* w;           // [T][H]
  int64_t sw_t;
  const int32_t* ctx;       // [T] pool-granular context lengths
  const int32_t* bt;        // [T][max_blocks]
  int64_t bt_stride;
  int max_blocks;
  int num_heads;
  int max_len;              // logits columns
  int keys_per_wg;
  float* logits;            // [T][max_len], row stride sl_t
  int64_t sl_t;
  int clean;                // write -inf at positions >= context length
};

__device__ __forceinline__ float row_sum4(float v) {
  // sum over lanes l, l^16, l^32, l^48 (the four 16-lane rows)
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int kGroups>
__global__ __launch_bounds__(kLogitThreads) void fp8_paged_mqa_logits_kernel(const LogitsArgs a) {
  const int t = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int j_begin = blockIdx.x * a.keys_per_wg;
  const int j_end = j_begin + a.keys_per_wg < a.max_len ? j_begin + a.keys_per_wg : a.max_len;
  const int cap = a.max_blocks * a.block_size;
  int len = a.ctx[t];
  len = len < 0 ? 0 : len > cap ? cap : len;
  const int n_tiles = a.num_heads / 16;

  // q fragments (A operand) and the weights of this lane's heads.
  uint64_t qf[kMaxHeads / 16][4];
  float wv[kMaxHeads / 16][4];
#pragma unroll
  for (int ht = 0; ht < kMaxHeads / 16; ht++) {
    if (ht < n_tiles) {
      const uint4* qp = reinterpret_cast<const uint4*>(a.q + t * a.sq_t + (16 * ht + c) * a.sq_h + 32 * g);
      const uint4 lo = qp[0], hi = qp[1];
      qf[ht][0] = (static_cast<uint64_t>(lo.y) << 32) | lo.x;
      qf[ht][1] = (static_cast<uint64_t>(lo.w) << 32) | lo.z;
      qf[ht][2] = (static_cast<uint64_t>(hi.y) << 32) | hi.x;
      qf[ht][3] = (static_cast<uint64_t>(hi.w) << 32) | hi.z;
#pragma unroll
      for (int i = 0; i < 4; i++) wv[ht][i] = a.w[t * a.sw_t + 16 * ht + 4 * g + i];
    } else {
#pragma unroll
      for (int m = 0; m < 4; m++) qf[ht][m] = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) wv[ht][i] = 0.f;
    }
  }

  const int64_t key_bytes = static_cast<int64_t>(a.block_size) * kHeadDim;
  float* out = a.logits + t * a.sl_t;
  // This wave's groups: keys j0 = j_begin + 16 * (w + kLogitWaves * u).
  for (int base = j_begin + 16 * w; base < j_end; base += 16 * kLogitWaves * kGroups) {
    uint4 kd[kGroups][2];
    float sc[kGroups];
    bool live[kGroups];   // the group's first page is in the cache (uniform)
    bool kok[kGroups];    // this lane's key is valid and its page in the cache
#pragma unroll
    for (int u = 0; u < kGroups; u++) {
      const int j0 = base + 16 * kLogitWaves * u;
      const int j = j0 + c;
      int blk = -1;
      if (j0 < j_end && j0 < len) blk = a.bt[t * a.bt_stride + j0 / a.block_size];   // uniform
      live[u] = blk >= 0 && blk < a.num_blocks;
      kd[u][0] = kd[u][1] = make_uint4(0, 0, 0, 0);
      sc[u] = 0.f;
      kok[u] = false;
      if (live[u]) {
        // keys of a 16-group may straddle a page only when block_size % 16 != 0
        const int jb = j < len ? j : j0;
        const int bj = jb / a.block_size == j0 / a.block_size ? blk : a.bt[t * a.bt_stride + jb / a.block_size];
        const bool ok = bj >= 0 && bj < a.num_blocks;
        const uint8_t* page = a.kv + static_cast<int64_t>(ok ? bj : 0) * a.page_bytes;
        const int off = jb % a.block_size;
        const uint4* kp = reinterpret_cast<const uint4*>(page + static_cast<int64_t>(off) * kHeadDim + 32 * g);
        kd[u][0] = kp[0];
        kd[u][1] = kp[1];
        kok[u] = ok && j < len;
        sc[u] = kok[u] ? *reinterpret_cast<const float*>(page + key_bytes + 4 * off) : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kGroups; u++) {
      const int j0 = base + 16 * kLogitWaves * u;
      if (j0 >= j_end) break;   // uniform
      const int j = j0 + c;
      float v = 0.f;
      if (live[u]) {
        const uint64_t k0 = (static_cast<uint64_t>(kd[u][0].y) << 32) | kd[u][0].x;
        const uint64_t k1 = (static_cast<uint64_t>(kd[u][0].w) << 32) | kd[u][0].z;
        const uint64_t k2 = (static_cast<uint64_t>(kd[u][1].y) << 32) | kd[u][1].x;
        const uint64_t k3 = (static_cast<uint64_t>(kd[u][1].w) << 32) | kd[u][1].z;
#pragma unroll
        for (int ht = 0; ht < kMaxHeads / 16; ht++) {
          if (ht >= n_tiles) break;   // uniform
          f32x4v d = {0.f, 0.f, 0.f, 0.f};
          d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(static_cast<long>(qf[ht][0]), static_cast<long>(k0), d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(static_cast<long>(qf[ht][1]), static_cast<long>(k1), d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(static_cast<long>(qf[ht][2]), static_cast<long>(k2), d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(static_cast<long>(qf[ht][3]), static_cast<long>(k3), d, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; i++) v = __builtin_fmaf(wv[ht][i], fmaxf(sc[u] * d[i], 0.f), v);
        }
        v = row_sum4(v);
      }
      if (g == 0 && j < j_end) {
        if (kok[u]) out[j] = v;
        else if (j < len || a.clean) out[j] = -__builtin_inff();   // page outside the cache, or past the context
      }
    }
  }
}

// ------------------------------------------------------------------ top-k
constexpr int kTopkThreads = 1024;
constexpr int kHistBins = 4096;

struct TopkArgs {
  const float* logits;      // [rows][*], row stride sl
  int64_t sl;
  const int32_t* lengths;   // [rows] valid columns per row
  int max_len;              // columns available in a row
  int k;
  int32_t* out;             // [rows][k], row stride so
  int64_t so;
};

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  if (f != f) return 0u;                                   // NaN ranks last
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);      // larger float -> larger key
}

struct TopkShared {
  uint32_t hist[kHistBins];
  uint32_t scan[kTopkThreads];
  uint32_t scan2[kTopkThreads];
  uint32_t pick[2];   // digit, count of keys above it
};

// Inclusive prefix sum over the workgroup of one value per thread (Hillis-Steele in LDS).
__device__ uint32_t block_inclusive_scan(uint32_t* buf, uint32_t v) {
  const int tid = threadIdx.x;
  buf[tid] = v;
  __syncthreads();
  for (int off = 1; off < kTopkThreads; off <<= 1) {
    const uint32_t add = tid >= off ? buf[tid - off] : 0u;
    __syncthreads();
    buf[tid] += add;
    __syncthreads();
  }
  return buf[tid];
}

__global__ __launch_bounds__(kTopkThreads) void indexer_topk_kernel(const TopkArgs a) {
  __shared__ TopkShared sh;
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  int len = a.lengths[row];
  len = len < 0 ? 0 : len > a.max_len ? a.max_len : len;
  const float* x = a.logits + row * a.sl;
  int32_t* out = a.out + row * a.so;
  const int k = a.k;
  if (len <= k) {   // every valid position is selected (uniform)
    for (int i = tid; i < k; i += kTopkThreads) out[i] = i < len ? i : -1;
    return;
  }
  // Thread tid owns the contiguous positions [lo, hi).
  const int seg = (len + kTopkThreads - 1) / kTopkThreads;
  const int lo = tid * seg < len ? tid * seg : len;
  const int hi = lo + seg < len ? lo + seg : len;

  uint32_t prefix = 0, pmask = 0;
  uint32_t need = static_cast<uint32_t>(k);   // keys still to take at or below the current prefix
  const int shifts[3] = {20, 8, 0};
  const int widths[3] = {12, 12, 8};
#pragma unroll
  for (int pass = 0; pass < 3; pass++) {
    const int shift = shifts[pass];
    const uint32_t dmask = (1u << widths[pass]) - 1u;
    const int nbins = 1 << widths[pass];
    for (int b = tid; b < kHistBins; b += kTopkThreads) sh.hist[b] = 0u;
    __syncthreads();
    for (int i = lo; i < hi; i++) {
      const uint32_t key = order_key(x[i]);
      if ((key & pmask) == prefix) atomicAdd(&sh.hist[(key >> shift) & dmask], 1u);
    }
    __syncthreads();
    // Suffix counts: thread tid owns bins [bpt*(T-1-tid), ...) so that an
    // inclusive scan over tid counts keys in the highest bins first.
    const int bpt = nbins / kTopkThreads > 0 ? nbins / kTopkThreads : 1;
    const int b0 = nbins - bpt * (tid + 1);   // this thread's lowest bin (bins above it belong to lower tids)
    uint32_t mine = 0;
    if (b0 >= 0)
      for (int b = b0; b < b0 + bpt; b++) mine += sh.hist[b];
    const uint32_t incl = block_inclusive_scan(sh.scan, mine);
    const uint32_t excl = incl - mine;        // keys in bins above this thread's range
    if (b0 >= 0 && excl < need && incl >= need) {
      uint32_t above = excl;
      for (int b = b0 + bpt - 1; b >= b0; b--) {
        if (above + sh.hist[b] >= need) {
          sh.pick[0] = static_cast<uint32_t>(b);
          sh.pick[1] = above;
          break;
        }
        above += sh.hist[b];
      }
    }
    __syncthreads();
    prefix |= sh.pick[0] << shift;
    pmask |= dmask << shift;
    need -= sh.pick[1];
    __syncthreads();
  }
  // prefix = the k-th largest key; take every key above it and the first
  // `need` keys equal to it, in position order.
  uint32_t gt = 0, eq = 0;
  for (int i = lo; i < hi; i++) {
    const uint32_t key = order_key(x[i]);
    gt += key > prefix;
    eq += key == prefix;
  }
  const uint32_t eq_incl = block_inclusive_scan(sh.scan, eq);
  const uint32_t eq_before = eq_incl - eq;
  const uint32_t eq_take = eq_before >= need ? 0u : (need - eq_before < eq ? need - eq_before : eq);
  const uint32_t sel = gt + eq_take;
  const uint32_t sel_incl = block_inclusive_scan(sh.scan2, sel);
  uint32_t pos = sel_incl - sel;
  uint32_t eq_left = eq_take;
  for (int i = lo; i < hi; i++) {
    const uint32_t key = order_key(x[i]);
    if (key > prefix || (key == prefix && eq_left > 0)) {
      if (key == prefix) eq_left--;
      out[pos++] = i;
    }
  }
}

bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }

}  // namespace
}  // namespace glm53

using namespace glm53;

extern "C" int glm53_fp8_paged_mqa_logits(const void* q, int64_t sq_t, int64_t sq_h, const void* kv_cache,
                                          int64_t page_bytes, int64_t block_size, int64_t num_blocks,
                                          const float* weights, int64_t sw_t, const int32_t* context_lens,
                                          const int32_t* block_table, int64_t bt_stride, int64_t max_blocks,
                                          int64_t num_tokens, int64_t num_heads, int64_t head_dim,
                                          int64_t max_len, int clean_logits, float* logits, int64_t sl_t,
                                          void* stream) {
  if (!q || !kv_cache || !weights || !context_lens || !block_table || !logits) return GLM53_ERR_NULL_POINTER;
  if (head_dim != kHeadDim || num_heads < 16 || num_heads > kMaxHeads || num_heads % 16 || num_tokens < 0 ||
      num_tokens > 65535 || block_size < 1 || num_blocks < 1 || max_blocks < 1 || max_len < 0 ||
      max_blocks * block_size > (int64_t(1) << 31) - 1 || page_bytes < block_size * (kHeadDim + 4) ||
      sq_h < kHeadDim || sq_t < num_heads * sq_h || sw_t < num_heads || sl_t < max_len || bt_stride < max_blocks)
    return GLM53_ERR_BAD_SHAPE;
  if (!aligned(q, 16) || sq_t % 16 || sq_h % 16 || !aligned(kv_cache, 16) || page_bytes % 16 ||
      (block_size * kHeadDim) % 4 || !aligned(weights, 4) || !aligned(logits, 4))
    return GLM53_ERR_MISALIGNED;
  if (num_tokens == 0 || max_len == 0) return 0;
  // 16 groups (1024 keys) per workgroup when that still gives the CUs a few
  // workgroups each, else 4 (256 keys).
  const int64_t wg_large = num_tokens * ((max_len + 1023) / 1024);
  const bool large = wg_large >= 512;
  const int keys_per_wg = large ? 16 * kLogitWaves * 16 : 16 * kLogitWaves * 4;
  LogitsArgs a{static_cast<const uint8_t*>(q), sq_t, sq_h, static_cast<const uint8_t*>(kv_cache), page_bytes,
               static_cast<int>(block_size), static_cast<int>(num_blocks), weights, sw_t, context_lens,
               block_table, bt_stride, static_cast<int>(max_blocks), static_cast<int>(num_heads),
               static_cast<int>(max_len), keys_per_wg, logits, sl_t, clean_logits ? 1 : 0};
  const dim3 grid(static_cast<unsigned>((max_len + keys_per_wg - 1) / keys_per_wg), static_cast<unsigned>(num_tokens));
  (void)hipGetLastError();
  if (large)
    hipLaunchKernelGGL(fp8_paged_mqa_logits_kernel<16>, grid, dim3(kLogitThreads), 0,
                       static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(fp8_paged_mqa_logits_kernel<4>, grid, dim3(kLogitThreads), 0,
                       static_cast<hipStream_t>(stream), a);
  return static_cast<int>(hipGetLastError());
}

extern "C" int glm53_indexer_topk(const float* logits, int64_t sl, const int32_t* lengths, int64_t num_rows,
                                  int64_t max_len, int64_t k, int32_t* out, int64_t so, void* stream) {
  if (!logits || !lengths || !out) return GLM53_ERR_NULL_POINTER;
  if (num_rows < 0 || num_rows > (1 << 30) || k < 1 || k > max_len || max_len > (int64_t(1) << 30) ||
      sl < max_len || so < k)
    return GLM53_ERR_BAD_SHAPE;
  if (num_rows == 0) return 0;
  TopkArgs a{logits, sl, lengths, static_cast<int>(max_len), static_cast<int>(k), out, so};
  (void)hipGetLastError();
  hipLaunchKernelGGL(indexer_topk_kernel, dim3(static_cast<unsigned>(num_rows)), dim3(kTopkThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return static_cast<int>(hipGetLastError());
}
