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
// a run of 16-key groups.  Per group: the 16 keys' 128 bytes (one contiguous
// 2 KB block when the keys share a page) and scales, then per head tile one
// v_mfma_scale_f32_16x16x128_f8f6f4 (unit scales) with A = q (16 heads x
// 128 dims), B = k^T (128 dims x 16 keys).  Lane (g, c) of D holds key c for
// heads 4g + [0, 4) of each head tile, so the relu-weighted head sum is 4
// clamps and 4 FMAs per tile and two cross-row swaps, the key's scale one
// multiply after the sum (relu(s d) = |s| relu(+-d)).  Each lane's B operand is dims
// [16g, 16g + 16) and [64 + 16g, 64 + 16g + 16) of key c and the A operand
// the same dims of its head: k-slot 32g + 8m + e is dim 16g + 8m + e
// (m < 2), 64 + 16g + 8(m - 2) + e (m >= 2) on both sides, so each of the
// two 16-byte load instructions covers whole 64-byte halves of its 16 keys'
// lines (each half requested once, however soon the L1 evicts it).  A wave reads
// its groups' block-table entries at once and streams the groups through a
// register ring with three groups' loads in flight.
//
// Top-k: order-preserving 32-bit keys, radix select with 12-, 12- and 8-bit
// digits (LDS histograms) for the k-th largest key, then an ordered
// compaction (two workgroup scans) that writes the selected positions in
// ascending order, ties at the threshold resolved by position:
// deterministic.  One workgroup per row is bound by its CU's vector rate, so
// long rows run in two stages: workgroups (row, chunk) keep each chunk's
// local top-k in position order (a key of the row's top k is in its chunk's
// top k), then one workgroup per row selects from those candidates.  Keys
// stay in registers (thread-contiguous runs of positions) through every
// pass; rows too long for the two stages are re-read from L2 per pass.
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
  int keys_per_wg;          // 64 * groups per wave
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

// The same sum for four values at once: on return lane (g, c) holds v[g]
// summed over the four rows at column c.  Three swaps instead of eight, and
// every addition in the order row_sum4 uses: (g0 + g2) + (g1 + g3).
__device__ __forceinline__ float row_sum4x4(const float (&v)[4]) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[0]), __float_as_uint(v[2]), false, false);
  const float s02 = __uint_as_float(a[0]) + __uint_as_float(a[1]);   // lanes 0-31: v[0], 32-63: v[2]
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[1]), __float_as_uint(v[3]), false, false);
  const float s13 = __uint_as_float(b[0]) + __uint_as_float(b[1]);   // lanes 0-31: v[1], 32-63: v[3]
  const auto d = __builtin_amdgcn_permlane16_swap(__float_as_uint(s02), __float_as_uint(s13), false, false);
  return __uint_as_float(d[0]) + __uint_as_float(d[1]);
}

typedef int i32x8 __attribute__((ext_vector_type(8)));

// A lane's 32 bytes of a key (dims 16g + [0, 16) and 64 + 16g + [0, 16)) as
// the B operand of the K = 128 FP8 product.
__device__ __forceinline__ i32x8 key_operand(uint64_t k0, uint64_t k1, uint64_t k2, uint64_t k3) {
  return i32x8{static_cast<int>(k0), static_cast<int>(k0 >> 32), static_cast<int>(k1), static_cast<int>(k1 >> 32),
               static_cast<int>(k2), static_cast<int>(k2 >> 32), static_cast<int>(k3), static_cast<int>(k3 >> 32)};
}

// q . k for 16 heads x 16 keys over all 128 dims in one
// v_mfma_scale_f32_16x16x128_f8f6f4 (both operands FP8 E4M3, unit E8M0
// scales): lane (g, c) gives the same 32 dims of its head (A) and of its key
// (B), so every q byte meets the k byte of the same dim.
__device__ __forceinline__ f32x4v dot128_fp8(const uint64_t (&q)[4], const i32x8& kb) {
  const i32x8 qa = key_operand(q[0], q[1], q[2], q[3]);
  const f32x4v zero = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(qa, kb, zero, 0, 0, 0, 127, 0, 127);
}

// The key's scale taken out of the head sum: relu(s d) = |s| relu(d') with
// d' = d for s >= 0 and d' = -d for s < 0 (the key's E4M3 sign bits
// flipped, which negates its products exactly), so a (key, head) costs a
// clamp and an FMA and the scale one multiply per key.  A NaN scale gives
// 0, as fmax(NaN * d, 0) = 0 does for every head.
__device__ __forceinline__ i32x8 signed_key(i32x8 kb, float sc) {
  const int flip = sc < 0.f ? static_cast<int>(0x80808080u) : 0;
#pragma unroll
  for (int i = 0; i < 8; i++) kb[i] ^= flip;
  return kb;
}
__device__ __forceinline__ float key_factor(float sc) { return sc != sc ? 0.f : fabsf(sc); }

// relu of an unscaled product: v_med3_f32 clamps into [0, 3e38] (|q . k| <=
// 128 * 448^2), and for a NaN input returns the minimum of the other two
// (IEEE mode drops a quiet NaN), 0 -- the fmax(x, 0) semantics, in one
// instruction: fmaxf itself would first quiet its input, since the compiler
// cannot tell that a matrix-core result is never a signalling NaN.
__device__ __forceinline__ float relu_dot(float d) { return __builtin_amdgcn_fmed3f(d, 0.f, 3.0e38f); }

// Loads of one 16-key group (keys j0 + c) into registers: the 32 key bytes
// of this lane (dims 32g + [0, 32)) and the key's scale.  blk is the page of
// the group's first key (uniform); keys of a group straddle pages only when
// block_size % 16 != 0 (kAligned false), and then read their own table
// entry -- a dependent load, which drains the loads in flight, so aligned
// block sizes take the path without it.
struct Group {
  uint4 kd[2];
  float sc;    // the key's scale (meaningful when kok)
  bool live;   // the group is computed: its page is in the cache (aligned), always (straddling)
  bool kok;    // this lane's key is valid and its page in the cache
};

template <bool kAligned>
__device__ __forceinline__ void load_group(const LogitsArgs& a, int t, int j0, int blk, int len, int g, int c,
                                           Group& gr) {
  const int j = j0 + c;
  const int jb = j < len ? j : j0;
  int bj = blk;
  if (!kAligned && jb / a.block_size != j0 / a.block_size) bj = a.bt[t * a.bt_stride + jb / a.block_size];
  // aligned: the group shares one page, valid or not; straddling: each key
  // has its own page, so the group is computed whatever its first page is
  gr.live = !kAligned || (blk >= 0 && blk < a.num_blocks);
  const bool ok = bj >= 0 && bj < a.num_blocks;
  // The loads are issued on every path (page 0 stands in for a page outside
  // the cache), so the count of loads in flight is the same on all paths
  // and a wait for one group never drains the later groups' loads.
  const uint8_t* page = a.kv + static_cast<int64_t>(ok ? bj : 0) * a.page_bytes;
  // aligned: j0 is uniform and the group within one page, so the division is scalar
  const int off = kAligned ? j0 % a.block_size + (jb - j0) : jb % a.block_size;
  const uint4* kp = reinterpret_cast<const uint4*>(page + static_cast<int64_t>(off) * kHeadDim + 16 * g);
  gr.kd[0] = kp[0];   // dims 16g + [0, 16): with the other 3 lane groups, the key's first 64-byte half
  gr.kd[1] = kp[4];   // dims 64 + 16g + [0, 16): its second half
  gr.kok = ok && j < len;
  gr.sc = *reinterpret_cast<const float*>(page + static_cast<int64_t>(a.block_size) * kHeadDim + 4 * off);
}

// Wave = a run of kN 16-key groups of one token's row; the block-table
// entries of all its groups are read at once (lane i: group i), then the
// groups stream through a kDepth-deep ring of register slots, the loads of
// group i + kDepth - 1 issued before group i is reduced, so each wave keeps
// kDepth - 1 groups (6 KB at depth 4) in flight.  The run is unrolled
// whole and its loads issued on every path, and the results wait in LDS
// for stores after the last load (stores count with the loads in vmcnt):
// every wait then counts exactly the group it needs.
template <int kTiles, int kN, bool kAligned>
__global__ __launch_bounds__(kLogitThreads) void fp8_paged_mqa_logits_kernel(
    const int32_t* ctx, const int32_t* bt, int64_t bt_stride, const uint8_t* q, int64_t sq_t, int keys_per_wg,
    int max_len, int block_size, int max_blocks, const LogitsArgs a) {
  constexpr int kDepth = 4;
  const int t = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int j_wave = blockIdx.x * keys_per_wg + w * 16 * kN;
  const int j_end = j_wave + 16 * kN < max_len ? j_wave + 16 * kN : max_len;
  if (j_wave >= j_end) return;   // uniform (no barriers in this kernel)
  const int n = (j_end - j_wave + 15) / 16;
  const int cap = max_blocks * block_size;
  int len = ctx[t];
  len = len < 0 ? 0 : len > cap ? cap : len;

  // page of each group's first key (lane i < n: group i; -1 past the context)
  int blk_l = -1;
  if (lane < n) {
    const int j0 = j_wave + 16 * lane;
    if (j0 < len) blk_l = bt[t * bt_stride + j0 / block_size];
  }

  // q fragments (A operand) and the weights of this lane's heads.
  uint64_t qf[kTiles][4];
  float wv[kTiles][4];
#pragma unroll
  for (int ht = 0; ht < kTiles; ht++) {
    const uint4* qp = reinterpret_cast<const uint4*>(q + t * sq_t + (16 * ht + c) * a.sq_h + 16 * g);
    const uint4 lo = qp[0], hi = qp[4];
    qf[ht][0] = (static_cast<uint64_t>(lo.y) << 32) | lo.x;
    qf[ht][1] = (static_cast<uint64_t>(lo.w) << 32) | lo.z;
    qf[ht][2] = (static_cast<uint64_t>(hi.y) << 32) | hi.x;
    qf[ht][3] = (static_cast<uint64_t>(hi.w) << 32) | hi.z;
#pragma unroll
    for (int i = 0; i < 4; i++) wv[ht][i] = a.w[t * a.sw_t + 16 * ht + 4 * g + i];
  }

  float* out = a.logits + t * a.sl_t;
  __shared__ float res[kLogitWaves][16 * kN];
  Group ring[kDepth];
  // group i of the run, or past the run's end (a row's tail) its last group
  // again, loaded and not used
  auto load = [&](int i, Group& gr) {
    const int ic = i < n ? i : n - 1;
    load_group<kAligned>(a, t, j_wave + 16 * ic, __builtin_amdgcn_readlane(blk_l, ic), len, g, c, gr);
  };
#pragma unroll
  for (int s = 0; s < kDepth - 1; s++)
    if (s < kN) load(s, ring[s]);
  {
#pragma unroll
    for (int i = 0; i < kN; i++) {
      if (i + kDepth - 1 < kN) load(i + kDepth - 1, ring[(i + kDepth - 1) % kDepth]);
      if (i >= n) continue;   // uniform (the tail of a row)
      const Group& gr = ring[i % kDepth];
      float v = 0.f;
      if (gr.live) {
        const uint64_t k0 = (static_cast<uint64_t>(gr.kd[0].y) << 32) | gr.kd[0].x;
        const uint64_t k1 = (static_cast<uint64_t>(gr.kd[0].w) << 32) | gr.kd[0].z;
        const uint64_t k2 = (static_cast<uint64_t>(gr.kd[1].y) << 32) | gr.kd[1].x;
        const uint64_t k3 = (static_cast<uint64_t>(gr.kd[1].w) << 32) | gr.kd[1].z;
        const i32x8 kb = signed_key(key_operand(k0, k1, k2, k3), gr.sc);
#pragma unroll
        for (int ht = 0; ht < kTiles; ht++) {
          const f32x4v d = dot128_fp8(qf[ht], kb);
#pragma unroll
          for (int e = 0; e < 4; e++) v = __builtin_fmaf(wv[ht][e], relu_dot(d[e]), v);
        }
        v = key_factor(gr.sc) * row_sum4(v);
      }
      // page outside the cache, or past the context: -inf (written past the
      // context only when cleaning, which the stores below decide)
      if (g == 0) res[w][16 * i + c] = gr.kok ? v : -__builtin_inff();
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int r = 0; r < (16 * kN + 63) / 64; r++) {
    const int idx = 64 * r + lane;
    const int j = j_wave + idx;   // written inside the run, and past the context only when cleaning
    if (idx < 16 * n && j < j_end && (j < len || a.clean)) out[j] = res[w][idx];
  }
}

// Rows that share one block table (the query rows of one request's prefill
// chunk, each with its own causal length): workgroup = (run of kN 16-key
// groups, 16 rows); wave w scores rows 4w .. 4w + 3 of the block over the
// run, so each key group is loaded once per wave and used for 4 rows x
// kTiles head tiles, and the four waves load the same groups (the later
// waves' loads hit the CU's L1) -- the keys are read from L2 once per 16 rows
// instead of once per row.  Same arithmetic per (row, key) as the per-token
// kernel above; block sizes that are a multiple of 16 only.
template <int kTiles, int kN>
__global__ __launch_bounds__(kLogitThreads) void fp8_mqa_logits_rows_kernel(const LogitsArgs a, int num_tokens) {
  constexpr int kR = 4;        // rows per wave (row_sum4x4 leaves row g's sums in lane group g)
  constexpr int kDepth = 4;
  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int t0 = blockIdx.y * (kR * kLogitWaves) + kR * w;   // first row of this wave
  const int j_run = blockIdx.x * a.keys_per_wg;
  const int j_end = j_run + 16 * kN < a.max_len ? j_run + 16 * kN : a.max_len;
  const int n = (j_end - j_run + 15) / 16;
  const int cap = a.max_blocks * a.block_size;
  int len[kR];
  int len_max = 0;
#pragma unroll
  for (int r = 0; r < kR; r++) {
    int l = t0 + r < num_tokens ? a.ctx[t0 + r] : 0;
    l = l < 0 ? 0 : l > cap ? cap : l;
    len[r] = l;
    len_max = len_max > l ? len_max : l;
  }
  const int my_len = g == 0 ? len[0] : g == 1 ? len[1] : g == 2 ? len[2] : len[3];   // row 4w + g

  // page of each group's first key (lane i < n: group i; -1 past every row's context)
  int blk_l = -1;
  if (lane < n) {
    const int j0 = j_run + 16 * lane;
    if (j0 < len_max) blk_l = a.bt[j0 / a.block_size];
  }

  // q fragments (A operand) and weights of this lane's heads, per row
  uint64_t qf[kR][kTiles][4];
  float wv[kR][kTiles][4];
#pragma unroll
  for (int r = 0; r < kR; r++) {
    const int t = t0 + r < num_tokens ? t0 + r : num_tokens - 1;   // rows past the end: loaded, never stored
#pragma unroll
    for (int ht = 0; ht < kTiles; ht++) {
      const uint4* qp = reinterpret_cast<const uint4*>(a.q + t * a.sq_t + (16 * ht + c) * a.sq_h + 16 * g);
      const uint4 lo = qp[0], hi = qp[4];
      qf[r][ht][0] = (static_cast<uint64_t>(lo.y) << 32) | lo.x;
      qf[r][ht][1] = (static_cast<uint64_t>(lo.w) << 32) | lo.z;
      qf[r][ht][2] = (static_cast<uint64_t>(hi.y) << 32) | hi.x;
      qf[r][ht][3] = (static_cast<uint64_t>(hi.w) << 32) | hi.z;
#pragma unroll
      for (int i = 0; i < 4; i++) wv[r][ht][i] = a.w[t * a.sw_t + 16 * ht + 4 * g + i];
    }
  }

  __shared__ float res[kLogitWaves][kR][16 * kN];
  Group ring[kDepth];
  // group i of the run, or past the run's end its last group again (loaded, not used)
  auto load = [&](int i, Group& gr) {
    const int ic = i < n ? i : n - 1;
    load_group<true>(a, 0, j_run + 16 * ic, __builtin_amdgcn_readlane(blk_l, ic), len_max, g, c, gr);
  };
  if (n > 0) {
#pragma unroll
    for (int s = 0; s < kDepth - 1; s++)
      if (s < kN) load(s, ring[s]);
#pragma unroll
    for (int i = 0; i < kN; i++) {
      if (i + kDepth - 1 < kN) load(i + kDepth - 1, ring[(i + kDepth - 1) % kDepth]);
      if (i >= n) continue;   // uniform (the tail of the rows)
      const Group& gr = ring[i % kDepth];
      const int j = j_run + 16 * i + c;
      float tot = 0.f;   // lane (g, c): row 4w + g at key j
      if (gr.live) {
        const uint64_t k0 = (static_cast<uint64_t>(gr.kd[0].y) << 32) | gr.kd[0].x;
        const uint64_t k1 = (static_cast<uint64_t>(gr.kd[0].w) << 32) | gr.kd[0].z;
        const uint64_t k2 = (static_cast<uint64_t>(gr.kd[1].y) << 32) | gr.kd[1].x;
        const uint64_t k3 = (static_cast<uint64_t>(gr.kd[1].w) << 32) | gr.kd[1].z;
        const i32x8 kb = signed_key(key_operand(k0, k1, k2, k3), gr.sc);
        float v[kR] = {};
#pragma unroll
        for (int r = 0; r < kR; r++) {
#pragma unroll
          for (int ht = 0; ht < kTiles; ht++) {
            const f32x4v d = dot128_fp8(qf[r][ht], kb);
#pragma unroll
            for (int e = 0; e < 4; e++) v[r] = __builtin_fmaf(wv[r][ht][e], relu_dot(d[e]), v[r]);
          }
        }
        tot = key_factor(gr.sc) * row_sum4x4(v);
      }
      // page outside the cache, or past the row's context: -inf (written past
      // the context only when cleaning, which the stores below decide)
      res[w][g][16 * i + c] = gr.kok && j < my_len ? tot : -__builtin_inff();
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int r = 0; r < kR; r++) {
    if (t0 + r >= num_tokens) break;   // uniform
    float* out = a.logits + (t0 + r) * a.sl_t;
#pragma unroll
    for (int q = 0; q < (16 * kN + 63) / 64; q++) {
      const int idx = 64 * q + lane;
      const int j = j_run + idx;   // written inside the run, and past the row's context only when cleaning
      if (idx < 16 * n && j < j_end && (j < len[r] || a.clean)) out[j] = res[w][r][idx];
    }
  }
}

// ------------------------------------------------------------------ top-k
constexpr int kHistBins = 4096;
constexpr int kChunkThreads = 512;
constexpr int kChunkThreadsWide = 1024;   // chunk workgroups of the few-rows plan (8 keys per thread)
constexpr int kFinalThreads = 1024;
constexpr int kSweepThreads = 1024;
constexpr int kSweepKeys = 32;                      // keys per thread per sweep
constexpr int kSweep = kSweepThreads * kSweepKeys;  // positions per sweep (32768)

struct TopkArgs {
  const float* logits;      // [rows][*], row stride sl
  int64_t sl;
  const int32_t* lengths;   // [rows] valid columns per row
  int max_len;              // columns available in a row
  int k;
  int32_t* out;             // [rows][k], row stride so
  int64_t so;
  uint32_t* cand_key;       // [rows][chunks * k] chunk-local top-k keys, in position order
  int32_t* cand_pos;        // [rows][chunks * k] their positions
  int chunks;
  int chunk_len;
  bool vec;                 // logits rows 16-byte aligned
};

// Order-preserving key: a larger float has a larger key; NaN -> 0, below
// everything else (-inf is 0x007FFFFF).  Positions past the row's length
// also get key 0: with more valid positions than k they are never reached,
// and at equal keys a smaller position always wins.
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  if (f != f) return 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int kThreads>
struct SelShared {
  __attribute__((aligned(16))) uint32_t hist[2][kHistBins];   // passes alternate, so a pass clears the one after next
  uint32_t wsum[kThreads / 64];
  uint32_t wmin[kThreads / 64];
  uint32_t wmax[kThreads / 64];
  uint32_t pick[3];              // digit, keys above it, keys in it
};

// Zero both histograms.  Callers issue it while their keys' loads are in
// flight; the first barrier of radix_threshold orders it before the first
// atomics.
template <int kThreads>
__device__ __forceinline__ void clear_hist(SelShared<kThreads>& sh) {
  for (int b = threadIdx.x; b < 2 * kHistBins / 4; b += kThreads)
    reinterpret_cast<uint4*>(&sh.hist[0][0])[b] = make_uint4(0u, 0u, 0u, 0u);
}

// Inclusive scan of one value per lane within the wave: row_shr 1, 2, 4, 8
// inside rows of 16 lanes, then row_bcast 15 and 31 carry row totals upward.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_or_zero(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, kRowMask, 0xf, false));
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  v += dpp_or_zero<0x111, 0xf>(v);
  v += dpp_or_zero<0x112, 0xf>(v);
  v += dpp_or_zero<0x114, 0xf>(v);
  v += dpp_or_zero<0x118, 0xf>(v);
  v += dpp_or_zero<0x142, 0xa>(v);
  v += dpp_or_zero<0x143, 0xc>(v);
  return v;
}

// Largest value of the wave (broadcast).
__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
  v = max(v, dpp_or_zero<0x111, 0xf>(v));
  v = max(v, dpp_or_zero<0x112, 0xf>(v));
  v = max(v, dpp_or_zero<0x114, 0xf>(v));
  v = max(v, dpp_or_zero<0x118, 0xf>(v));
  v = max(v, dpp_or_zero<0x142, 0xa>(v));
  v = max(v, dpp_or_zero<0x143, 0xc>(v));
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// Exclusive scan over the workgroup of one value per thread; *total gets the
// sum.  sh.wsum is read after the return: a barrier must separate the
// return from the next scan.
template <int kThreads>
__device__ __forceinline__ uint32_t block_excl_scan(SelShared<kThreads>& sh, uint32_t v, uint32_t* total) {
  constexpr int kWaves = kThreads / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t incl = wave_incl_scan(v);
  if (lane == 63) sh.wsum[w] = incl;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int i = 0; i < kWaves; i++) {
    const uint32_t t = sh.wsum[i];
    before += i < w ? t : 0u;
    all += t;
  }
  *total = all;
  return before + incl - v;
}

// Selection threshold: keys whose bits under pmask exceed thr are all in the
// top k; of the keys equal to thr under pmask the first `need` (by index)
// are.  pmask is all ones unless a pass found that a whole digit bin is
// taken, which ends the search early.
struct Threshold {
  uint32_t thr, pmask, need;
};

// Radix select of the k-th largest key with LDS histograms of up to 12-bit
// digits, starting below the bits that kmin and kmax (this thread's smallest
// and largest key, over keys that must count) share across the workgroup: a
// concentrated set of keys (a chunk's candidates) still spreads over the
// bins, which keeps the histogram atomics from piling onto a few addresses.
// for_keys(f) calls f(key) for every key of this thread; the keys matching
// the shared bits must number at least k.  The caller has zeroed both
// histograms (clear_hist) before the call.
template <int kThreads, class ForKeys>
__device__ Threshold radix_threshold(SelShared<kThreads>& sh, ForKeys for_keys, uint32_t k, uint32_t kmin,
                                     uint32_t kmax) {
  constexpr int kWaves = kThreads / 64;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  kmin = ~wave_max(~kmin);
  kmax = wave_max(kmax);
  if (lane == 0) { sh.wmin[w] = kmin; sh.wmax[w] = kmax; }
  __syncthreads();   // also orders the caller's clear_hist before the first atomics
#pragma unroll
  for (int i = 0; i < kWaves; i++) { kmin = min(kmin, sh.wmin[i]); kmax = max(kmax, sh.wmax[i]); }
  const uint32_t diff = kmin ^ kmax;
  if (diff == 0) return {kmax, ~0u, k};   // one distinct key
  int top = 32 - __clz(static_cast<int>(diff));   // bits [top, 32) are shared
  uint32_t pmask = top == 32 ? 0u : ~((1u << top) - 1u);
  uint32_t prefix = kmax & pmask, need = k;
  for (int pass = 0; top > 0; pass++) {
    const int width = top < 12 ? top : 12;
    const int shift = top - width;
    top = shift;
    const int nb = 1 << width;
    const uint32_t dmask = static_cast<uint32_t>(nb - 1);
    uint32_t* hist = sh.hist[pass & 1];
    for_keys([&](uint32_t key) {
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & dmask], 1u);
    });
    if (pass == 1)   // pass 0's histogram is no longer read: clear it for pass 2
      for (int b = tid; b < kHistBins / 4; b += kThreads)
        reinterpret_cast<uint4*>(sh.hist[0])[b] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
    // Thread tid owns bpt bins counted from the top (held in registers): the
    // keys in higher bins are the wave totals of lower waves plus the lanes
    // below in this wave.
    constexpr int kMaxBpt = kHistBins / kThreads;
    const int bpt = nb >= kThreads ? nb / kThreads : 1;
    const int b0 = nb - bpt * (tid + 1);
    uint32_t hb[kMaxBpt];
#pragma unroll
    for (int i = 0; i < kMaxBpt; i++) hb[i] = 0u;
    if (b0 >= 0) {
      if ((bpt & 3) == 0) {
#pragma unroll
        for (int q = 0; q < kMaxBpt / 4; q++)
          if (4 * q < bpt) {
            const uint4 v = *reinterpret_cast<const uint4*>(hist + b0 + 4 * q);
            hb[4 * q] = v.x; hb[4 * q + 1] = v.y; hb[4 * q + 2] = v.z; hb[4 * q + 3] = v.w;
          }
      } else {
#pragma unroll
        for (int i = 0; i < kMaxBpt; i++)
          if (i < bpt) hb[i] = hist[b0 + i];
      }
    }
    uint32_t mine = 0;
#pragma unroll
    for (int i = 0; i < kMaxBpt; i++) mine += hb[i];
    const uint32_t incl = wave_incl_scan(mine);
    if (lane == 63) sh.wsum[w] = incl;
    __syncthreads();
    uint32_t excl = incl - mine;
#pragma unroll
    for (int i = 0; i < kWaves; i++) excl += i < w ? sh.wsum[i] : 0u;
    if (b0 >= 0 && excl < need && excl + mine >= need) {
      uint32_t above = excl;
      bool found = false;
#pragma unroll
      for (int i = kMaxBpt - 1; i >= 0; i--) {
        if (i < bpt && !found) {
          if (above + hb[i] >= need) {
            sh.pick[0] = static_cast<uint32_t>(b0 + i);
            sh.pick[1] = above;
            sh.pick[2] = hb[i];
            found = true;
          } else {
            above += hb[i];
          }
        }
      }
    }
    __syncthreads();
    prefix |= sh.pick[0] << shift;
    pmask |= dmask << shift;
    need -= sh.pick[1];
    if (sh.pick[2] == need) break;   // the whole bin is taken (uniform)
  }
  return {prefix, pmask, need};
}

// Ordered compaction of the keys kk of this thread, which hold workgroup
// indices base + [0, P) (thread-contiguous): the keys above the threshold and
// the first `need` keys at it, counting from eq_seen keys at it already seen
// at lower indices outside the workgroup's keys; emit(o, j) is called with
// the output rank o (from written) of key j.  Returns the keys at the
// threshold and the keys selected in *n_eq, *n_sel.  Counts must stay below
// 65536 per workgroup (they are packed in one scan).
template <int kThreads, int P, class Emit>
__device__ void emit_selected(SelShared<kThreads>& sh, const uint32_t (&kk)[P], const Threshold& t,
                              uint32_t eq_seen, uint32_t written, Emit emit, uint32_t* n_eq, uint32_t* n_sel) {
  uint32_t ngt = 0, neq = 0;
#pragma unroll
  for (int j = 0; j < P; j++) {
    const uint32_t m = kk[j] & t.pmask;
    ngt += m > t.thr;
    neq += m == t.thr;
  }
  uint32_t tot;
  const uint32_t ex = block_excl_scan(sh, (ngt << 16) | neq, &tot);
  const uint32_t taken_before = eq_seen < t.need ? eq_seen : t.need;
  const uint32_t eq_tot = eq_seen + (tot & 0xffffu);
  *n_eq = tot & 0xffffu;
  *n_sel = (tot >> 16) + (eq_tot < t.need ? eq_tot : t.need) - taken_before;
  uint32_t r = eq_seen + (ex & 0xffffu);
  uint32_t o = written + (ex >> 16) + (r < t.need ? r : t.need) - taken_before;
  if (ngt + neq == 0) return;
#pragma unroll
  for (int j = 0; j < P; j++) {
    const uint32_t m = kk[j] & t.pmask;
    const bool eq = m == t.thr;
    if (m > t.thr || (eq && r < t.need)) emit(o++, j);
    r += eq;
  }
}

// Keys of row positions i0 + [0, P) (P and i0 multiples of 4); positions at
// or past n get key 0 (n >= 1).  vec: x is 16-byte aligned (rows of a stride
// that is a multiple of 4 floats).  Every load of the thread is issued before
// any key is formed: converting each load's value inside its own branch made
// the compiler wait for it before issuing the next.  A thread whose
// positions are all valid takes P / 4 16-byte loads; the others (the row's
// tail) P single loads from positions clamped to n - 1, masked afterwards.
template <int P>
__device__ __forceinline__ void issue_row_loads(const float* x, int n, int i0, bool vec, float (&f)[P]) {
  if (vec && i0 + P <= n) {
#pragma unroll
    for (int q = 0; q < P / 4; q++) {
      const float4 v = *reinterpret_cast<const float4*>(x + i0 + 4 * q);
      f[4 * q] = v.x; f[4 * q + 1] = v.y; f[4 * q + 2] = v.z; f[4 * q + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < P; j++) f[j] = x[i0 + j < n ? i0 + j : n - 1];
  }
}

template <int P>
__device__ __forceinline__ void form_keys(const float (&f)[P], int n, int i0, uint32_t (&kk)[P]) {
#pragma unroll
  for (int j = 0; j < P; j++) kk[j] = i0 + j < n ? order_key(f[j]) : 0u;
}

template <int P>
__device__ __forceinline__ void load_row_keys(const float* x, int n, int i0, bool vec, uint32_t (&kk)[P]) {
  float f[P];
  issue_row_loads<P>(x, n, i0, vec, f);
  form_keys<P>(f, n, i0, kk);
}

template <int P, class F>
__device__ __forceinline__ void for_each_key(const uint32_t (&kk)[P], F&& f) {
#pragma unroll
  for (int j = 0; j < P; j++) f(kk[j]);
}

__device__ __forceinline__ int clamp_len(const int32_t* lengths, int max_len, int row) {
  const int len = lengths[row];
  return len < 0 ? 0 : len > max_len ? max_len : len;
}

__device__ __forceinline__ int clamp_len(const TopkArgs& a, int row) { return clamp_len(a.lengths, a.max_len, row); }

// Chunk stage: workgroup (row, chunk c) keeps the local top-k of positions
// [c * chunk_len, (c + 1) * chunk_len) of the row, in position order, as
// candidates (every valid position when the chunk holds at most k).  A key of
// the row's top k is in its chunk's top k, so the candidates hold the answer.
template <int P, int kThreads>
__global__ __launch_bounds__(kThreads) void topk_chunk_kernel(
    const float* p_logits, int64_t p_sl, const int32_t* p_lengths, int p_max_len, int p_k, int p_chunk_len,
    int p_chunks, int p_vec, const TopkArgs a) {
  __shared__ SelShared<kThreads> sh;
  const int row = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
  const int len = clamp_len(p_lengths, p_max_len, row);
  const int k = p_k;
  const int start = c * p_chunk_len;
  const int rest = len - start;
  const int valid = rest < 0 ? 0 : rest > p_chunk_len ? p_chunk_len : rest;
  if (len <= k || valid == 0) return;   // uniform
  float f[P];
  issue_row_loads<P>(p_logits + row * p_sl + start, valid, tid * P, p_vec, f);
  if (valid > k) clear_hist(sh);   // under the loads' latency (uniform)
  uint32_t kk[P];
  form_keys<P>(f, valid, tid * P, kk);
  const int64_t cb = (static_cast<int64_t>(row) * p_chunks + c) * k;
  uint32_t* ck = a.cand_key + cb;
  int32_t* cp = a.cand_pos + cb;
  if (valid <= k) {
#pragma unroll
    for (int j = 0; j < P; j++) {
      const int i = tid * P + j;
      if (i < valid) { ck[i] = kk[j]; cp[i] = start + i; }
    }
    return;
  }
  uint32_t kmin = ~0u, kmax = 0u;
#pragma unroll
  for (int j = 0; j < P; j++)
    if (tid * P + j < valid) { kmin = min(kmin, kk[j]); kmax = max(kmax, kk[j]); }
  const Threshold t = radix_threshold(sh, [&](auto f) { for_each_key(kk, f); }, static_cast<uint32_t>(k), kmin, kmax);
  uint32_t n_eq, n_sel;
  emit_selected(sh, kk, t, 0u, 0u, [&](uint32_t o, int j) {
    if (o < static_cast<uint32_t>(k)) { ck[o] = kk[j]; cp[o] = start + tid * P + j; }
  }, &n_eq, &n_sel);
}

// Final stage: one workgroup per row selects the top k, in position order,
// from the row itself (kCand false: row length at most kFinalThreads * P) or
// from the chunk stage's candidates (chunk-major, so in position order too).
// Candidate slot s of chunk c is filled when s < min(k, valid positions of
// the chunk); the chunk length exceeds k, so only the last chunk holding
// valid positions can be short and every empty slot (key 0) follows every
// filled one: never selected.
template <int P, bool kCand>
__global__ __launch_bounds__(kFinalThreads) void topk_final_kernel(
    const int32_t* p_lengths, int p_max_len, int p_k, int p_chunks, uint32_t* p_cand_key, int32_t* p_cand_pos,
    int32_t* p_out, int64_t p_so, int p_chunk_len, const TopkArgs a) {
  __shared__ SelShared<kFinalThreads> sh;
  const int row = blockIdx.x, tid = threadIdx.x;
  const int len = clamp_len(p_lengths, p_max_len, row);
  const int k = p_k;
  int32_t* out = p_out + row * p_so;
  if (len <= k) {   // every valid position is selected (uniform)
    for (int i = tid; i < k; i += kFinalThreads) out[i] = i < len ? i : -1;
    return;
  }
  uint32_t kk[P];
  int32_t pos[kCand ? P : 1];
  uint32_t kmin = ~0u, kmax = 0u;
  const int64_t cb = kCand ? static_cast<int64_t>(row) * p_chunks * k : 0;
  if (kCand) {
    // Candidate i = tid * P + j is slot sl of chunk c (i = c * k + sl).  The
    // loads are unconditional (issued together), from clamped indices when
    // k is not a multiple of 4, else as 4-candidate vectors (a vector never
    // straddles chunks then); filled slots are picked afterwards.
    const int n_cand = p_chunks * k;
    if ((k & 3) == 0) {   // keys first: the first pass waits for them only
#pragma unroll
      for (int q = 0; q < P / 4; q++) {
        const int i = tid * P + 4 * q < n_cand ? tid * P + 4 * q : n_cand - 4;
        const uint4 kv = *reinterpret_cast<const uint4*>(p_cand_key + cb + i);
        kk[4 * q] = kv.x; kk[4 * q + 1] = kv.y; kk[4 * q + 2] = kv.z; kk[4 * q + 3] = kv.w;
      }
#pragma unroll
      for (int q = 0; q < P / 4; q++) {
        const int i = tid * P + 4 * q < n_cand ? tid * P + 4 * q : n_cand - 4;
        const int4 pv = *reinterpret_cast<const int4*>(p_cand_pos + cb + i);
        pos[4 * q] = pv.x; pos[4 * q + 1] = pv.y; pos[4 * q + 2] = pv.z; pos[4 * q + 3] = pv.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < P; j++) {
        const int i = tid * P + j < n_cand ? tid * P + j : n_cand - 1;
        kk[j] = p_cand_key[cb + i];
        pos[j] = p_cand_pos[cb + i];
      }
    }
    clear_hist(sh);   // under the loads' latency
    int c = (tid * P) / k, sl = tid * P - c * k;
#pragma unroll
    for (int j = 0; j < P; j++) {
      const int rest = len - c * p_chunk_len;
      const int n_c = rest < 0 ? 0 : rest > k ? k : rest;
      const bool ok = c < p_chunks && sl < n_c;
      kk[j] = ok ? kk[j] : 0u;
      if (ok) { kmin = min(kmin, kk[j]); kmax = max(kmax, kk[j]); }
      if (++sl == k) { sl = 0; c++; }
    }
  } else {
    float f[P];
    issue_row_loads<P>(a.logits + row * a.sl, len, tid * P, a.vec, f);
    clear_hist(sh);   // under the loads' latency
    form_keys<P>(f, len, tid * P, kk);
#pragma unroll
    for (int j = 0; j < P; j++)
      if (tid * P + j < len) { kmin = min(kmin, kk[j]); kmax = max(kmax, kk[j]); }
  }
  const Threshold t = radix_threshold(sh, [&](auto f) { for_each_key(kk, f); }, static_cast<uint32_t>(k), kmin, kmax);
  uint32_t n_eq, n_sel;
  emit_selected(sh, kk, t, 0u, 0u, [&](uint32_t o, int j) {
    if (o < static_cast<uint32_t>(k)) out[o] = kCand ? pos[kCand ? j : 0] : tid * P + j;
  }, &n_eq, &n_sel);
}

// Rows too long for the two stages: one workgroup per row re-reads the row
// (from L2) in sweeps of 32768 positions for each radix pass and for the
// compaction, which carries its counts from sweep to sweep.
__global__ __launch_bounds__(kSweepThreads) void topk_sweep_kernel(const TopkArgs a) {
  __shared__ SelShared<kSweepThreads> sh;
  const int row = blockIdx.x, tid = threadIdx.x;
  const int len = clamp_len(a, row);
  const int k = a.k;
  int32_t* out = a.out + row * a.so;
  if (len <= k) {
    for (int i = tid; i < k; i += kSweepThreads) out[i] = i < len ? i : -1;
    return;
  }
  const float* x = a.logits + row * a.sl;
  const int sweeps = (len + kSweep - 1) / kSweep;
  clear_hist(sh);
  const Threshold t = radix_threshold(sh, [&](auto f) {
    for (int sw = 0; sw < sweeps; sw++) {
      uint32_t kk[kSweepKeys];
      load_row_keys<kSweepKeys>(x + sw * kSweep, len - sw * kSweep, tid * kSweepKeys, a.vec, kk);
      for_each_key(kk, f);
    }
  }, static_cast<uint32_t>(k), 0u, ~0u);
  uint32_t eq_seen = 0, written = 0;
  for (int sw = 0; sw < sweeps; sw++) {
    uint32_t kk[kSweepKeys];
    const int base = sw * kSweep;
    load_row_keys<kSweepKeys>(x + base, len - base, tid * kSweepKeys, a.vec, kk);
    uint32_t n_eq, n_sel;
    emit_selected(sh, kk, t, eq_seen, written, [&](uint32_t o, int j) {
      if (o < static_cast<uint32_t>(k)) out[o] = base + tid * kSweepKeys + j;
    }, &n_eq, &n_sel);
    eq_seen += n_eq;
    written += n_sel;
    __syncthreads();   // the next sweep's scan rewrites sh.wsum
  }
}

bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }

// The per-token logits kernel: the fields of its first loads lead as scalar
// arguments (preloaded into SGPRs), the rest in LogitsArgs.
using LogitsKernel = void (*)(const int32_t*, const int32_t*, int64_t, const uint8_t*, int64_t, int, int, int, int,
                              LogitsArgs);

template <int kTiles, bool kAligned>
LogitsKernel pick_logits_n(int gpw) {
  switch (gpw) {
    case 1: return fp8_paged_mqa_logits_kernel<kTiles, 1, kAligned>;
    case 2: return fp8_paged_mqa_logits_kernel<kTiles, 2, kAligned>;
    case 4: return fp8_paged_mqa_logits_kernel<kTiles, 4, kAligned>;
    case 8: return fp8_paged_mqa_logits_kernel<kTiles, 8, kAligned>;
    default: return fp8_paged_mqa_logits_kernel<kTiles, 16, kAligned>;
  }
}

// Kernel for 16 * tiles heads and gpw groups per wave (unaligned block
// sizes: one group per wave only).
template <bool kAligned>
LogitsKernel pick_logits_kernel(int tiles, int gpw) {
  if constexpr (kAligned) {
    switch (tiles) {
      case 1: return pick_logits_n<1, true>(gpw);
      case 2: return pick_logits_n<2, true>(gpw);
      case 3: return pick_logits_n<3, true>(gpw);
      default: return pick_logits_n<4, true>(gpw);
    }
  } else {
    (void)gpw;
    switch (tiles) {
      case 1: return fp8_paged_mqa_logits_kernel<1, 1, false>;
      case 2: return fp8_paged_mqa_logits_kernel<2, 1, false>;
      case 3: return fp8_paged_mqa_logits_kernel<3, 1, false>;
      default: return fp8_paged_mqa_logits_kernel<4, 1, false>;
    }
  }
}

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
      num_tokens > 65535 || block_size < 1 || num_blocks < 1 || num_blocks > (int64_t(1) << 31) - 1 ||
      max_blocks < 1 || max_len < 0 || max_len > (int64_t(1) << 30) ||
      max_blocks * block_size > (int64_t(1) << 31) - 1 || page_bytes < block_size * (kHeadDim + 4) ||
      sq_h < kHeadDim || sq_t < num_heads * sq_h || sw_t < num_heads || sl_t < max_len ||
      (bt_stride != 0 && bt_stride < max_blocks))
    return GLM53_ERR_BAD_SHAPE;
  if (!aligned(q, 16) || sq_t % 16 || sq_h % 16 || !aligned(kv_cache, 16) || page_bytes % 16 ||
      (block_size * kHeadDim) % 4 || !aligned(weights, 4) || !aligned(logits, 4))
    return GLM53_ERR_MISALIGNED;
  if (num_tokens == 0 || max_len == 0) return 0;
  // Runs of 2^m groups per wave, sized for about 512 workgroups over all
  // rows (one resident round at 2 workgroups per CU), 1 to 16 groups; one
  // group when groups straddle pages (block_size % 16 != 0).
  const bool al = block_size % 16 == 0;
  if (bt_stride == 0 && al && num_tokens >= 16) {
    // one table shared by every row (a request's prefill chunk): 16 rows x 512 keys per workgroup
    constexpr int kRowsN = 32;
    LogitsArgs a{static_cast<const uint8_t*>(q), sq_t, sq_h, static_cast<const uint8_t*>(kv_cache), page_bytes,
                 static_cast<int>(block_size), static_cast<int>(num_blocks), weights, sw_t, context_lens,
                 block_table, 0, static_cast<int>(max_blocks), static_cast<int>(num_heads),
                 static_cast<int>(max_len), 16 * kRowsN, logits, sl_t, clean_logits ? 1 : 0};
    const dim3 grid(static_cast<unsigned>((max_len + 16 * kRowsN - 1) / (16 * kRowsN)),
                    static_cast<unsigned>((num_tokens + 4 * kLogitWaves - 1) / (4 * kLogitWaves)));
    void (*kernel)(LogitsArgs, int);
    switch (num_heads / 16) {
      case 1: kernel = fp8_mqa_logits_rows_kernel<1, kRowsN>; break;
      case 2: kernel = fp8_mqa_logits_rows_kernel<2, kRowsN>; break;
      case 3: kernel = fp8_mqa_logits_rows_kernel<3, kRowsN>; break;
      default: kernel = fp8_mqa_logits_rows_kernel<4, kRowsN>; break;
    }
    (void)hipGetLastError();
    hipLaunchKernelGGL(kernel, grid, dim3(kLogitThreads), 0, static_cast<hipStream_t>(stream), a,
                       static_cast<int>(num_tokens));
    return static_cast<int>(hipGetLastError());
  }
  const int64_t groups = num_tokens * ((max_len + 15) / 16);
  int gpw = 1;
  while (al && gpw < 16 && groups >= int64_t(kLogitWaves) * 512 * gpw * 2) gpw *= 2;
  const int keys_per_wg = 16 * kLogitWaves * gpw;
  LogitsArgs a{static_cast<const uint8_t*>(q), sq_t, sq_h, static_cast<const uint8_t*>(kv_cache), page_bytes,
               static_cast<int>(block_size), static_cast<int>(num_blocks), weights, sw_t, context_lens,
               block_table, bt_stride, static_cast<int>(max_blocks), static_cast<int>(num_heads),
               static_cast<int>(max_len), keys_per_wg, logits, sl_t, clean_logits ? 1 : 0};
  const dim3 grid(static_cast<unsigned>((max_len + keys_per_wg - 1) / keys_per_wg), static_cast<unsigned>(num_tokens));
  (void)hipGetLastError();
  const int tiles = static_cast<int>(num_heads / 16);
  LogitsKernel kernel = al ? pick_logits_kernel<true>(tiles, gpw) : pick_logits_kernel<false>(tiles, 1);
  hipLaunchKernelGGL(kernel, grid, dim3(kLogitThreads), 0, static_cast<hipStream_t>(stream), a.ctx, a.bt,
                     a.bt_stride, a.q, a.sq_t, a.keys_per_wg, a.max_len, a.block_size, a.max_blocks, a);
  return static_cast<int>(hipGetLastError());
}

namespace {

// How the top-k of rows of max_len columns runs: one final workgroup over
// the row (direct, P keys per thread), or the chunk stage (chunks of
// chunk_threads * chunk_p positions, chunk_len > k; 512 threads x 8, 16 or
// 32 keys, or 1024 threads x 8) then the final stage over chunks * k
// candidates, or the sweep kernel.  For a few rows (latency) the chunking
// with the fewest keys per thread over the two stages wins, the first listed
// on a tie: at 65536 positions and k = 512, 1024-thread workgroups over
// 8192-position chunks (4096 candidates) rather than 512 over 4096 (8192
// candidates): B=8 16.4 -> 15.6 us, B=1 11.75 -> 11.66 us.  From 32 rows on
// (throughput: the chunk stage alone is many workgroups per CU) 512-thread
// workgroups over 8192-position chunks, half the workgroups and candidates
// of 4096 (2048 rows x 65536 positions, k = 512: 283 -> 242 us; 32 rows
// 16.6 -> 15.6 us; 16 rows 15.0 -> 15.5 us, so the latency choice stays
// below 32).
struct TopkPlan {
  enum Mode { kDirect, kChunked, kSweepMode } mode;
  int chunk_p, final_p, chunks, chunk_len, chunk_threads;
};

int final_p_for(int64_t n) {
  for (int p : {4, 8, 16, 32})
    if (n <= int64_t(kFinalThreads) * p) return p;
  return 0;
}

constexpr int64_t kTopkThroughputRows = 32;

TopkPlan plan_topk(int64_t num_rows, int64_t max_len, int64_t k) {
  if (max_len <= int64_t(kFinalThreads) * 4) return {TopkPlan::kDirect, 0, 4, 0, 0, 0};
  TopkPlan best{TopkPlan::kSweepMode, 0, 0, 0, 0, 0};
  int best_cost = 1 << 30;
  for (int threads : {kChunkThreads, kChunkThreadsWide}) {
    for (int p : {8, 16, 32}) {
      if (threads == kChunkThreadsWide && p != 8) continue;
      const int64_t len_c = int64_t(threads) * p;
      if (len_c <= k) continue;
      const int64_t chunks = (max_len + len_c - 1) / len_c;
      if (chunks < 2) continue;
      const int fp = final_p_for(chunks * k);
      if (fp == 0) continue;
      const bool throughput = num_rows >= kTopkThroughputRows;
      if (throughput && threads != kChunkThreads) continue;
      const int cost = throughput && p == 16 ? 0 : p + fp;
      if (cost < best_cost) {
        best_cost = cost;
        best = {TopkPlan::kChunked, p, fp, static_cast<int>(chunks), static_cast<int>(len_c), threads};
      }
    }
  }
  if (best.mode == TopkPlan::kSweepMode) {
    const int fp = final_p_for(max_len);
    if (fp) return {TopkPlan::kDirect, 0, fp, 0, 0, 0};
  }
  return best;
}

int64_t topk_ws_bytes(const TopkPlan& p, int64_t rows, int64_t k) {
  if (p.mode != TopkPlan::kChunked) return 0;
  return (rows * p.chunks * k * 8 + 255) / 256 * 256;
}

bool topk_shape_ok(int64_t num_rows, int64_t max_len, int64_t k) {
  return num_rows >= 0 && num_rows <= (int64_t(1) << 30) && k >= 1 && k <= max_len && max_len <= (int64_t(1) << 30);
}

template <int P>
void launch_final(bool cand, dim3 grid, hipStream_t st, const TopkArgs& a) {
  // the fields of the first loads lead as scalar arguments (preloaded into SGPRs)
  void (*kernel)(const int32_t*, int, int, int, uint32_t*, int32_t*, int32_t*, int64_t, int, TopkArgs) =
      cand ? topk_final_kernel<P, true> : topk_final_kernel<P, false>;
  hipLaunchKernelGGL(kernel, grid, dim3(kFinalThreads), 0, st, a.lengths, a.max_len, a.k, a.chunks, a.cand_key,
                     a.cand_pos, a.out, a.so, a.chunk_len, a);
}

}  // namespace

// Enough for every call of at most num_rows rows: the plan switches to
// 512-thread chunks at kTopkThroughputRows rows, whose candidates can take
// less room than the latency plan's at fewer rows, so the query covers the
// largest row count under that switch too.
extern "C" int64_t glm53_indexer_topk_workspace_bytes(int64_t num_rows, int64_t max_len, int64_t k) {
  if (!topk_shape_ok(num_rows, max_len, k)) return 0;
  const int64_t at_rows = topk_ws_bytes(plan_topk(num_rows, max_len, k), num_rows, k);
  const int64_t below = num_rows < kTopkThroughputRows ? num_rows : kTopkThroughputRows - 1;
  const int64_t at_below = topk_ws_bytes(plan_topk(below, max_len, k), below, k);
  return at_rows > at_below ? at_rows : at_below;
}

extern "C" int glm53_indexer_topk(const float* logits, int64_t sl, const int32_t* lengths, int64_t num_rows,
                                  int64_t max_len, int64_t k, void* workspace, int64_t workspace_bytes,
                                  int32_t* out, int64_t so, void* stream) {
  if (!logits || !lengths || !out) return GLM53_ERR_NULL_POINTER;
  if (!topk_shape_ok(num_rows, max_len, k) || sl < max_len || so < k) return GLM53_ERR_BAD_SHAPE;
  if (num_rows == 0) return 0;
  if (!aligned(logits, 4)) return GLM53_ERR_MISALIGNED;
  const TopkPlan plan = plan_topk(num_rows, max_len, k);
  const int64_t need = topk_ws_bytes(plan, num_rows, k);
  if (need && (!workspace || workspace_bytes < need || !aligned(workspace, 16))) return GLM53_ERR_WORKSPACE;
  TopkArgs a{logits, sl, lengths, static_cast<int>(max_len), static_cast<int>(k), out, so, nullptr, nullptr,
             plan.chunks, plan.chunk_len, aligned(logits, 16) && sl % 4 == 0};
  if (need) {
    a.cand_key = static_cast<uint32_t*>(workspace);
    a.cand_pos = reinterpret_cast<int32_t*>(a.cand_key + num_rows * plan.chunks * k);
  }
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 rows_grid(static_cast<unsigned>(num_rows));
  (void)hipGetLastError();
  if (plan.mode == TopkPlan::kSweepMode) {
    hipLaunchKernelGGL(topk_sweep_kernel, rows_grid, dim3(kSweepThreads), 0, st, a);
    return static_cast<int>(hipGetLastError());
  }
  const bool cand = plan.mode == TopkPlan::kChunked;
  if (cand) {
    const dim3 grid(static_cast<unsigned>(num_rows), static_cast<unsigned>(plan.chunks));
    // the fields of the first loads lead as scalar arguments (preloaded into SGPRs)
#define CHUNK_LEAD a.logits, a.sl, a.lengths, a.max_len, a.k, a.chunk_len, a.chunks, a.vec ? 1 : 0, a
    if (plan.chunk_threads == kChunkThreadsWide)
      hipLaunchKernelGGL((topk_chunk_kernel<8, kChunkThreadsWide>), grid, dim3(kChunkThreadsWide), 0, st,
                         CHUNK_LEAD);
    else switch (plan.chunk_p) {
      case 8:
        hipLaunchKernelGGL((topk_chunk_kernel<8, kChunkThreads>), grid, dim3(kChunkThreads), 0, st, CHUNK_LEAD);
        break;
      case 16:
        hipLaunchKernelGGL((topk_chunk_kernel<16, kChunkThreads>), grid, dim3(kChunkThreads), 0, st, CHUNK_LEAD);
        break;
      default:
        hipLaunchKernelGGL((topk_chunk_kernel<32, kChunkThreads>), grid, dim3(kChunkThreads), 0, st, CHUNK_LEAD);
        break;
    }
#undef CHUNK_LEAD
  }
  switch (plan.final_p) {
    case 4: launch_final<4>(cand, rows_grid, st, a); break;
    case 8: launch_final<8>(cand, rows_grid, st, a); break;
    case 16: launch_final<16>(cand, rows_grid, st, a); break;
    default: launch_final<32>(cand, rows_grid, st, a); break;
  }
  return static_cast<int>(hipGetLastError());
}
