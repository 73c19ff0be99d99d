// Sparse NoPE MLA decode over the 528-byte INT8 cache for gfx950.
//
// Behaviour of kernels/titan_mla.py: for each query token t and head h,
//   logit_j = (q_h . k_j) * scale_j * fp32(sm_scale * log2 e)      (base 2)
//   out_h   = sum_j softmax_j * v_j,   v_j = k_j = int8 row j,
// with the online softmax of _sparse_mla_compute_tile (:117-180): per tile a
// running max m, p = exp2(logit - m), the PV operand bf16(p * scale_j), the
// denominator l += sum p; indices outside [0, seq_kv) masked (-1e30, p = 0).
// With num_splits > 1 each split writes acc / l and the natural-log LSE
// (m + log2 l) * ln 2 (:330-354) and a merge kernel combines them (:403-429);
// with one split the kernel writes bf16(acc / l) directly (:245-255).
//
// Work decomposition (one workgroup = one (split, token, 16-head group)):
//   * 8 wavefronts = 2 key groups x 4 latent slices.  Wave w owns latent
//     columns [128 s, 128 s + 128) with s = w % 4, and the tiles of 32 keys of
//     key group w / 4 (even / odd tiles), each key group running its own
//     online softmax; the two are merged through LDS at the end.  Two waves
//     per SIMD interleave their tiles, hiding each other's latencies.
//     Splits of exactly three tiles (65-96 keys: B=8's 23 splits) take a
//     12-wave variant, 3 key groups x 4 slices, that consumes them in one
//     round instead of two (the second with one group idle); one-tile
//     splits (B=1's 68) a 4-wave variant, one key group, whose partials
//     leave the accumulators with no LDS combine.
//   * Lane (g = lane / 16, c = lane % 16) gathers 32 bytes of its wave's
//     slice from keys c and 16 + c of a tile: four 16-byte loads per tile,
//     slice bytes 16g + [0, 16) and 64 + 16g + [0, 16), so each load
//     instruction covers whole 64-byte halves of the slice.
//     The gathers of a whole chunk (8 tiles, 256 keys) are issued before any
//     is consumed, so a decode split pays one index and one row latency.
//   * S^T = K Q^T on v_mfma_f32_16x16x32_bf16: A = 16 keys x 32 latents
//     (int8 converted to bf16 in registers), B = Q^T, 4 K-steps per wave;
//     the four slices' partial S^T are summed through LDS in a fixed order.
//   * The C layout of S^T gives lane (g, c) head c and keys {4g+i, 16+4g+i}:
//     exactly the B operand P^T of O^T = V^T P^T, so the softmax needs no
//     shuffle of P; the per-head max and sum over the four 16-lane rows use
//     v_permlane16_swap / v_permlane32_swap (VALU, no LDS round trip).
//   * V^T comes from the same gathered rows: each wave stores its bf16 slice
//     row-major in LDS and reads it back with ds_read_b64_tr_b16 (two reads
//     per 16x32 operand).  O^T accumulates in 8 MFMA tiles per wave.
//   * Splits longer than one chunk (the prefill-shaped call's single split
//     of 2176 keys per token) run sparse_mla_pair_kernel instead: two waves
//     per (token, 16-head group) share one online-softmax stream over the
//     split's tiles in order.
//   * Workgroups are numbered so that a token's splits share an XCD (its L2
//     holds the token's q and indices, and the merge kernel is numbered the
//     same way); see sparse_mla_kernel.
#include "glm53_common.h"

#include <atomic>

namespace glm53 {
namespace {

constexpr int kLatent = 512;
constexpr int kHeads = 16;       // heads per workgroup (one MFMA M/N tile)
constexpr int kTile = 32;        // keys per tile
constexpr int kSlices = 4;       // latent slices of 128
constexpr int kGroups = 2;       // key groups
constexpr int kWaves = kSlices * kGroups;
constexpr int kThreads = 64 * kWaves;
constexpr int kSlice = kLatent / kSlices;
constexpr int kVStride = kSlice + 16;  // bf16 per LDS row: 288 bytes, rows 8 banks apart
constexpr int kChunkTiles = 8;         // tiles whose gathers are in flight together
constexpr int kMergeLanes = 8;         // split lanes per output chunk in the LSE merge
constexpr int kMaxMergeSplits = 1024;
constexpr int kMaxGridTokens = 65535;   // query tokens per call: the split kernel's grid y
constexpr float kNegLarge = -1.0e30f;
constexpr float kLn2 = 0.6931471805599453f;

struct MlaArgs {
  const uint16_t* q;
  int64_t sq_t, sq_h;
  const uint8_t* kv;
  int64_t skv;
  int64_t seq_kv;
  const int32_t* idx;
  int64_t si_t;
  int num_heads;
  int topk;
  int num_splits;
  int split_len;
  float scale_log2;
  float* part;    // fp32 blocks of 16 heads x 512 per (t, split, head group), accumulator order (part_block)
  float* lse;     // [T][S][Hp]
  int heads_padded;
  uint16_t* out;
  int64_t so_t, so_h;
  int partials_only;   // write part/lse even for a single split
  int out_align16;     // out rows 16-byte aligned (else 8-byte stores)
  // Paged indices (sparse_mla_kernel<true>): idx holds request-relative
  // token positions, mapped by to_page_unit to the row's 16-byte unit in a
  // paged cache (kv = page 0, pages page_units units apart, rows row_units
  // units apart within a page).
  const int32_t* req_id;   // [T] request of each query token
  const int32_t* bt;       // block table, row r at bt + r * bt_stride
  int64_t bt_stride;
  int max_blocks;          // entries per block-table row
  int num_reqs;            // block-table rows: other request ids map to -1
  int block_size;          // tokens per cache block
  int num_blocks;          // physical pages: other table entries map to -1
  int page_units;          // page stride / 16
  int row_units;           // row stride / 16
  // Pooled positions (kPooledPos): slot k of token t comes from
  // pooled_position(pools + t * sp_t, num_pools, pool_size, seq_lens[t], k).
  const int32_t* pools;
  int64_t sp_t;
  int num_pools;
  int pool_size;
  const int32_t* seq_lens; // nullptr: no tail slots
};

__device__ __forceinline__ float f4_get(const float4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// 2^x on the hardware exponential (v_exp_f32); results below 2^-126 flush to
// 0, which only drops softmax weights smaller than 1e-38.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Max / sum of v over the four 16-lane rows at the same column, returned to
// every lane in the same summation order: rows (0,1) and (2,3) are paired by
// v_permlane16_swap, then the halves by v_permlane32_swap.
__device__ __forceinline__ float rows_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// 16 int8 (one uint4) -> two bf16x8 (exact: |v| <= 128 fits bf16).
__device__ __forceinline__ void i8x16_to_bf16(const uint4 v, bf16x8& lo, bf16x8& hi) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint32_t o[8];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int32_t x = static_cast<int32_t>(w[k]);
    const float f0 = static_cast<float>((x << 24) >> 24);
    const float f1 = static_cast<float>((x << 16) >> 24);
    const float f2 = static_cast<float>((x << 8) >> 24);
    const float f3 = static_cast<float>(x >> 24);
    // exact small integers: the bf16 pattern is the high half of the fp32 one
    o[2 * k] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
    o[2 * k + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
  }
  uint4 a = make_uint4(o[0], o[1], o[2], o[3]);
  uint4 b = make_uint4(o[4], o[5], o[6], o[7]);
  lo = __builtin_bit_cast(bf16x8, a);
  hi = __builtin_bit_cast(bf16x8, b);
}

// Shape of the split kernel for kG key groups of kSlices waves: two groups
// take chunks of 8 tiles in 4 rounds (any decode split); three take one
// round of 3 tiles (splits of 65-96 keys: B=8's 23 splits of 95 keys in one
// round instead of two); one takes a single tile (splits of at most 32).
template <int kG>
struct SplitShape {
  static constexpr int kWaves = kSlices * kG;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kChunkTiles = kG == 2 ? 8 : kG;
  static constexpr int kRounds = kChunkTiles / kG;
  static constexpr int kRedBufs = kRounds > 1 ? 2 : 1;   // partial S^T double-buffered across rounds
};

template <int kG>
struct __attribute__((aligned(16))) MlaShared {
  using S = SplitShape<kG>;
  uint16_t vbuf[S::kWaves][kTile][kVStride];         // per-wave bf16 V slice of a tile, then its parked acc
  float ml[kG][kHeads][2];                             // each key group's (m, l) per head
  float4 red[S::kRedBufs][kG][kSlices][2][64];         // partial S^T per slice: [half][lane]
  float scl[2][S::kChunkTiles][kTile];                 // row scales of the chunk
};

// Request-relative token position -> flat cache row, the conversion vLLM's
// triton_convert_req_index_to_global_index performs before the reference's
// attention call (integration/titan_backend.py:48-52): a negative position,
// or one whose block lies beyond the block-table row, gives -1; otherwise
// block_table[req][pos / block_size] * page_rows + pos % block_size, in
// wrapping 32-bit arithmetic like the Triton kernel.  page_rows is the
// padded page's row count in the flat view (BLOCK_STRIDE_ROWS; block_size
// when pages are unpadded).
__device__ __forceinline__ int to_flat_row(const int32_t* bt_req, int max_blocks, int block_size,
                                           int page_rows, int pos) {
  if (pos < 0) return -1;
  const int blk = pos / block_size;
  if (blk >= max_blocks) return -1;
  const int off = pos - blk * block_size;
  return static_cast<int>(static_cast<uint32_t>(bt_req[blk]) * static_cast<uint32_t>(page_rows) +
                          static_cast<uint32_t>(off));
}

// The fused gather's form of the same mapping: the 16-byte unit of the
// row in the paged cache, or -1 (also for a table entry that is not one of
// the num_blocks pages, which the flat-row form leaves to the attention's
// row mask).  The host keeps num_blocks * page_units below 2^31.
__device__ __forceinline__ int to_page_unit(const int32_t* bt_req, int max_blocks, int block_size,
                                            int num_blocks, int page_units, int row_units, int pos) {
  if (pos < 0) return -1;
  const int blk = pos / block_size;
  if (blk >= max_blocks) return -1;
  const int phys = bt_req[blk];
  if (phys < 0 || phys >= num_blocks) return -1;
  return phys * page_units + (pos - blk * block_size) * row_units;
}

// Index modes of the attention kernel.
constexpr int kFlatRows = 0;   // indices are rows of a flat cache
constexpr int kPagedPos = 1;   // request-relative positions into a paged cache
constexpr int kPooledPos = 2;  // positions expanded from top-k pool ids, then paged

// Token position held by slot k of a row expanded from pool ids, as the
// indexer's kpool expansion lays it out (model: tests/verify_indexer_sharding.py:
// 72-79): slot k < num_pools * pool_size is token pool[k / pool_size] *
// pool_size + k % pool_size (-1 for a negative pool id); the next
// pool_size - 1 slots, when seq_len >= 0, are the tail tokens
// seq_len / pool_size * pool_size + j for j < seq_len % pool_size (-1
// otherwise); later slots are -1.
// pool(j) returns pool id j as an int (-1 for an invalid id).
template <class PoolAt>
__device__ __forceinline__ int pooled_position(PoolAt pool, int num_pools, int pool_size, int seq_len,
                                               int k) {
  const int expanded = num_pools * pool_size;
  if (k < expanded) {
    const int pid = pool(k / pool_size);
    return pid >= 0 ? pid * pool_size + k % pool_size : -1;
  }
  const int j = k - expanded;
  if (seq_len < 0 || j >= pool_size - 1) return -1;
  return j < seq_len % pool_size ? seq_len / pool_size * pool_size + j : -1;
}

// V slice element (row, col) in LDS.  The LDS serves 128 bytes (32 banks of
// 4 bytes) per pass: a ds_read_b64_tr_b16 pass is 16 lanes (4 rows x 32
// bytes), a ds_write_b128 pass 8 lanes (8 rows x 16 bytes).  Rows are 288
// bytes (72 dwords, 8 banks) apart, so the four rows of a transposing read
// land on distinct banks; rows r and r + 4 would then share banks in a
// write pass, so the 16-byte chunks of rows 4-7 of every 8 (row bit 2) are
// XOR-swapped in pairs, which the 4-row-aligned reads do not see.  (With
// the swap on row bit 3 instead, every 16-byte V write cost 8 conflict
// cycles: SQ_LDS_BANK_CONFLICT, 64 per 32-key tile per wave.)
// Wave w's parked accumulators: its V buffer holding the wave's 8 MFMA
// accumulator tiles in register order (float4 of lane l of tile dt at
// (64 dt + l) * 4): each 16-byte write and read instruction covers 1 KB.
template <class Shared>
__device__ __forceinline__ float* park_of(Shared& sh, int w) {
  static_assert(8 * 64 * 16 <= kTile * kVStride * 2, "a wave's park fits its V buffer");
  return reinterpret_cast<float*>(&sh.vbuf[w][0][0]);
}

// Split partials in the accumulator order.  Per (token, split, head group)
// one block of 16 heads x 512 latents; within it the float4 at
// ((8 sl + dt) * 64 + 16 g + c) * 4 holds head c, latents 128 sl + 16 dt +
// 4 g + [0, 4) -- what lane (g, c) of latent slice sl holds in accumulator
// tile dt -- so every store instruction of a wave writes 1 KB contiguously.
__device__ __forceinline__ float* part_block(const MlaArgs& a, int t, int split, int hg) {
  return a.part + ((static_cast<int64_t>(t) * a.num_splits + split) * (a.heads_padded / kHeads) + hg) *
                      (kHeads * kLatent);
}

// A 16-byte store written through to device scope (cache policy sc1) at
// byte `off` of the uniform `base`: the key-group kernels' split partials,
// which the merge kernel reads after the kernel boundary.  Written through,
// they leave no dirty lines for the boundary's L2 writeback to flush and wait
// for the merge in the memory-side cache (B=8 over rotating caches 11.40 ->
// 11.10 us per step, warm 11.16 -> 10.77, B=4 10.39 -> 10.25, paged B=8 11.85
// -> 11.61 against non-temporal stores; plain stores, sc0 + sc1 and
// non-temporal + sc1 measured alike or slower; the one-key-group kernel's
// partials keep plain stores, its B=1 step did not gain).
__device__ __forceinline__ void store_through(float* base, int off, const float4 v) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, kHeads * kLatent * 4, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(
      u32x4{__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)}, r, off, 0,
      16 /* sc1 */);
}

template <class Shared>
__device__ __forceinline__ uint16_t* vbuf_at(Shared& sh, int w, int row, int col) {
  const int chunk = (col >> 3) ^ ((row >> 2) & 1);
  return &sh.vbuf[w][row][(chunk << 3) | (col & 7)];
}

// The fields a split workgroup needs before its first loads come ahead of
// MlaArgs as scalar arguments (the grid dims among them): the library is
// built to preload the first 16 dwords of scalar arguments into SGPRs, so
// these arrive with the wave instead of through a scalar load that would
// head the index -> row chain.
template <int kMode, bool kPipe, int kG, bool kPad = false>
__global__ __launch_bounds__(SplitShape<kG>::kThreads) void sparse_mla_kernel(
    const int32_t* idx, int64_t si_t, int split_len, int topk, int grid_x, int grid_y, int grid_z, int num_heads,
    const uint16_t* q, int64_t sq_t, int64_t sq_h, const MlaArgs a) {
  constexpr bool kPaged = kMode != kFlatRows;
  constexpr int kChunkTiles = SplitShape<kG>::kChunkTiles;
  constexpr int kRounds = SplitShape<kG>::kRounds;
  constexpr int kRedBufs = SplitShape<kG>::kRedBufs;
  static_assert(kG == 2 || !kPipe, "three key groups take single-chunk splits only");
  __shared__ MlaShared<kG> sh;

  // Workgroups go to the 8 XCDs round robin by linear id; numbering the
  // (token, head group) units fastest puts all splits of a unit on one XCD
  // when there are a multiple of 8 units (B=8: token t on XCD t), and on
  // two XCDs for a multiple of 4 (B=4: token t on XCDs t and t + 4; 10.83
  // -> 10.37 us per call over rotating caches), where the merge kernel
  // reads them back.
  // kPad: batches of 3, 5, 6 or 7 tokens are numbered as 4 or 8 (grid_y
  // holds the numbered tokens in its low 16 bits, the batch's in the high
  // 16); the extra tokens' workgroups return at once.  (B=1 and B=2 keep the
  // plain mapping: at B=1 the divisions cost 0.35 us for nothing, and B=2
  // gains nothing from four XCDs per token.)
  const int gy = kPad ? (grid_y & 0xffff) : grid_y;
  int split = blockIdx.x, t = blockIdx.y, hg = blockIdx.z;
  if ((gy * grid_z) % 4 == 0) {
    const int lin = blockIdx.x + grid_x * (blockIdx.y + gy * blockIdx.z);
    const int units = gy * grid_z;
    split = lin / units;
    t = (lin % units) % gy;
    hg = (lin % units) / gy;
  }
  if (kPad && t >= static_cast<int>(static_cast<unsigned>(grid_y) >> 16)) return;   // uniform
  const int w = uniform(threadIdx.x >> 6);
  const int sl = w & (kSlices - 1);
  const int kg = w / kSlices;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int start = split * split_len;
  const int end = min(start + split_len, topk);
  const int head = hg * kHeads + c;
  const bool head_ok = head < num_heads;
  const int32_t* idx_t = idx + t * si_t;
  // A request id outside the block table maps every index to -1.
  const int req = kPaged ? a.req_id[t] : 0;
  const bool req_ok = req >= 0 && req < a.num_reqs;
  const int32_t* bt_req = kPaged && req_ok ? a.bt + static_cast<int64_t>(req) * a.bt_stride : a.bt;
  const int max_blocks = req_ok ? a.max_blocks : 0;
  const int32_t* pools_t = kMode == kPooledPos ? a.pools + t * a.sp_t : nullptr;
  const int seq_len_t = kMode == kPooledPos && a.seq_lens ? a.seq_lens[t] : -1;

  f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegLarge, l_run = 0.f;
  bool acc_zero = true;  // wave-uniform: no PV product accumulated yet

  // kPipe (splits of several chunks): the next chunk's indices are
  // requested before this chunk's first rounds and its rows after its first
  // half, so their latency overlaps this chunk's compute.  Without kPipe
  // (one-chunk decode splits) a chunk's loads are issued at its start.
  // Index addresses are clamped into the split; positions past it become -1
  // and load no rows.
  auto load_ids = [&](int c0, int (&id)[kRounds]) {
#pragma unroll
    for (int r = 0; r < kRounds; r++) {
      const int pos = c0 + (kG * r + kg) * kTile + (lane & 31);
      int v;
      if (kMode == kPooledPos)
        v = pos < end ? pooled_position([&](int j) { return pools_t[j]; }, a.num_pools, a.pool_size,
                                        seq_len_t, pos)
                      : -1;
      else if (kPipe)
        v = idx_t[min(pos, end - 1)];   // unconditional: the prefetch needs no branch
      else
        v = pos < end ? idx_t[pos] : -1;
      id[r] = v;
    }
  };
  auto issue_rows = [&](int c0, const int (&raw)[kRounds], uint4 (&kd)[kRounds][2][2], float (&sv)[kRounds],
                        uint32_t (&vmask)[kRounds]) {
#pragma unroll
    for (int r = 0; r < kRounds; r++) {
      const int pos = c0 + (kG * r + kg) * kTile + (lane & 31);
      int v = pos < end ? raw[r] : -1;
      if (kPaged)
        v = to_page_unit(bt_req, max_blocks, a.block_size, a.num_blocks, a.page_units, a.row_units, v);
      else if (v < 0 || static_cast<int64_t>(v) >= a.seq_kv)
        v = -1;
      // The row scale first: issued after the rows, its load waited for them
      // (its register reused one of theirs), a second round trip per split.
      sv[r] = 0.f;
      if (sl == 0 && lane < kTile && v >= 0)
        sv[r] = *reinterpret_cast<const float*>(a.kv + static_cast<int64_t>(v) * (kPaged ? 16 : a.skv) +
                                                kLatent);
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int kid = __shfl(v, 16 * u + c, 64);
        kd[r][u][0] = make_uint4(0, 0, 0, 0);
        kd[r][u][1] = make_uint4(0, 0, 0, 0);
        if (kid >= 0) {
          const uint4* rp = reinterpret_cast<const uint4*>(
              a.kv + static_cast<int64_t>(kid) * (kPaged ? 16 : a.skv) + kSlice * sl + 16 * g);
          kd[r][u][0] = rp[0];   // slice bytes 16g + [0, 16): with the 3 other lane groups, its first 64 bytes
          kd[r][u][1] = rp[4];   // slice bytes 64 + 16g + [0, 16): its last 64
        }
      }
      vmask[r] = static_cast<uint32_t>(__ballot(v >= 0));
    }
  };

  int buf = 0, cbuf = 0;
  int idc[kRounds], idn[kRounds];
  uint4 kdc[kRounds][2][2], kdn[kRounds][2][2];
  float svc[kRounds], svn[kRounds];
  uint32_t vmc[kRounds], vmn[kRounds];
  if (kPipe && start < end) {
    load_ids(start, idc);
    issue_rows(start, idc, kdc, svc, vmc);
  }
  // A one-chunk (decode) split requests its indices before q: they head the
  // dependent index -> row chain, while q is first needed by the products.
  // Its chunk runs outside any loop, so no loop-carried wait makes the index
  // load wait for q.
  if (!kPipe && start < end) load_ids(start, idc);

  // Q^T fragment (B operand of S^T = K Q^T): head c, latents 128 sl + 16g +
  // [0, 16) and 128 sl + 64 + 16g + [0, 16) -> four K-steps of 8 (the same
  // latents as the lane's gathered key bytes).
  // The loads are unconditional (a padded head reads head 0 and is zeroed
  // after): under a branch the compiler's wait for the index load would also
  // wait for them.
  bf16x8 qf[4];
  {
    const uint4* qp = reinterpret_cast<const uint4*>(q + t * sq_t + (head_ok ? head : 0) * sq_h +
                                                     kSlice * sl + 16 * g);
    const uint4 z = make_uint4(0, 0, 0, 0);
    const uint4 q0 = qp[0], q1 = qp[1], q2 = qp[8], q3 = qp[9];
    qf[0] = __builtin_bit_cast(bf16x8, head_ok ? q0 : z);
    qf[1] = __builtin_bit_cast(bf16x8, head_ok ? q1 : z);
    qf[2] = __builtin_bit_cast(bf16x8, head_ok ? q2 : z);
    qf[3] = __builtin_bit_cast(bf16x8, head_ok ? q3 : z);
  }
  if (!kPipe && start < end) issue_rows(start, idc, kdc, svc, vmc);

  auto consume_chunk = [&](const int c0) {
    const int c1 = c0 + kChunkTiles * kTile;
    if (sl == 0 && lane < kTile) {
#pragma unroll
      for (int r = 0; r < kRounds; r++) sh.scl[cbuf][kG * r + kg][lane] = svc[r];
    }
    if (kPipe) load_ids(c1, idn);

    // ---- consume the chunk: one tile per key group per round.
#pragma unroll
    for (int r = 0; r < kRounds; r++, buf ^= 1) {
      if (kPipe && r == kRounds / 2) issue_rows(c1, idn, kdn, svn, vmn);   // next chunk's rows (-1 past the split)
      if (c0 + kG * r * kTile >= end) continue;                  // uniform across the workgroup
      const bool has_tile = c0 + (kG * r + kg) * kTile < end;    // uniform across the wave
      uint4 (&kd)[kRounds][2][2] = kdc;
      uint32_t (&vmask)[kRounds] = vmc;

      if (has_tile) {
        f32x4 s_part[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
          bf16x8 k01, k23, k45, k67;
          i8x16_to_bf16(kd[r][u][0], k01, k23);
          i8x16_to_bf16(kd[r][u][1], k45, k67);
          f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
          sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k01, qf[0], sacc, 0, 0, 0);
          sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k23, qf[1], sacc, 0, 0, 0);
          sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k45, qf[2], sacc, 0, 0, 0);
          sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k67, qf[3], sacc, 0, 0, 0);
          s_part[u] = sacc;
          // V slice for the PV product: row 16u + c, latents 16g + [0, 16) and 64 + 16g + [0, 16).
          const int vrow = 16 * u + c;
          *reinterpret_cast<uint4*>(vbuf_at(sh, w, vrow, 16 * g)) = __builtin_bit_cast(uint4, k01);
          *reinterpret_cast<uint4*>(vbuf_at(sh, w, vrow, 16 * g + 8)) = __builtin_bit_cast(uint4, k23);
          *reinterpret_cast<uint4*>(vbuf_at(sh, w, vrow, 64 + 16 * g)) = __builtin_bit_cast(uint4, k45);
          *reinterpret_cast<uint4*>(vbuf_at(sh, w, vrow, 64 + 16 * g + 8)) = __builtin_bit_cast(uint4, k67);
        }
        sh.red[buf % kRedBufs][kg][sl][0][lane] = make_float4(s_part[0][0], s_part[0][1], s_part[0][2], s_part[0][3]);
        sh.red[buf % kRedBufs][kg][sl][1][lane] = make_float4(s_part[1][0], s_part[1][1], s_part[1][2], s_part[1][3]);
      }
      __syncthreads();
      if (!has_tile) continue;

      const int tile = kG * r + kg;
      const float4 sc0 = *reinterpret_cast<const float4*>(&sh.scl[cbuf][tile][4 * g]);
      const float4 sc1 = *reinterpret_cast<const float4*>(&sh.scl[cbuf][tile][16 + 4 * g]);
      const float sc[8] = {sc0.x, sc0.y, sc0.z, sc0.w, sc1.x, sc1.y, sc1.z, sc1.w};
      const uint32_t kv_ok = ((vmask[r] >> (4 * g)) & 0xfu) | (((vmask[r] >> (16 + 4 * g)) & 0xfu) << 4);

      // Full scores (fixed summation order over the four slices).
      float s[8];
      {
        float4 rr[kSlices][2];
#pragma unroll
        for (int ss = 0; ss < kSlices; ss++) {
          rr[ss][0] = sh.red[buf % kRedBufs][kg][ss][0][lane];
          rr[ss][1] = sh.red[buf % kRedBufs][kg][ss][1][lane];
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
          float v = f4_get(rr[0][j >> 2], j & 3);
          v += f4_get(rr[1][j >> 2], j & 3);
          v += f4_get(rr[2][j >> 2], j & 3);
          v += f4_get(rr[3][j >> 2], j & 3);
          v *= sc[j];
          v *= a.scale_log2;
          s[j] = (kv_ok >> j) & 1 ? v : kNegLarge;
        }
      }
      float mx = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
      mx = rows_max(mx);
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);
      float pr[8];
#pragma unroll
      for (int j = 0; j < 8; j++) pr[j] = (kv_ok >> j) & 1 ? fast_exp2(s[j] - m_new) : 0.f;
      float psum = ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
      psum = rows_sum(psum);
      l_run = l_run * alpha + psum;
      m_run = m_new;

      // P^T operand: k-slot 8g + j <-> key 16(j/4) + 4g + (j%4).
      const uint4 pw = make_uint4(pack_bf16x2(pr[0] * sc[0], pr[1] * sc[1]),
                                  pack_bf16x2(pr[2] * sc[2], pr[3] * sc[3]),
                                  pack_bf16x2(pr[4] * sc[4], pr[5] * sc[5]),
                                  pack_bf16x2(pr[6] * sc[6], pr[7] * sc[7]));
      const bf16x8 pb = __builtin_bit_cast(bf16x8, pw);

      // The running max changes rarely after the first tiles: rescale only
      // when it moved for some head of this wave (alpha == 1 otherwise), and
      // not before the wave's first PV product (acc is still exactly 0).
      if (!acc_zero && __ballot(alpha != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
          acc[dt][0] *= alpha; acc[dt][1] *= alpha; acc[dt][2] *= alpha; acc[dt][3] *= alpha;
        }
      }
      // O^T += V^T P^T for the 8 latent tiles of this wave.
      // ds_read_b64_tr_b16: in each 16-lane group, lane 4r + q addresses row r,
      // columns [4q, 4q + 4); lane c receives column c of the 4 rows.
      const int tr_row = 4 * g + (c >> 2);
      const int tr_col = 4 * (c & 3);
#pragma unroll
      for (int dt = 0; dt < 8; dt++) {
        const i16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            GLM53_LDS(i16x4, vbuf_at(sh, w, tr_row, 16 * dt + tr_col)));
        const i16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            GLM53_LDS(i16x4, vbuf_at(sh, w, 16 + tr_row, 16 * dt + tr_col)));
        const i32x2 v0i = __builtin_bit_cast(i32x2, v0);
        const i32x2 v1i = __builtin_bit_cast(i32x2, v1);
        const uint4 vv = make_uint4(v0i[0], v0i[1], v1i[0], v1i[1]);
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vv), pb, acc[dt], 0, 0, 0);
      }
      acc_zero = false;
    }
  };
  if constexpr (kPipe) {
    for (int c0 = start; c0 < end; c0 += kChunkTiles * kTile, cbuf ^= 1) {
      consume_chunk(c0);
#pragma unroll
      for (int r = 0; r < kRounds; r++) {
        vmc[r] = vmn[r];
        svc[r] = svn[r];
#pragma unroll
        for (int u = 0; u < 2; u++) {
          kdc[r][u][0] = kdn[r][u][0];
          kdc[r][u][1] = kdn[r][u][1];
        }
      }
    }
  } else if (start < end) {
    consume_chunk(start);   // split_len <= kChunkTiles * kTile: one chunk
  }

  // ---- one key group: nothing to merge.  Each wave stores its 16 heads x
  // 128 latents straight from its accumulators, with no LDS round trip and
  // no barrier: the partials are in the accumulator order (1 KB per store
  // instruction); a single split's bf16 rows take 8 bytes per lane.
  if constexpr (kG == 1) {
    const float inv_l = 1.f / (l_run > 0.f ? l_run : 1.f);
    const bool direct = a.num_splits == 1 && !a.partials_only;
    if (direct) {
      if (!head_ok) return;
#pragma unroll
      for (int dt = 0; dt < 8; dt++) {
        const int col = kSlice * sl + 16 * dt + 4 * g;   // head c, latents 128 sl + 16 dt + 4 g + [0, 4)
        *reinterpret_cast<uint2*>(a.out + t * a.so_t + head * a.so_h + col) =
            make_uint2(pack_bf16x2(acc[dt][0] * inv_l, acc[dt][1] * inv_l),
                       pack_bf16x2(acc[dt][2] * inv_l, acc[dt][3] * inv_l));
      }
      return;
    }
    float* pb = part_block(a, t, split, hg) + (8 * sl * 64 + lane) * 4;
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
      *reinterpret_cast<float4*>(pb + dt * 64 * 4) =
          make_float4(acc[dt][0] * inv_l, acc[dt][1] * inv_l, acc[dt][2] * inv_l, acc[dt][3] * inv_l);
    if (head_ok && sl == 0 && g == 0)
      a.lse[(static_cast<int64_t>(t) * a.num_splits + split) * a.heads_padded + head] = (m_run + log2f(l_run)) * kLn2;
    return;
  } else {
  // ---- combine the key groups.  Accumulator tile dt of every slice belongs
  // to key group dt * kG / 8 (3-3-2 tiles for three groups, 4-4 for two):
  // each wave parks the tiles that other groups own in its V buffer (register
  // order, 1 KB per instruction) and writes its (m, l); after one barrier
  // every wave adds the other groups' parked copies of its own tiles to its
  // registers, in group order (x0 a0 + x1 a1) + x2 a2, and stores them
  // straight from registers in the partials' accumulator order (1 KB per
  // instruction; a single split's bf16 rows take 8 bytes per lane).
  auto owner = [](int dt) { return dt * kG / 8; };
  {
    float* pk = park_of(sh, w) + 4 * lane;
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
      if (owner(dt) != kg)
        *reinterpret_cast<float4*>(pk + dt * 64 * 4) = make_float4(acc[dt][0], acc[dt][1], acc[dt][2], acc[dt][3]);
  }
  if (sl == 0 && g == 0) {
    sh.ml[kg][c][0] = m_run;
    sh.ml[kg][c][1] = l_run;
  }
  __syncthreads();
  float mg[kG], ag[kG];
  float mm = kNegLarge;
#pragma unroll
  for (int i = 0; i < kG; i++) {
    mg[i] = sh.ml[i][c][0];
    mm = i == 0 ? mg[0] : fmaxf(mm, mg[i]);
  }
  float l = 0.f;
#pragma unroll
  for (int i = 0; i < kG; i++) {
    ag[i] = fast_exp2(mg[i] - mm);
    const float li = sh.ml[i][c][1] * ag[i];
    l = i == 0 ? li : l + li;
  }
  // 1 / l once, then multiplies (the reference divides; the two differ by
  // at most one fp32 ulp before the bf16 / fp32 store).
  const float inv_l = 1.f / (l > 0.f ? l : 1.f);
  const bool direct = a.num_splits == 1 && !a.partials_only;
#pragma unroll
  for (int dt = 0; dt < 8; dt++) {
    if (owner(dt) != kg) continue;   // uniform across the wave
    float4 v;
#pragma unroll
    for (int i = 0; i < kG; i++) {
      const float4 x = i == kg ? make_float4(acc[dt][0], acc[dt][1], acc[dt][2], acc[dt][3])
                               : *reinterpret_cast<const float4*>(park_of(sh, i * kSlices + sl) + (dt * 64 + lane) * 4);
      v = i == 0 ? make_float4(x.x * ag[0], x.y * ag[0], x.z * ag[0], x.w * ag[0])
                 : make_float4(v.x + x.x * ag[i], v.y + x.y * ag[i], v.z + x.z * ag[i], v.w + x.w * ag[i]);
    }
    v = make_float4(v.x * inv_l, v.y * inv_l, v.z * inv_l, v.w * inv_l);
    if (direct) {
      const int col = kSlice * sl + 16 * dt + 4 * g;   // head c, latents 128 sl + 16 dt + 4 g + [0, 4)
      if (head_ok)
        *reinterpret_cast<uint2*>(a.out + t * a.so_t + head * a.so_h + col) =
            make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
    } else {
      store_through(part_block(a, t, split, hg), ((8 * sl + dt) * 64 + lane) * 16, v);
    }
  }
  if (!direct && head_ok && kg == 0 && sl == 0 && g == 0)
    a.lse[(static_cast<int64_t>(t) * a.num_splits + split) * a.heads_padded + head] = (mm + log2f(l)) * kLn2;
  }
}

// ---------------------------------------------------------------- long splits: waves in pairs
// Splits of more than one chunk of flat-row indices (the prefill-shaped call:
// one split of 2176 keys per token) take this kernel.  One workgroup of two
// waves per (split, token, 16-head group) runs a single online-softmax stream
// over the split's 32-key tiles in order -- the loop structure of
// _sparse_mla_compute_tile with BLOCK_N = 32 -- and the two waves split the
// latent: wave w gathers, converts and multiplies latents [256 w, 256 w + 256)
// of every key.
//   * S^T = K Q^T per 16-key half on v_mfma_f32_16x16x32_bf16 over the wave's
//     256 latents (8 K-steps); the two waves' partial S^T meet in LDS (one
//     barrier per tile) and both add them in the same order, so both run the
//     same softmax on the same scores.  Row scales come from the lane that
//     gathered the key (ds_bpermute).
//   * O^T += V^T P^T for the wave's 16 latent tiles; V^T from the wave's bf16
//     rows in LDS through ds_read_b64_tr_b16.  Rows are 544 bytes (8 banks
//     apart) and rows 4-7 of every 8 swap the 16-byte halves of each
//     32-byte block, so both the 8 rows of each write pass and the 4 rows
//     of each transposing read pass land on distinct banks (the LDS serves
//     128 bytes per pass), while every address stays a per-lane base plus a
//     constant (no per-tile address registers).
//   * The partial S^T buffer is single: a second barrier before a wave
//     overwrites its half keeps it from racing the other wave's read.
//   * Gathers run one tile ahead and index loads three, and two waves share
//     each SIMD (two workgroups of a CU's four): while one wave waits for its
//     next tile's rows the other computes.  (Gathers two tiles ahead with one
//     wave per SIMD needed 280 registers and ran 14 % slower.)  No barrier
//     waits for the loads (a workgroup barrier here waits only for LDS
//     traffic).  Every
//     load is unconditional: a masked key reads row 0 (its score becomes
//     -1e30, its weight and scale 0, and int8 codes are finite); a branch
//     around the loads would make the compiler's wait before the next use
//     count no load as outstanding, draining the prefetch every tile.
//   * 38 KB of LDS per workgroup (four fit a CU's 160 KB) and at most 256
//     registers per wave (249 used, no scratch).
constexpr int kHalfLat = kLatent / 2;
constexpr int kPairVStride = kHalfLat + 16;   // bf16 per LDS V row: 544 bytes
constexpr int kPairRowBytes = kPairVStride * 2;

struct __attribute__((aligned(16))) PairShared {
  uint16_t vbuf[2][kTile][kPairVStride];      // per wave: bf16 V half-rows of the tile
  float4 red[2][2][64];                       // [wave][key half][lane]: partial S^T
};

// Byte offset of bf16 element (row, col) of a wave's V buffer: 16-byte chunk
// (col / 8) ^ (row / 4 % 2) of the row.
__device__ __forceinline__ int pair_vofs(int row, int col) {
  return row * kPairRowBytes + 16 * ((col >> 3) ^ ((row >> 2) & 1)) + 2 * (col & 7);
}

template <int kMode>
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(2, 2)))
void sparse_mla_pair_kernel(const MlaArgs a) {
  constexpr bool kPaged = kMode != kFlatRows;
  __shared__ PairShared sh;
  const int split = blockIdx.x, t = blockIdx.y, hg = blockIdx.z;
  const int w = uniform(threadIdx.x >> 6);   // latent half of this wave
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int start = split * a.split_len;
  const int end = min(start + a.split_len, a.topk);
  const int ntiles = end > start ? (end - start + kTile - 1) / kTile : 0;
  const int head = hg * kHeads + c;
  const bool head_ok = head < a.num_heads;
  const int32_t* idx_t = a.idx + t * a.si_t;
  // Paged modes: the request's block-table row.  Every table read below is
  // unconditional, from an address clamped into that row; a request id
  // outside the table (or a zero-width table) reads req_id[t] instead and
  // maps every key to -1.
  const int req = kPaged ? a.req_id[t] : 0;
  const bool req_ok = kPaged && req >= 0 && req < a.num_reqs && a.max_blocks > 0;
  const int32_t* bt_req = !kPaged ? nullptr : req_ok ? a.bt + static_cast<int64_t>(req) * a.bt_stride : a.req_id + t;
  const int max_blocks = req_ok ? a.max_blocks : 0;
  const int last_blk = max(max_blocks, 1) - 1;
  // Pooled mode: the token's pool ids (with none, req_id[t] stands in and is never used)
  const int32_t* pools_t = kMode != kPooledPos ? nullptr : a.num_pools > 0 ? a.pools + t * a.sp_t : a.req_id + t;
  const int last_pool = max(a.num_pools, 1) - 1;
  const int seq_len_t = kMode == kPooledPos && a.seq_lens ? a.seq_lens[t] : -1;
  uint8_t* vb = reinterpret_cast<uint8_t*>(&sh.vbuf[w][0][0]);
  // per-lane LDS bases (pair_vofs of the lane's first element)
  const int wr_lo = pair_vofs(c, 16 * g);        // row c, columns 16 g + [0, 8)
  const int wr_hi = pair_vofs(c, 16 * g + 8);    //        columns 16 g + 8 + [0, 8)
  const int tr_base = pair_vofs(4 * g + (c >> 2), 4 * (c & 3));

  // Q^T fragments (B operand): head c, K-step (i, j) = latents
  // 256 w + 64 i + 16 g + 8 j + [0, 8) -- the latents of the lane's gathered
  // chunk 4 i + g of each key.
  bf16x8 qf[4][2];
  {
    const uint4* qp = reinterpret_cast<const uint4*>(a.q + t * a.sq_t + head * a.sq_h + kHalfLat * w);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
        qf[i][j] = __builtin_bit_cast(bf16x8, head_ok ? qp[8 * i + 2 * g + j] : make_uint4(0, 0, 0, 0));
  }

  f32x4 acc[16];
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegLarge, l_run = 0.f;
  bool acc_zero = true;

  // Key l of tile n is handled by lane l < 32 in three steps, each one tile
  // ahead of the next so that no step waits for a load younger than the
  // gathers in flight (loads complete in order):
  //   load_raw (tile n - 3): its index (pooled mode: its pool id), read
  //     from an address clamped into the split, with no branch;
  //   lookup   (tile n - 2): the position's block-table entry (paged modes;
  //     flat rows need no load), again from a clamped address;
  //   issue_rows (tile n - 1): the scale and the row gathers.
  // Positions past the split and invalid keys are masked in lookup and
  // issue_rows; masked keys read row 0 (unit 0 of the paged cache), which
  // exists because the launch requires a non-empty cache.  (Masking right
  // after a load would make the wave wait for it, and with it for every
  // gather issued before it.)
  auto tile_pos = [&](int n) { return start + n * kTile + (lane & 31); };
  auto load_raw = [&](int n) {
    const int k = min(tile_pos(n), end - 1);
    if constexpr (kMode == kPooledPos) return pools_t[min(k / a.pool_size, last_pool)];
    else return idx_t[k];
  };
  struct Look {
    int e;     // flat: the row or -1; paged: the block-table entry (checked in issue_rows)
    int rel;   // paged: the row within its page, or -1 for a masked key
  };
  auto lookup = [&](int raw, int n) {
    const int pos = tile_pos(n);
    Look l;
    if constexpr (kMode == kFlatRows) {
      l.e = pos < end && raw >= 0 && static_cast<int64_t>(raw) < a.seq_kv ? raw : -1;
      l.rel = 0;
    } else {
      int p = raw;   // request-relative position (pooled_position for the pooled layout)
      if constexpr (kMode == kPooledPos) {
        const int expanded = a.num_pools * a.pool_size;
        const int j = pos - expanded;
        const int pq = pos / a.pool_size;
        p = pos < expanded ? (raw >= 0 ? raw * a.pool_size + (pos - pq * a.pool_size) : -1)
            : seq_len_t >= 0 && j < a.pool_size - 1 && j < seq_len_t % a.pool_size
                ? seq_len_t / a.pool_size * a.pool_size + j
                : -1;
      }
      const int blk = static_cast<int>(static_cast<uint32_t>(max(p, 0)) / static_cast<uint32_t>(a.block_size));
      l.e = bt_req[min(blk, last_blk)];
      l.rel = pos < end && p >= 0 && blk < max_blocks ? p - blk * a.block_size : -1;
    }
    return l;
  };
  struct Rows {
    uint4 d[2][4];      // [key half][chunk i]: latents 256 w + 64 i + 16 g + [0, 16) of key 16 u + c
    float sv;           // lane l < 32: scale of key l (garbage for a masked key)
    uint32_t vmask;     // bit l: key l valid
  };
  // flat: row index, rows skv bytes apart; paged: 16-byte unit of the row
  const int64_t unit_bytes = kPaged ? 16 : a.skv;
  auto issue_rows = [&](Rows& r, const Look& l) {
    int v = l.e;
    if constexpr (kPaged)
      v = l.rel >= 0 && l.e >= 0 && l.e < a.num_blocks ? l.e * a.page_units + l.rel * a.row_units : -1;
    // the scale first: older than the rows, its wait comes free with theirs
    r.sv = *reinterpret_cast<const float*>(a.kv + static_cast<int64_t>(max(v, 0)) * unit_bytes + kLatent);
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int kid = max(__shfl(v, 16 * u + c, 64), 0);
      const uint4* rp = reinterpret_cast<const uint4*>(a.kv + static_cast<int64_t>(kid) * unit_bytes + kHalfLat * w);
#pragma unroll
      for (int i = 0; i < 4; i++) r.d[u][i] = rp[4 * i + g];
    }
    r.vmask = static_cast<uint32_t>(__ballot(lane < kTile && v >= 0));
  };

  // One tile: convert + S^T + V to LDS, then the index of tile n + 3, the
  // lookup of tile n + 2 and the gathers of tile n + 1 (into the registers
  // this tile's rows just left), then the exchange, softmax and PV.  On
  // entry raw_s holds tile n + 2's index (the slot of n's parity) and look_o
  // tile n + 1's lookup.
  auto tile = [&](int n, Rows& cur, int& raw_s, int& raw_o, Look& look_s, Look& look_o) {
    f32x4 s_part[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
      f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        bf16x8 lo, hi;
        i8x16_to_bf16(cur.d[u][i], lo, hi);
        sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, qf[i][0], sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, qf[i][1], sacc, 0, 0, 0);
        // row 16 u + c, columns 64 i + 16 g + [0, 16): pair_vofs as base + constant
        *reinterpret_cast<uint4*>(vb + wr_lo + u * 16 * kPairRowBytes + 128 * i) = __builtin_bit_cast(uint4, lo);
        *reinterpret_cast<uint4*>(vb + wr_hi + u * 16 * kPairRowBytes + 128 * i) = __builtin_bit_cast(uint4, hi);
        __builtin_amdgcn_sched_barrier(0);
      }
      s_part[u] = sacc;
    }
    __syncthreads();   // the other wave has read this wave's previous partial
    sh.red[w][0][lane] = make_float4(s_part[0][0], s_part[0][1], s_part[0][2], s_part[0][3]);
    sh.red[w][1][lane] = make_float4(s_part[1][0], s_part[1][1], s_part[1][2], s_part[1][3]);
    // scales of the lane's keys 16 u + 4 g + r (0 for a masked key), and the validity bits
    float sc[8];
    const uint32_t kv_ok = ((cur.vmask >> (4 * g)) & 0xfu) | (((cur.vmask >> (16 + 4 * g)) & 0xfu) << 4);
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float v = __shfl(cur.sv, 16 * u + 4 * g + r, 64);
        sc[4 * u + r] = (kv_ok >> (4 * u + r)) & 1 ? v : 0.f;
      }
    // the registers of this tile are free: gathers of tile n + 1, index of tile n + 3
    // (kept below the conversions: hoisted above them the loads would hold a
    // second tile's registers while the converted operands are still live)
    __builtin_amdgcn_sched_barrier(0);
    raw_o = load_raw(n + 3);
    look_s = lookup(raw_s, n + 2);
    issue_rows(cur, look_o);
    __syncthreads();

    // Full scores: wave 0's partial + wave 1's, the same order in both waves.
    float s[8];
    {
      const float4 p00 = sh.red[0][0][lane], p01 = sh.red[0][1][lane];
      const float4 p10 = sh.red[1][0][lane], p11 = sh.red[1][1][lane];
      const float4 h0[2] = {p00, p01}, h1[2] = {p10, p11};
#pragma unroll
      for (int jj = 0; jj < 8; jj++) {
        float v = f4_get(h0[jj >> 2], jj & 3) + f4_get(h1[jj >> 2], jj & 3);
        v *= sc[jj];
        v *= a.scale_log2;
        s[jj] = (kv_ok >> jj) & 1 ? v : kNegLarge;
      }
    }
    float mx = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
    mx = rows_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - m_new);
    float pr[8];
#pragma unroll
    for (int jj = 0; jj < 8; jj++) pr[jj] = (kv_ok >> jj) & 1 ? fast_exp2(s[jj] - m_new) : 0.f;
    float psum = ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
    psum = rows_sum(psum);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // P^T operand: k-slot 8 g + jj <-> key 16 (jj / 4) + 4 g + jj % 4.
    const uint4 pw = make_uint4(pack_bf16x2(pr[0] * sc[0], pr[1] * sc[1]), pack_bf16x2(pr[2] * sc[2], pr[3] * sc[3]),
                                pack_bf16x2(pr[4] * sc[4], pr[5] * sc[5]), pack_bf16x2(pr[6] * sc[6], pr[7] * sc[7]));
    const bf16x8 pb = __builtin_bit_cast(bf16x8, pw);
    if (!acc_zero && __ballot(alpha != 1.f)) {
#pragma unroll
      for (int dt = 0; dt < 16; dt++) {
        acc[dt][0] *= alpha; acc[dt][1] *= alpha; acc[dt][2] *= alpha; acc[dt][3] *= alpha;
      }
    }
    // ds_read_b64_tr_b16: in each 16-lane group, lane 4 r + q addresses row r,
    // columns [4 q, 4 q + 4); lane c receives column c of the 4 rows.
#pragma unroll
    for (int dt = 0; dt < 16; dt++) {
      // groups of 4 tiles: the reads of a group are not hoisted above the
      // previous group's products (registers)
      if (dt % 4 == 0 && dt > 0) __builtin_amdgcn_sched_barrier(0);
      // rows 4 g + c / 4 and 16 + 4 g + c / 4, columns 16 dt + 4 (c % 4) + [0, 4)
      const i16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(GLM53_LDS(i16x4, vb + tr_base + 32 * dt));
      const i16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          GLM53_LDS(i16x4, vb + tr_base + 16 * kPairRowBytes + 32 * dt));
      const i32x2 v0i = __builtin_bit_cast(i32x2, v0);
      const i32x2 v1i = __builtin_bit_cast(i32x2, v1);
      const uint4 vv = make_uint4(v0i[0], v0i[1], v1i[0], v1i[1]);
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vv), pb, acc[dt], 0, 0, 0);
    }
    acc_zero = false;
  };

  // Tiles go in pairs (an odd count ends with a fully masked tile, which
  // changes nothing): no branch in the loop body.
  Rows ra;                               // the one tile of rows in flight
  int r0 = -1, r1 = -1;                  // raw slots (even, odd tiles)
  Look l0 = {-1, -1}, l1 = {-1, -1};     // lookup slots
  if (ntiles > 0) {
    const int i0 = load_raw(0), i1 = load_raw(1);
    r0 = load_raw(2);
    const Look k0 = lookup(i0, 0);
    l1 = lookup(i1, 1);
    issue_rows(ra, k0);
  }
  for (int n = 0; n < ntiles; n += 2) {
    tile(n, ra, r0, r1, l0, l1);
    tile(n + 1, ra, r1, r0, l1, l0);
  }

  // Both waves hold the same m and l; each writes its latent half.
  const float inv_l = 1.f / (l_run > 0.f ? l_run : 1.f);
  if (!head_ok) return;
  if (a.num_splits == 1 && !a.partials_only) {
    uint16_t* op = a.out + t * a.so_t + head * a.so_h + kHalfLat * w + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 16; dt++)
      *reinterpret_cast<uint2*>(op + 16 * dt) = make_uint2(pack_bf16x2(acc[dt][0] * inv_l, acc[dt][1] * inv_l),
                                                           pack_bf16x2(acc[dt][2] * inv_l, acc[dt][3] * inv_l));
  } else {
    // accumulator order: latents 256 w + 16 dt + 4 g are slice 2 w + dt / 8, tile dt % 8
    float* pb = part_block(a, t, split, hg) + (16 * w * 64 + lane) * 4;
#pragma unroll
    for (int dt = 0; dt < 16; dt++)
      *reinterpret_cast<float4*>(pb + dt * 64 * 4) = make_float4(acc[dt][0] * inv_l, acc[dt][1] * inv_l,
                                                                 acc[dt][2] * inv_l, acc[dt][3] * inv_l);
    if (w == 0 && g == 0)
      a.lse[(static_cast<int64_t>(t) * a.num_splits + split) * a.heads_padded + head] = (m_run + log2f(l_run)) * kLn2;
  }
}

// ---------------------------------------------------------------- gather floor (diagnostic)
// The memory chain of sparse_mla_kernel's decode splits alone: the same grid
// and workgroup shape, the same index loads, row gathers and scale loads per
// lane, and the same partial-row and LSE stores, with no arithmetic between
// them (the loaded bytes are folded with XOR so that no load is dead).  Its
// duration is the floor that the split kernel's conversions, products and
// softmax add to.
template <int kG>
__global__ __launch_bounds__(SplitShape<kG>::kThreads) void sparse_mla_gather_floor_kernel(
    const int32_t* idx, int64_t si_t, int split_len, int topk, int grid_x, int grid_y, int grid_z, int num_heads,
    const uint16_t* q, int64_t sq_t, int64_t sq_h, const MlaArgs a) {
  constexpr int kRounds = SplitShape<kG>::kRounds;
  int split = blockIdx.x, t = blockIdx.y, hg = blockIdx.z;
  if ((grid_y * grid_z) % 4 == 0) {
    const int lin = blockIdx.x + grid_x * (blockIdx.y + grid_y * blockIdx.z);
    const int units = grid_y * grid_z;
    split = lin / units;
    t = (lin % units) % grid_y;
    hg = (lin % units) / grid_y;
  }
  const int w = uniform(threadIdx.x >> 6);
  const int sl = w & (kSlices - 1);
  const int kg = w / kSlices;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int start = split * split_len;
  const int end = min(start + split_len, topk);
  const int32_t* idx_t = idx + t * si_t;
  const int head = hg * kHeads + c;
  // The split kernel's load order: the split's indices, q, then per tile the
  // row scale and the rows, all in flight before any is used (decode splits
  // are one chunk: split_len <= kChunkTiles * kTile, checked by the host).
  int ids[kRounds];
#pragma unroll
  for (int r = 0; r < kRounds; r++) {
    const int pos = start + (kG * r + kg) * kTile + (lane & 31);
    ids[r] = pos < end ? idx_t[pos] : -1;
  }
  const uint4* qp = reinterpret_cast<const uint4*>(q + t * sq_t + (head < num_heads ? head : 0) * sq_h +
                                                   kSlice * sl + 16 * g);
  const uint4 q0 = qp[0], q1 = qp[1], q2 = qp[8], q3 = qp[9];
  uint32_t sv[kRounds];
  uint4 kd[kRounds][2][2];
#pragma unroll
  for (int r = 0; r < kRounds; r++) {
    int v = ids[r];
    if (v < 0 || static_cast<int64_t>(v) >= a.seq_kv) v = -1;
    sv[r] = 0;
    if (sl == 0 && lane < kTile && v >= 0)
      sv[r] = *reinterpret_cast<const uint32_t*>(a.kv + static_cast<int64_t>(v) * a.skv + kLatent);
    // Row loads unconditional (a masked key reads row 0, then counts 0; the
    // host requires a non-empty cache): a branch around them made the
    // compiler copy the first load's result before issuing the second.
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int kid = __shfl(v, 16 * u + c, 64);
      const uint4* rp = reinterpret_cast<const uint4*>(a.kv + static_cast<int64_t>(max(kid, 0)) * a.skv +
                                                       kSlice * sl + 16 * g);
      const uint4 z = make_uint4(0, 0, 0, 0);
      const uint4 k0 = rp[0], k1 = rp[4];
      kd[r][u][0] = kid >= 0 ? k0 : z;
      kd[r][u][1] = kid >= 0 ? k1 : z;
    }
  }
  uint32_t fold = head < num_heads ? q0.x ^ q1.y ^ q2.z ^ q3.w : 0u;   // folded last: no early wait
#pragma unroll
  for (int r = 0; r < kRounds; r++) {
    fold ^= sv[r];
#pragma unroll
    for (int u = 0; u < 2; u++)
      fold ^= kd[r][u][0].x ^ kd[r][u][0].y ^ kd[r][u][0].z ^ kd[r][u][0].w ^
              kd[r][u][1].x ^ kd[r][u][1].y ^ kd[r][u][1].z ^ kd[r][u][1].w;
  }
  // a finite float from the folded bits, stored where and as the split
  // kernel stores: each wave its key group's accumulator tiles (tile dt of
  // group dt * kG / 8), 1 KB per instruction in the accumulator order
  const float x = static_cast<float>(fold & 0xffff);
  float* pb = part_block(a, t, split, hg) + (8 * sl * 64 + lane) * 4;
#pragma unroll
  for (int dt = 0; dt < 8; dt++)
    if (dt * kG / 8 == kg) *reinterpret_cast<float4*>(pb + dt * 64 * 4) = make_float4(x, x, x, x);
  if (head < num_heads && kg == 0 && sl == 0 && g == 0)
    a.lse[(static_cast<int64_t>(t) * a.num_splits + split) * a.heads_padded + head] = x;
}

// Standalone conversion (the vLLM helper the reference's adapter calls):
// out[t][k] = to_flat_row(block_table[req_id[t]], ..., indices[t][k]).
__global__ __launch_bounds__(256) void convert_req_index_kernel(const int32_t* __restrict__ req_id,
                                                                const int32_t* __restrict__ bt,
                                                                int64_t bt_stride, int max_blocks,
                                                                int num_reqs,
                                                                const int32_t* __restrict__ idx,
                                                                int64_t si_t, int32_t* __restrict__ out,
                                                                int64_t so_t, int topk, int block_size,
                                                                int page_rows) {
  const int t = blockIdx.y;
  const int k = blockIdx.x * 256 + threadIdx.x;
  if (k >= topk) return;
  const int req = req_id[t];
  const bool req_ok = req >= 0 && req < num_reqs;   // other ids: every index maps to -1
  const int32_t* bt_req = req_ok ? bt + static_cast<int64_t>(req) * bt_stride : bt;
  out[t * so_t + k] = to_flat_row(bt_req, req_ok ? max_blocks : 0, block_size, page_rows,
                                  idx[t * si_t + k]);
}

// Standalone pool expansion: out[t][k] = pooled_position(pools[t], ...) for
// k < out_cols.  pools are int32 or int64; an id outside [0, 2^31) is
// treated as invalid (-1).
template <typename PoolT>
__global__ __launch_bounds__(256) void expand_pools_kernel(const PoolT* __restrict__ pools, int64_t sp_t,
                                                           int num_pools, int pool_size,
                                                           const int32_t* __restrict__ seq_lens,
                                                           int32_t* __restrict__ out, int64_t so_t,
                                                           int out_cols) {
  const int t = blockIdx.y;
  const int k = blockIdx.x * 256 + threadIdx.x;
  if (k >= out_cols) return;
  const PoolT* src = pools + t * sp_t;
  const int seq_len = seq_lens ? seq_lens[t] : -1;
  auto pool = [&](int j) {
    const int64_t v = static_cast<int64_t>(src[j]);
    return v >= 0 && v <= 0x7fffffff ? static_cast<int>(v) : -1;
  };
  out[t * so_t + k] = pooled_position(pool, num_pools, pool_size, seq_len, k);
}

// N-way LSE merge (kernels/titan_mla.py:403-429).  One workgroup per
// (token, head group, 16-latent tile of the accumulator order: slice sl,
// tile dt); 512 threads = 8 split lanes x 64 positions, position p = 16 g +
// c holding head c, latents 128 sl + 16 dt + 4 g + [0, 4) -- each split's
// 1 KB block of the tile is one contiguous load per split lane.  Split lane
// k handles splits k, k + 8, ...: it loads their partials and LSEs together
// (one memory round trip), the block takes the maximum M of the head's
// LSEs, and each lane accumulates sum e^{lse_s - M} part_s and
// sum e^{lse_s - M} over its splits in order; the 8 lanes are then summed in
// a fixed order.  out = acc / den: the reference's running rescaled sum
// written without a serial dependency, deterministic.  Empty splits carry
// lse = -inf and weigh 0; no valid split gives 0.
constexpr int kMergeRegs = 16;   // splits per lane held in registers (S <= 128)
constexpr int kMergeThreads = kMergeLanes * 64;

template <bool kPad>
__global__ __launch_bounds__(kMergeThreads) void sparse_mla_merge_kernel(const float* __restrict__ part,
                                                                          const float* __restrict__ lse,
                                                                          int num_splits, int heads_padded,
                                                                          int num_heads, int num_tokens,
                                                                          uint16_t* __restrict__ out,
                                                                          int64_t so_t, int64_t so_h) {
  __shared__ float red_m[kMergeLanes][64];
  __shared__ float part_den[kMergeLanes][64];
  __shared__ __attribute__((aligned(16))) float4 part_sum[kMergeLanes][64];
  // token fastest in the linear id: with a multiple of 8 (4) tokens, token
  // t's workgroups share the XCD (the two XCDs) that ran its splits
  // (num_tokens * groups is gridDim.x, passed in with the leading arguments
  // so that it arrives preloaded).  kPad: num_tokens holds the numbered
  // tokens (low 16 bits) and the batch's (high 16), as the split kernel's
  // grid_y does.
  const int nt = kPad ? (num_tokens & 0xffff) : num_tokens;
  const int groups = heads_padded / kHeads;
  int t = blockIdx.x / groups, hg = blockIdx.x % groups, tile = blockIdx.y;
  if (nt % 4 == 0) {
    const int lin = blockIdx.x + nt * groups * blockIdx.y;
    t = lin % nt;
    hg = (lin / nt) % groups;
    tile = lin / (nt * groups);
  }
  if (kPad && t >= static_cast<int>(static_cast<unsigned>(num_tokens) >> 16)) return;   // uniform
  const int tid = threadIdx.x;
  const int sp = tid >> 6;          // split lane (one wave each)
  const int p = tid & 63;           // position 16 g + c
  const int head = hg * kHeads + (p & 15);
  // split s: block (t * S + s) * groups + hg, float4 tile * 64 + p in it
  const int64_t blk0 = static_cast<int64_t>(t) * num_splits * groups + hg;
  const int64_t blk_stride = static_cast<int64_t>(groups) * kHeads * kLatent;
  const float* pp = part + blk0 * kHeads * kLatent + (tile * 64 + p) * 4;
  const float* lp = lse + static_cast<int64_t>(t) * num_splits * heads_padded + head;
  const bool in_regs = num_splits <= kMergeLanes * kMergeRegs;

  float4 pv[kMergeRegs];
  float lv[kMergeRegs];
  float m = kNegLarge;
  if (in_regs) {
#pragma unroll
    for (int j = 0; j < kMergeRegs; j++) {
      const int s = sp + kMergeLanes * j;
      f32x4 x = f32x4{0.f, 0.f, 0.f, 0.f};   // read once: streaming loads
      if (s < num_splits) x = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(pp + s * blk_stride));
      pv[j] = make_float4(x[0], x[1], x[2], x[3]);
      lv[j] = s < num_splits ? lp[static_cast<int64_t>(s) * heads_padded] : kNegLarge;
    }
#pragma unroll
    for (int j = 0; j < kMergeRegs; j++) m = fmaxf(m, lv[j]);
  } else {
    for (int s = sp; s < num_splits; s += kMergeLanes) m = fmaxf(m, lp[static_cast<int64_t>(s) * heads_padded]);
  }
  red_m[sp][p] = m;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kMergeLanes; k++) m = fmaxf(m, red_m[k][p]);

  float den = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (in_regs) {
#pragma unroll
    for (int j = 0; j < kMergeRegs; j++) {
      if (sp + kMergeLanes * j < num_splits) {
        const float e = expf(lv[j] - m);
        acc.x += e * pv[j].x;
        acc.y += e * pv[j].y;
        acc.z += e * pv[j].z;
        acc.w += e * pv[j].w;
        den += e;
      }
    }
  } else {
    for (int s = sp; s < num_splits; s += kMergeLanes) {
      const float e = expf(lp[static_cast<int64_t>(s) * heads_padded] - m);
      const float4 v = *reinterpret_cast<const float4*>(pp + s * blk_stride);
      acc.x += e * v.x;
      acc.y += e * v.y;
      acc.z += e * v.z;
      acc.w += e * v.w;
      den += e;
    }
  }
  part_sum[sp][p] = acc;
  part_den[sp][p] = den;
  __syncthreads();
  if (sp == 0 && head < num_heads) {
    float4 r = part_sum[0][p];
    float dsum = part_den[0][p];
#pragma unroll
    for (int k = 1; k < kMergeLanes; k++) {
      const float4 v = part_sum[k][p];
      r.x += v.x; r.y += v.y; r.z += v.z; r.w += v.w;
      dsum += part_den[k][p];
    }
    const float inv = 1.f / (dsum > 0.f ? dsum : 1.f);
    uint2 o;
    o.x = pack_bf16x2(r.x * inv, r.y * inv);
    o.y = pack_bf16x2(r.z * inv, r.w * inv);
    const int d = kSlice * (tile >> 3) + 16 * (tile & 7) + 4 * (p >> 4);
    *reinterpret_cast<uint2*>(out + t * so_t + head * so_h + d) = o;
  }
}

}  // namespace
}  // namespace glm53

using namespace glm53;

namespace glm53 {
namespace {

int64_t partial_rows(int64_t num_tokens, int64_t num_heads, int64_t num_splits) {
  return num_tokens * num_splits * ((num_heads + kHeads - 1) / kHeads * kHeads);
}

// Validates the attention arguments and fills MlaArgs (all but the outputs).
int prepare(MlaArgs& a, const void* q, int64_t sq_t, int64_t sq_h, const void* kv, int64_t skv_t,
            int64_t seq_kv, const int32_t* indices, int64_t si_t, int64_t num_tokens,
            int64_t num_heads, int64_t topk, double sm_scale, int64_t num_splits) {
  if (num_tokens < 0 || num_heads < 1 || topk < 0 || num_splits < 1 || seq_kv < 0)
    return GLM53_ERR_BAD_SHAPE;
  if (num_tokens > 0 && (!q || (!kv && seq_kv > 0) || (!indices && topk > 0)))
    return GLM53_ERR_NULL_POINTER;
  // tokens are the grid's y dimension and head groups its z dimension
  if (topk > 0x7fffffff || num_tokens > kMaxGridTokens || num_splits > kMaxMergeSplits ||
      (num_heads + kHeads - 1) / kHeads > 65535)
    return GLM53_ERR_BAD_SHAPE;
  if (reinterpret_cast<uintptr_t>(q) % 16 || sq_t % 8 || sq_h % 8 ||
      reinterpret_cast<uintptr_t>(kv) % 16 || skv_t % 16)
    return GLM53_ERR_MISALIGNED;
  a.q = static_cast<const uint16_t*>(q);
  a.sq_t = sq_t;
  a.sq_h = sq_h;
  a.kv = static_cast<const uint8_t*>(kv);
  a.skv = skv_t;
  a.seq_kv = seq_kv;
  a.idx = indices;
  a.si_t = si_t;
  a.num_heads = static_cast<int>(num_heads);
  a.topk = static_cast<int>(topk);
  a.num_splits = static_cast<int>(num_splits);
  a.split_len = static_cast<int>((topk + num_splits - 1) / num_splits);
  a.scale_log2 = static_cast<float>(sm_scale * 1.4426950408889634);
  a.heads_padded = static_cast<int>((num_heads + kHeads - 1) / kHeads * kHeads);
  a.part = nullptr;
  a.lse = nullptr;
  a.out = nullptr;
  a.partials_only = 0;
  a.out_align16 = 0;
  a.req_id = nullptr;
  a.bt = nullptr;
  a.bt_stride = 0;
  a.max_blocks = 0;
  a.num_reqs = 0;
  a.block_size = 1;
  a.num_blocks = 0;
  a.page_units = 0;
  a.row_units = 0;
  a.pools = nullptr;
  a.sp_t = 0;
  a.num_pools = 0;
  a.pool_size = 1;
  a.seq_lens = nullptr;
  a.so_t = a.so_h = 0;
  return 0;
}

// Tokens the split and merge kernels number: 3, 5, 6 or 7 tokens (one head
// group) as 4 or 8, so that a token's splits share one XCD (two at 4) --
// when they fit its CUs -- and the merge reads them back there, the extra
// tokens' workgroups returning at once.  Interleaved A/B over rotating
// HBM-resident caches, 23 splits: B=5 11.92 -> 11.11 us, B=6 12.05 -> 11.29,
// B=7 12.25 -> 11.31; B=3 (34 splits) 10.48 -> 10.37; bit-identical.
int64_t tokens_grid(int64_t num_tokens, int heads_padded, int64_t num_splits) {
  if (heads_padded != kHeads || num_tokens < 3 || num_tokens > 7 || num_tokens == 4) return num_tokens;
  const int64_t tp = num_tokens == 3 ? 4 : 8;
  return num_splits <= 32 * (8 / tp) ? tp : num_tokens;   // each XCD's share within its 32 CUs
}

void launch_attention(const MlaArgs& a, int64_t num_tokens, hipStream_t st) {
  // Splits longer than one chunk of gathers pipeline their chunks.
  const bool pipe = a.split_len > kChunkTiles * kTile;
  // Long splits go to the pair kernel, whose masked keys read row 0 (page 0):
  // it needs a non-empty cache (seq_kv counts rows, or pages when paged).
  const bool pair = pipe && a.seq_kv > 0;
  // Splits of exactly three tiles (65 to 96 keys) run in one round on three
  // key groups, splits of one tile on one key group.
  const bool three = a.split_len > 2 * kTile && a.split_len <= 3 * kTile;
  const bool one = a.split_len <= kTile;
  const int64_t tg = pipe || one ? num_tokens : tokens_grid(num_tokens, a.heads_padded, a.num_splits);
  const bool pad = tg != num_tokens;
  const dim3 grid(static_cast<unsigned>(a.num_splits), static_cast<unsigned>(tg),
                  static_cast<unsigned>(a.heads_padded / kHeads));
  const int gy_arg = pad ? static_cast<int>(tg | (num_tokens << 16)) : static_cast<int>(tg);
  const int mode = a.pools != nullptr ? kPooledPos : a.bt != nullptr ? kPagedPos : kFlatRows;
#define GLM53_LEAD a.idx, a.si_t, a.split_len, a.topk, static_cast<int>(grid.x), gy_arg, \
                   static_cast<int>(grid.z), a.num_heads, a.q, a.sq_t, a.sq_h, a
#define GLM53_LAUNCH(M, P)                                                                        \
  do {                                                                                            \
    if (pad && !P)                                                                                \
      hipLaunchKernelGGL((sparse_mla_kernel<M, P, 2, true>), grid, dim3(kThreads), 0, st, GLM53_LEAD); \
    else                                                                                          \
      hipLaunchKernelGGL((sparse_mla_kernel<M, P, 2>), grid, dim3(kThreads), 0, st, GLM53_LEAD);       \
  } while (0)
#define GLM53_PAIR(M) hipLaunchKernelGGL((sparse_mla_pair_kernel<M>), grid, dim3(128), 0, st, a)
#define GLM53_KG(M, G)                                                                                 \
  do {                                                                                                 \
    if (pad && G == 3)                                                                                 \
      hipLaunchKernelGGL((sparse_mla_kernel<M, false, 3, true>), grid, dim3(SplitShape<3>::kThreads), 0, st, \
                         GLM53_LEAD);                                                                  \
    else                                                                                               \
      hipLaunchKernelGGL((sparse_mla_kernel<M, false, G>), grid, dim3(SplitShape<G>::kThreads), 0, st,       \
                         GLM53_LEAD);                                                                  \
  } while (0)
  if (mode == kPooledPos) {
    if (pair) GLM53_PAIR(kPooledPos); else if (pipe) GLM53_LAUNCH(kPooledPos, true);
    else if (three) GLM53_KG(kPooledPos, 3); else if (one) GLM53_KG(kPooledPos, 1); else GLM53_LAUNCH(kPooledPos, false);
  } else if (mode == kPagedPos) {
    if (pair) GLM53_PAIR(kPagedPos); else if (pipe) GLM53_LAUNCH(kPagedPos, true);
    else if (three) GLM53_KG(kPagedPos, 3); else if (one) GLM53_KG(kPagedPos, 1); else GLM53_LAUNCH(kPagedPos, false);
  } else {
    if (pair) GLM53_PAIR(kFlatRows); else if (pipe) GLM53_LAUNCH(kFlatRows, true);
    else if (three) GLM53_KG(kFlatRows, 3); else if (one) GLM53_KG(kFlatRows, 1); else GLM53_LAUNCH(kFlatRows, false);
  }
#undef GLM53_KG
#undef GLM53_PAIR
#undef GLM53_LAUNCH
#undef GLM53_LEAD
}

void launch_merge(const float* part, const float* lse, int64_t num_tokens, int num_splits,
                  int heads_padded, int num_heads, uint16_t* out, int64_t so_t, int64_t so_h,
                  hipStream_t st) {
  const int64_t tg = tokens_grid(num_tokens, heads_padded, num_splits);
  const dim3 grid(static_cast<unsigned>(tg * (heads_padded / kHeads)), 32);
  if (tg != num_tokens)
    hipLaunchKernelGGL(sparse_mla_merge_kernel<true>, grid, dim3(kMergeThreads), 0, st, part, lse, num_splits,
                       heads_padded, num_heads, static_cast<int>(tg | (num_tokens << 16)), out, so_t, so_h);
  else
    hipLaunchKernelGGL(sparse_mla_merge_kernel<false>, grid, dim3(kMergeThreads), 0, st, part, lse, num_splits,
                       heads_padded, num_heads, static_cast<int>(num_tokens), out, so_t, so_h);
}

}  // namespace
}  // namespace glm53

extern "C" int64_t glm53_sparse_mla_workspace_bytes(int64_t num_tokens, int64_t num_heads,
                                                    int64_t num_splits) {
  if (num_tokens < 0 || num_heads < 1 || num_splits < 1) return -1;
  if (num_splits == 1) return 0;
  return glm53_sparse_mla_partials_bytes(num_tokens, num_heads, num_splits);
}

extern "C" int64_t glm53_sparse_mla_partials_bytes(int64_t num_tokens, int64_t num_heads,
                                                   int64_t num_splits) {
  if (num_tokens < 0 || num_heads < 1 || num_splits < 1) return -1;
  const int64_t rows = partial_rows(num_tokens, num_heads, num_splits);
  return rows * kLatent * 4 + rows * 4;
}

namespace glm53 {
namespace {

// Output checks, workspace split, the attention launch and (num_splits > 1)
// the merge launch: the common tail of glm53_sparse_mla and
// glm53_sparse_mla_paged.
int run_attention(MlaArgs& a, int64_t num_tokens, int64_t num_heads, int64_t num_splits,
                  void* workspace, int64_t workspace_bytes, void* out, int64_t so_t, int64_t so_h,
                  void* stream) {
  if (!out) return GLM53_ERR_NULL_POINTER;
  if (reinterpret_cast<uintptr_t>(out) % 8 || so_t % 4 || so_h % 4) return GLM53_ERR_MISALIGNED;
  const int64_t need = glm53_sparse_mla_workspace_bytes(num_tokens, num_heads, num_splits);
  if (num_splits > 1 && (!workspace || workspace_bytes < need)) return GLM53_ERR_WORKSPACE;
  const int64_t rows = partial_rows(num_tokens, num_heads, num_splits);
  a.part = num_splits > 1 ? static_cast<float*>(workspace) : nullptr;
  a.lse = num_splits > 1 ? static_cast<float*>(workspace) + rows * kLatent : nullptr;
  a.out = static_cast<uint16_t*>(out);
  a.so_t = so_t;
  a.so_h = so_h;
  a.out_align16 = reinterpret_cast<uintptr_t>(out) % 16 == 0 && so_t % 8 == 0 && so_h % 8 == 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  launch_attention(a, num_tokens, st);
  if (num_splits > 1)
    launch_merge(a.part, a.lse, num_tokens, a.num_splits, a.heads_padded, a.num_heads, a.out, so_t,
                 so_h, st);
  return static_cast<int>(hipGetLastError());
}

// Checks of the paged-index arguments shared by the two paged entry points.
int check_paged(const int32_t* req_id, const int32_t* block_table, int64_t num_reqs,
                int64_t bt_stride, int64_t max_blocks, int64_t block_size, int64_t page_rows) {
  if (!req_id || (!block_table && max_blocks > 0 && num_reqs > 0)) return GLM53_ERR_NULL_POINTER;
  if (block_size < 1 || page_rows < block_size || max_blocks < 0 || bt_stride < 0 ||
      num_reqs < 0 || block_size > 0x7fffffff || page_rows > 0x7fffffff ||
      max_blocks > 0x7fffffff || num_reqs > 0x7fffffff)
    return GLM53_ERR_BAD_SHAPE;
  return 0;
}

}  // namespace
}  // namespace glm53

namespace glm53 {
namespace {

// Static device scratch of glm53_sparse_mla_noalloc: the split partials of
// at most GLM53_NOALLOC_MAX_PARTIAL_ROWS (token, split, head) rows, laid out
// as the workspace of glm53_sparse_mla (rows x 512 floats of partials in
// their accumulator-order blocks, then lse [rows]).
// Every GPU the library runs on holds its own copy until the process ends.
static __device__ __align__(256) float scratch[GLM53_NOALLOC_MAX_PARTIAL_ROWS * (kLatent + 1)];

constexpr int kMaxDevices = 64;
std::atomic<void*> scratch_ptr[kMaxDevices];   // device address of `scratch`, per device

// The device address of the current device's `scratch`, looked up once per
// device (the array's host-side name is not a device address).
int device_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return GLM53_ERR_BAD_SHAPE;
  void* p = scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (!p) return static_cast<int>(hipErrorInvalidSymbol);
    scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return 0;
}

}  // namespace
}  // namespace glm53

extern "C" int glm53_sparse_mla_noalloc(const void* q, int64_t sq_t, int64_t sq_h, const void* kv,
                                        int64_t skv_t, int64_t seq_kv, const int32_t* indices,
                                        int64_t si_t, int64_t num_tokens, int64_t num_heads,
                                        int64_t topk, double sm_scale, int64_t num_splits, void* out,
                                        int64_t so_t, int64_t so_h, void* stream) {
  MlaArgs a;
  int rc = prepare(a, q, sq_t, sq_h, kv, skv_t, seq_kv, indices, si_t, num_tokens, num_heads, topk,
                   sm_scale, num_splits);
  if (rc) return rc;
  if (num_tokens == 0) return 0;
  if (num_splits > 1 && partial_rows(num_tokens, num_heads, num_splits) > GLM53_NOALLOC_MAX_PARTIAL_ROWS)
    return GLM53_ERR_SCRATCH_LIMIT;
  void* ws = nullptr;
  if (num_splits > 1) {
    rc = device_scratch(&ws);
    if (rc) return rc;
  }
  const int64_t ws_bytes = num_splits > 1 ? glm53_sparse_mla_workspace_bytes(num_tokens, num_heads, num_splits) : 0;
  return run_attention(a, num_tokens, num_heads, num_splits, ws, ws_bytes, out, so_t, so_h, stream);
}

extern "C" int glm53_sparse_mla(const void* q, int64_t sq_t, int64_t sq_h, const void* kv,
                                int64_t skv_t, int64_t seq_kv, const int32_t* indices,
                                int64_t si_t, int64_t num_tokens, int64_t num_heads, int64_t topk,
                                double sm_scale, int64_t num_splits, void* workspace,
                                int64_t workspace_bytes, void* out, int64_t so_t, int64_t so_h,
                                void* stream) {
  MlaArgs a;
  int rc = prepare(a, q, sq_t, sq_h, kv, skv_t, seq_kv, indices, si_t, num_tokens, num_heads, topk,
                   sm_scale, num_splits);
  if (rc) return rc;
  if (num_tokens == 0) return 0;
  return run_attention(a, num_tokens, num_heads, num_splits, workspace, workspace_bytes, out, so_t,
                       so_h, stream);
}

extern "C" int glm53_sparse_mla_paged(const void* q, int64_t sq_t, int64_t sq_h, const void* kv_pages,
                                      int64_t page_bytes, int64_t row_bytes, int64_t num_blocks,
                                      const int32_t* req_indices, int64_t si_t,
                                      const int32_t* req_id, const int32_t* block_table,
                                      int64_t num_reqs, int64_t bt_stride, int64_t max_blocks,
                                      int64_t block_size, int64_t num_tokens, int64_t num_heads,
                                      int64_t topk, double sm_scale, int64_t num_splits,
                                      void* workspace, int64_t workspace_bytes, void* out,
                                      int64_t so_t, int64_t so_h, void* stream) {
  if (num_blocks < 0 || row_bytes < 528 || page_bytes < 0 || page_bytes % 16 || row_bytes % 16)
    return num_blocks < 0 || row_bytes < 528 || page_bytes < 0 ? GLM53_ERR_BAD_SHAPE : GLM53_ERR_MISALIGNED;
  MlaArgs a;
  int rc = prepare(a, q, sq_t, sq_h, kv_pages, row_bytes, num_blocks, req_indices, si_t, num_tokens,
                   num_heads, topk, sm_scale, num_splits);
  if (rc) return rc;
  if (num_tokens == 0) return 0;
  rc = check_paged(req_id, block_table, num_reqs, bt_stride, max_blocks, block_size, block_size);
  if (rc) return rc;
  // Rows of a page must fit in it, and every row's 16-byte unit index in an int.
  if (num_blocks > 0 && (page_bytes < (block_size - 1) * row_bytes + 528 ||
                         (num_blocks * page_bytes) / 16 > 0x7fffffff))
    return GLM53_ERR_BAD_SHAPE;
  a.req_id = req_id;
  a.bt = block_table ? block_table : req_id;   // num_reqs == 0: never read
  a.num_reqs = block_table ? static_cast<int>(num_reqs) : 0;
  a.bt_stride = bt_stride;
  a.max_blocks = static_cast<int>(max_blocks);
  a.block_size = static_cast<int>(block_size);
  a.num_blocks = static_cast<int>(num_blocks);
  a.page_units = static_cast<int>(page_bytes / 16);
  a.row_units = static_cast<int>(row_bytes / 16);
  return run_attention(a, num_tokens, num_heads, num_splits, workspace, workspace_bytes, out, so_t,
                       so_h, stream);
}

extern "C" int glm53_convert_req_index(const int32_t* req_id, const int32_t* block_table,
                                       int64_t num_reqs, int64_t bt_stride, int64_t max_blocks,
                                       const int32_t* indices, int64_t si_t, int32_t* out,
                                       int64_t so_t, int64_t num_tokens, int64_t topk,
                                       int64_t block_size, int64_t page_rows, void* stream) {
  if (num_tokens < 0 || topk < 0 || num_tokens > 0x7fffffff || topk > 0x7fffffff)
    return GLM53_ERR_BAD_SHAPE;
  if (num_tokens == 0 || topk == 0) return 0;
  if (!indices || !out) return GLM53_ERR_NULL_POINTER;
  int rc = check_paged(req_id, block_table, num_reqs, bt_stride, max_blocks, block_size, page_rows);
  if (rc) return rc;
  if (num_tokens > 65535) return GLM53_ERR_BAD_SHAPE;   // grid y
  (void)hipGetLastError();
  hipLaunchKernelGGL(convert_req_index_kernel,
                     dim3(static_cast<unsigned>((topk + 255) / 256), static_cast<unsigned>(num_tokens)),
                     dim3(256), 0, static_cast<hipStream_t>(stream), req_id,
                     block_table ? block_table : req_id, bt_stride, static_cast<int>(max_blocks),
                     block_table ? static_cast<int>(num_reqs) : 0, indices, si_t, out, so_t, static_cast<int>(topk), static_cast<int>(block_size),
                     static_cast<int>(page_rows));
  return static_cast<int>(hipGetLastError());
}

extern "C" int glm53_expand_pools(const void* pool_ids, int ids_is_i64, int64_t sp_t,
                                  int64_t num_pools, const int32_t* seq_lens, int64_t pool_size,
                                  int32_t* out, int64_t so_t, int64_t num_rows, int64_t out_cols,
                                  void* stream) {
  if (num_rows < 0 || num_pools < 0 || out_cols < 0 || pool_size < 1 || num_rows > 65535 ||
      num_pools * pool_size + pool_size > 0x7fffffff || out_cols > 0x7fffffff)
    return GLM53_ERR_BAD_SHAPE;
  if (num_rows == 0 || out_cols == 0) return 0;
  if (!out || (!pool_ids && num_pools > 0)) return GLM53_ERR_NULL_POINTER;
  const dim3 grid(static_cast<unsigned>((out_cols + 255) / 256), static_cast<unsigned>(num_rows));
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  if (ids_is_i64)
    hipLaunchKernelGGL(expand_pools_kernel<int64_t>, grid, dim3(256), 0, st,
                       static_cast<const int64_t*>(pool_ids), sp_t, static_cast<int>(num_pools),
                       static_cast<int>(pool_size), seq_lens, out, so_t, static_cast<int>(out_cols));
  else
    hipLaunchKernelGGL(expand_pools_kernel<int32_t>, grid, dim3(256), 0, st,
                       static_cast<const int32_t*>(pool_ids), sp_t, static_cast<int>(num_pools),
                       static_cast<int>(pool_size), seq_lens, out, so_t, static_cast<int>(out_cols));
  return static_cast<int>(hipGetLastError());
}

extern "C" int glm53_sparse_mla_pooled(const void* q, int64_t sq_t, int64_t sq_h, const void* kv_pages,
                                       int64_t page_bytes, int64_t row_bytes, int64_t num_blocks,
                                       const int32_t* pool_ids, int64_t sp_t, int64_t num_pools,
                                       const int32_t* seq_lens, int64_t pool_size,
                                       const int32_t* req_id, const int32_t* block_table,
                                       int64_t num_reqs, int64_t bt_stride, int64_t max_blocks,
                                       int64_t block_size, int64_t num_tokens, int64_t num_heads,
                                       int64_t topk, double sm_scale, int64_t num_splits,
                                       void* workspace, int64_t workspace_bytes, void* out,
                                       int64_t so_t, int64_t so_h, void* stream) {
  if (num_pools < 0 || pool_size < 1 || num_pools * pool_size + pool_size > 0x7fffffff)
    return GLM53_ERR_BAD_SHAPE;
  if (num_tokens > 0 && num_pools > 0 && !pool_ids) return GLM53_ERR_NULL_POINTER;
  if (num_blocks < 0 || row_bytes < 528 || page_bytes < 0 || page_bytes % 16 || row_bytes % 16)
    return num_blocks < 0 || row_bytes < 528 || page_bytes < 0 ? GLM53_ERR_BAD_SHAPE : GLM53_ERR_MISALIGNED;
  MlaArgs a;
  // pool_ids stand in for the index pointer (never read as indices)
  int rc = prepare(a, q, sq_t, sq_h, kv_pages, row_bytes, num_blocks,
                   pool_ids ? pool_ids : reinterpret_cast<const int32_t*>(req_id), sp_t, num_tokens,
                   num_heads, topk, sm_scale, num_splits);
  if (rc) return rc;
  if (num_tokens == 0) return 0;
  rc = check_paged(req_id, block_table, num_reqs, bt_stride, max_blocks, block_size, block_size);
  if (rc) return rc;
  if (num_blocks > 0 && (page_bytes < (block_size - 1) * row_bytes + 528 ||
                         (num_blocks * page_bytes) / 16 > 0x7fffffff))
    return GLM53_ERR_BAD_SHAPE;
  a.req_id = req_id;
  a.bt = block_table ? block_table : req_id;
  a.num_reqs = block_table ? static_cast<int>(num_reqs) : 0;
  a.bt_stride = bt_stride;
  a.max_blocks = static_cast<int>(max_blocks);
  a.block_size = static_cast<int>(block_size);
  a.num_blocks = static_cast<int>(num_blocks);
  a.page_units = static_cast<int>(page_bytes / 16);
  a.row_units = static_cast<int>(row_bytes / 16);
  a.pools = pool_ids ? pool_ids : req_id;    // num_pools == 0: never read
  a.sp_t = sp_t;
  a.num_pools = static_cast<int>(num_pools);
  a.pool_size = static_cast<int>(pool_size);
  a.seq_lens = seq_lens;
  return run_attention(a, num_tokens, num_heads, num_splits, workspace, workspace_bytes, out, so_t,
                       so_h, stream);
}

extern "C" int glm53_sparse_mla_partials(const void* q, int64_t sq_t, int64_t sq_h, const void* kv,
                                         int64_t skv_t, int64_t seq_kv, const int32_t* indices,
                                         int64_t si_t, int64_t num_tokens, int64_t num_heads,
                                         int64_t topk, double sm_scale, int64_t num_splits,
                                         void* partials, int64_t partials_bytes, void* stream) {
  MlaArgs a;
  int rc = prepare(a, q, sq_t, sq_h, kv, skv_t, seq_kv, indices, si_t, num_tokens, num_heads, topk,
                   sm_scale, num_splits);
  if (rc) return rc;
  if (num_tokens == 0) return 0;
  const int64_t need = glm53_sparse_mla_partials_bytes(num_tokens, num_heads, num_splits);
  if (!partials || partials_bytes < need) return GLM53_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(partials) % 16) return GLM53_ERR_MISALIGNED;
  const int64_t rows = partial_rows(num_tokens, num_heads, num_splits);
  a.part = static_cast<float*>(partials);
  a.lse = static_cast<float*>(partials) + rows * kLatent;
  a.partials_only = 1;
  (void)hipGetLastError();
  launch_attention(a, num_tokens, static_cast<hipStream_t>(stream));
  return static_cast<int>(hipGetLastError());
}

extern "C" int glm53_sparse_mla_gather_floor(const void* q, int64_t sq_t, int64_t sq_h, const void* kv,
                                             int64_t skv_t, int64_t seq_kv, const int32_t* indices,
                                             int64_t si_t, int64_t num_tokens, int64_t num_heads,
                                             int64_t topk, int64_t num_splits, void* partials,
                                             int64_t partials_bytes, void* stream) {
  MlaArgs a;
  int rc = prepare(a, q, sq_t, sq_h, kv, skv_t, seq_kv, indices, si_t, num_tokens, num_heads, topk, 1.0,
                   num_splits);
  if (rc) return rc;
  if (num_tokens == 0) return 0;
  const int64_t need = glm53_sparse_mla_partials_bytes(num_tokens, num_heads, num_splits);
  if (!partials || partials_bytes < need) return GLM53_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(partials) % 16) return GLM53_ERR_MISALIGNED;
  if (a.split_len > kChunkTiles * kTile) return GLM53_ERR_BAD_SHAPE;   // decode splits only
  if (seq_kv < 1) return GLM53_ERR_BAD_SHAPE;                          // masked keys read row 0
  const int64_t rows = partial_rows(num_tokens, num_heads, num_splits);
  a.part = static_cast<float*>(partials);
  a.lse = static_cast<float*>(partials) + rows * kLatent;
  const dim3 grid(static_cast<unsigned>(a.num_splits), static_cast<unsigned>(num_tokens),
                  static_cast<unsigned>(a.heads_padded / kHeads));
  (void)hipGetLastError();
  // the split kernel's workgroup shape for this split length (three key
  // groups for 3-tile splits, one for 1-tile splits)
  const hipStream_t st = static_cast<hipStream_t>(stream);
#define GLM53_LEAD a.idx, a.si_t, a.split_len, a.topk, static_cast<int>(grid.x), static_cast<int>(grid.y), \
                   static_cast<int>(grid.z), a.num_heads, a.q, a.sq_t, a.sq_h, a
  if (a.split_len > 2 * kTile && a.split_len <= 3 * kTile)
    hipLaunchKernelGGL(sparse_mla_gather_floor_kernel<3>, grid, dim3(SplitShape<3>::kThreads), 0, st, GLM53_LEAD);
  else if (a.split_len <= kTile)
    hipLaunchKernelGGL(sparse_mla_gather_floor_kernel<1>, grid, dim3(SplitShape<1>::kThreads), 0, st, GLM53_LEAD);
  else
    hipLaunchKernelGGL(sparse_mla_gather_floor_kernel<2>, grid, dim3(kThreads), 0, st, GLM53_LEAD);
#undef GLM53_LEAD
  return static_cast<int>(hipGetLastError());
}

extern "C" int glm53_sparse_mla_merge(const void* partials, int64_t partials_bytes, int64_t num_tokens,
                                      int64_t num_heads, int64_t num_splits, void* out, int64_t so_t,
                                      int64_t so_h, void* stream) {
  if (num_tokens < 0 || num_heads < 1 || num_splits < 1 || num_splits > kMaxMergeSplits)
    return GLM53_ERR_BAD_SHAPE;
  if (num_tokens == 0) return 0;
  const int64_t need = glm53_sparse_mla_partials_bytes(num_tokens, num_heads, num_splits);
  if (!partials || partials_bytes < need) return GLM53_ERR_WORKSPACE;
  if (!out) return GLM53_ERR_NULL_POINTER;
  if (reinterpret_cast<uintptr_t>(partials) % 16 || reinterpret_cast<uintptr_t>(out) % 8 || so_t % 4 ||
      so_h % 4)
    return GLM53_ERR_MISALIGNED;
  const int64_t rows = partial_rows(num_tokens, num_heads, num_splits);
  const int hp = static_cast<int>((num_heads + kHeads - 1) / kHeads * kHeads);
  const float* part = static_cast<const float*>(partials);
  (void)hipGetLastError();
  launch_merge(part, part + rows * kLatent, num_tokens, static_cast<int>(num_splits), hp,
               static_cast<int>(num_heads), static_cast<uint16_t*>(out), so_t, so_h,
               static_cast<hipStream_t>(stream));
  return static_cast<int>(hipGetLastError());
}

extern "C" int glm53_abi_version(void) { return GLM53_ABI_VERSION; }

extern "C" const char* glm53_error_string(int code) {
  switch (code) {
    case 0: return "success";
    case GLM53_ERR_NULL_POINTER: return "null pointer argument";
    case GLM53_ERR_BAD_SHAPE: return "unsupported shape or size";
    case GLM53_ERR_MISALIGNED: return "pointer or stride not aligned as required";
    case GLM53_ERR_WORKSPACE: return "workspace missing or too small";
    case GLM53_ERR_BAD_DTYPE: return "unsupported dtype";
    case GLM53_ERR_SCRATCH_LIMIT:
      return "split partials exceed the static scratch of glm53_sparse_mla_noalloc "
             "(GLM53_NOALLOC_MAX_PARTIAL_ROWS rows of tokens x splits x heads rounded up to 16)";
    default: return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "unknown error";
  }
}
