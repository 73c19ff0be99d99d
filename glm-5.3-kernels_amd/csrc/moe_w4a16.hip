// W4A16 group-32 MoE expert GEMMs for gfx950: the consumer of the small
// route aligner at the GLM-5.3 decode shape (1..8 tokens, top-8 of 288
// experts, hidden 4096, per-rank expert intermediate 512).
//
// The computation is the one vLLM's fused Marlin MoE performs at that call
// site (profiles/sm74/titan_prefill/marlin.py:424-444 composes it from the
// same pieces; its gate, marlin.py:255-310, fixes the geometry):
//   c1[r]  = bf16(x[token(r)] . W13[e(r)]^T)               [R, 2N]
//   c2[r]  = bf16(silu(min(gate, L)) * clamp(up, -L, L))   [R, N], gate = c1[r, :N], up = c1[r, N:]
//   c3[r]  = bf16(w_r * (c2[r] . W2[e(r)]^T))               [R, K]
//   out[t] = bf16(sum over the token's 8 routes of c3)      [T, K]
// with W = (q - 8) * s: q an unsigned 4-bit code (uint4b8), s one bf16 scale
// per 32 consecutive input features of an output row.
//
// Weight layout (glm53_moe_w4a16_repack): the checkpoint's int32
// [E][n_out][K/8] words (word w of row n holds k = 8w + i in bits 4i) become
// tiles [E][n_out/16][K/128][64 lanes][4 words].  Lane l of a tile holds
// output row 16*tile + l%16; its word i holds k = 32*(4c + i) + 8*(l/16) +
// [0, 8) for the tile's 128-feature chunk c, with k = 2j in bits 4j and k =
// 2j + 1 in bits 16 + 4j.  So a 16-byte load per lane brings four groups of
// the MFMA's B operand, and (word >> 4j) & 0x000F000F | 0x43004300 is the
// bf16 pair (128 + q_2j, 128 + q_2j+1) with two VALU ops.  The checkpoint's
// bf16 scales [E][n_out][K/32] are reordered the same way, [E][n_out/16]
// [K/128][16 rows][4 groups]: a lane's four scales of a chunk are 8 bytes and
// the 16 rows of a tile's chunk one 128-byte line (row-major scales put the
// 16 rows 256 bytes apart, sixteen lines per load instruction).
//
// Per group of 32 features, D[m][n] = X[m][32] . B[32][n] runs on
// v_mfma_f32_16x16x32_bf16 with A = the activation rows (m = route slot) and
// B = the (128 + q) codes; a first MFMA with B = -136 everywhere seeds the
// accumulator with -136 * sum(x), so D = sum x * (q - 8) exactly as the group
// needs it, and the group's scale enters with one fp32 FMA per output:
// lane (l/16, l%16) holds column n = l%16 and rows m = 4*(l/16) + [0, 4), so
// each lane needs the single scale of its column.
//
// Gate/up kernels: the streaming kernel (K = 4096) gives each wavefront a
// tile pair (over all of K, or a part of K when there are few tile pairs)
// with a short register ring of weight chunks; the split-K kernel (other
// widths) runs one workgroup per (aligner block of 8 route slots, run of
// 16-column tiles), 8 wavefronts split K, and each tile's 8 partial tiles are
// summed in LDS in wave order.
// Down kernel: one workgroup per (token, 16 output features); wavefront j
// computes route slot j of the token (its expert's 16 rows over N), the 8
// weighted results are summed in slot order.  Both kernels are deterministic.
#include "moe_route.h"

namespace glm53 {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kTileN = 16;        // output rows per tile
constexpr int kChunkK = 128;      // features per 16-byte lane load (4 groups)
constexpr int kGroup = 32;
constexpr int kBatch = 4;         // chunks per wave whose loads are in flight together
constexpr int kBlock = 8;         // route slots per aligner block
constexpr uint32_t kMagic = 0x43004300u;   // bf16 pair (128, 128)
constexpr uint32_t kMinus136 = 0xC308C308u;  // bf16 pair (-136, -136)

// 0x000F000F in a VGPR.  With the mask in a register (and the magic in an
// SGPR) the compiler forms one v_and_or_b32 per pair; with both as literals
// it needs v_and + v_or (a VOP3 instruction takes no literal on gfx950).
__device__ __forceinline__ uint32_t nibble_mask() {
  uint32_t m;
  asm volatile("v_mov_b32 %0, 0xf000f" : "=v"(m));
  return m;
}

// The codes of one repacked word as the bf16x8 B operand (128 + q each).
__device__ __forceinline__ bf16x8 codes_to_bf16(uint32_t v, uint32_t mask) {
  uint4 r;
  r.x = (v & mask) | kMagic;
  r.y = ((v >> 4) & mask) | kMagic;
  r.z = ((v >> 8) & mask) | kMagic;
  r.w = ((v >> 12) & mask) | kMagic;
  return __builtin_bit_cast(bf16x8, r);
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// ------------------------------------------------------------------ repack
__global__ __launch_bounds__(256) void moe_w4a16_repack_kernel(const uint32_t* __restrict__ src,
                                                               const uint16_t* __restrict__ src_s,
                                                               uint32_t* __restrict__ dst,
                                                               uint16_t* __restrict__ dst_s,
                                                               int64_t total_words, int k_chunks) {
  const int64_t d = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (d >= total_words) return;
  const int i = static_cast<int>(d & 3);
  const int l = static_cast<int>((d >> 2) & 63);
  const int64_t rest = d >> 8;                  // (e * n_tiles + tile) * k_chunks + c
  const int c = static_cast<int>(rest % k_chunks);
  const int64_t et = rest / k_chunks;           // e * n_tiles + tile
  const int64_t row = et * kTileN + (l & 15);   // e * n_out + n
  const int k_words = 16 * k_chunks;
  const uint32_t w = src[row * k_words + 4 * (4 * c + i) + (l >> 4)];
  uint32_t o = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    o |= ((w >> (8 * j)) & 0xFu) << (4 * j);            // k = 2j
    o |= ((w >> (8 * j + 4)) & 0xFu) << (16 + 4 * j);   // k = 2j + 1
  }
  dst[d] = o;
  if (l < kTileN)   // scale of row l, group 4c + i
    dst_s[rest * 64 + 4 * l + i] = src_s[row * (4 * k_chunks) + 4 * c + i];
}

// ------------------------------------------------------------------ gate/up
constexpr int kMaxHidden = 4096;          // activation rows staged in LDS
constexpr int kXStride = kMaxHidden + 8;  // 16-byte pad: the 8 rows start 4 banks apart
constexpr int kMaxInter = 2048;           // c2 rows staged in LDS by the down kernel
constexpr int kActStride = kMaxInter + 8;

struct GateUpArgs {
  const uint16_t* x;        // bf16 [T][K], row stride sx (elements)
  int64_t sx;
  const uint4* w13;         // repacked [E][2N/16][K/128][64] uint4
  const uint16_t* s13;      // bf16 scales in tile order [E][2N/16][K/128][16][4]
  const int32_t* sorted_ids;  // aligner outputs (kSelfAlign = false)
  const int32_t* expert_ids;
  const void* topk_ids;     // contiguous [T * topk] routes (kSelfAlign = true)
  int ids_i64;
  int num_routes;           // R = T * topk (padding value of sorted_ids)
  int topk;
  int topk_log2;            // log2(topk) when topk is a power of two, else -1
  int tiles_per_wg;         // 16-column tiles per workgroup
  int num_experts;
  int n_inter;              // N
  int hidden;               // K
  float clamp;              // +inf: no clamp
  uint16_t* act;            // bf16 [R][N]
};

struct __align__(16) GateUpShared {
  uint16_t x[kBlock][kXStride];            // the block's activation rows
  f32x4 red[2][kWaves][2][64];             // partial tiles [buffer][wave][gate/up][lane]
};

// The MFMA loop over this wave's chunks of a gate tile and an up tile.
// kSingle: only D row 0 (slot 0) is kept, so one scale FMA per group and tile
// instead of four.
template <bool kSingle>
__device__ __forceinline__ void gate_up_chunks(const uint16_t* xs, int c_lo, int cpw, int k_chunks,
                                               const uint4 (&kg)[kBatch], const uint4 (&ku)[kBatch],
                                               const uint2 (&scg)[kBatch], const uint2 (&scu)[kBatch],
                                               f32x4& acc_g, f32x4& acc_u) {
  const bf16x8 minus136 = __builtin_bit_cast(bf16x8, make_uint4(kMinus136, kMinus136, kMinus136, kMinus136));
  const uint32_t mask = nibble_mask();
#pragma unroll
  for (int u = 0; u < kBatch; u++) {
    const int c = c_lo + u;
    if (u >= cpw || c >= k_chunks) break;   // uniform
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const bf16x8 xv = *reinterpret_cast<const bf16x8*>(xs + kChunkK * c + kGroup * i);
      const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
      const f32x4 corr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xv, minus136, zero, 0, 0, 0);
      const f32x4 dg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xv, codes_to_bf16(word_of(kg[u], i), mask), corr, 0, 0, 0);
      const f32x4 du = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xv, codes_to_bf16(word_of(ku[u], i), mask), corr, 0, 0, 0);
      const uint32_t pg = i < 2 ? scg[u].x : scg[u].y;
      const uint32_t pu = i < 2 ? scu[u].x : scu[u].y;
      const float s_g = __uint_as_float((i & 1) ? (pg & 0xFFFF0000u) : (pg << 16));
      const float s_u = __uint_as_float((i & 1) ? (pu & 0xFFFF0000u) : (pu << 16));
#pragma unroll
      for (int r = 0; r < (kSingle ? 1 : 4); r++) {
        acc_g[r] = __builtin_fmaf(s_g, dg[r], acc_g[r]);
        acc_u[r] = __builtin_fmaf(s_u, du[r], acc_u[r]);
      }
    }
  }
}

// Workgroup barrier for LDS traffic only: this wave's LDS accesses are
// complete (lgkmcnt 0) and no memory access moves across it.  Unlike
// __syncthreads(), whose release fence waits for every outstanding global
// load (vmcnt 0), it keeps the next tile's weight loads in flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One gate/up tile pair's operands for this wave: codes and scales of its
// chunks of the gate tile and of the up tile.
struct TileRegs {
  uint4 kg[kBatch], ku[kBatch];
  uint2 scg[kBatch], scu[kBatch];
};

__device__ __forceinline__ void load_tile(TileRegs& t, const GateUpArgs& a, int e, int jt, int c_lo, int cpw,
                                          int k_chunks, int lane, int col) {
  // Uniform tile bases (SGPRs) plus 32-bit lane offsets: each load is
  // base + lane offset + an immediate chunk offset.
  const int n_tiles13 = 2 * a.n_inter / kTileN;
  const int64_t tg = (static_cast<int64_t>(e) * n_tiles13 + jt) * k_chunks + c_lo;
  const int64_t tu = tg + static_cast<int64_t>(a.n_inter / kTileN) * k_chunks;
  const uint4* wg = a.w13 + tg * 64;
  const uint4* wu = a.w13 + tu * 64;
  const uint16_t* sg = a.s13 + tg * 64;
  const uint16_t* su = a.s13 + tu * 64;
#pragma unroll
  for (int u = 0; u < kBatch; u++) {   // chunks past the wave's range re-read its last one (not used)
    const int uu = c_lo + (u < cpw ? u : cpw - 1) < k_chunks ? (u < cpw ? u : cpw - 1) : k_chunks - 1 - c_lo;
    t.kg[u] = wg[64 * uu + lane];
    t.ku[u] = wu[64 * uu + lane];
    t.scg[u] = *reinterpret_cast<const uint2*>(sg + 64 * uu + 4 * col);
    t.scu[u] = *reinterpret_cast<const uint2*>(su + 64 * uu + 4 * col);
  }
  // Keep the loads here: the scheduler would otherwise sink them toward
  // their uses (behind the previous tile's compute), defeating the prefetch.
  __builtin_amdgcn_sched_barrier(0);
}

// Sum the 8 waves' partial tiles (fixed order), SiLU-and-multiply, store c2.
__device__ __forceinline__ void finish_tile(GateUpShared& sh, int buf, const GateUpArgs& a, int jt,
                                            const int (&slot)[kBlock], const f32x4& acc_g, const f32x4& acc_u,
                                            int w, int lane) {
  sh.red[buf][w][0][lane] = acc_g;
  sh.red[buf][w][1][lane] = acc_u;
  lds_barrier();
  if (threadIdx.x < kTileN * kBlock) {
    const int n = threadIdx.x & 15;
    const int m = threadIdx.x >> 4;   // slot 0..7: D row m sits in lane n + 16*(m/4), element m%4
    int route = a.num_routes;
#pragma unroll
    for (int mm = 0; mm < kBlock; mm++)
      if (m == mm) route = slot[mm];
    if (route < a.num_routes) {
      const float* rg = reinterpret_cast<const float*>(&sh.red[buf][0][0][n + 16 * (m >> 2)]) + (m & 3);
      const float* ru = reinterpret_cast<const float*>(&sh.red[buf][0][1][n + 16 * (m >> 2)]) + (m & 3);
      float g = 0.f, up = 0.f;
#pragma unroll
      for (int ww = 0; ww < kWaves; ww++) {   // wave stride: 2 * 64 float4
        g += rg[ww * 2 * 64 * 4];
        up += ru[ww * 2 * 64 * 4];
      }
      // compare-and-select rather than fminf/fmaxf: a NaN stays NaN (as
      // torch.clamp keeps it) instead of becoming a limit
      g = bf16_round(g);
      up = bf16_round(up);
      g = g > a.clamp ? a.clamp : g;
      up = up > a.clamp ? a.clamp : up < -a.clamp ? -a.clamp : up;
      const float v = g / (1.0f + expf(-g)) * up;
      a.act[static_cast<int64_t>(route) * a.n_inter + kTileN * jt + n] = static_cast<uint16_t>(f32_to_bf16_bits(v));
    }
  }
}

template <bool kSingle>
__device__ __forceinline__ void tile_step(GateUpShared& sh, int& buf, const GateUpArgs& a, int jt,
                                          const int (&slot)[kBlock], const uint16_t* xs, int c_lo, int cpw,
                                          int k_chunks, const TileRegs& t, int w, int lane) {
  f32x4 acc_g = {0.f, 0.f, 0.f, 0.f}, acc_u = {0.f, 0.f, 0.f, 0.f};
  gate_up_chunks<kSingle>(xs, c_lo, cpw, k_chunks, t.kg, t.ku, t.scg, t.scu, acc_g, acc_u);
  finish_tile(sh, buf, a, jt, slot, acc_g, acc_u, w, lane);
  buf ^= 1;
}

// The tiles [jt0, jt_end) of one block (jt_end - jt0 <= kTpw), fully
// unrolled: the next tile's loads are in flight while a tile is computed and
// finished (two register sets, two reduction buffers, one workgroup barrier
// per tile).  Loads past jt_end re-read the last tile, so every register set
// is defined on every path and no load waits on a branch merge.
template <bool kSingle, int kTpw>
__device__ __forceinline__ void gate_up_tiles(GateUpShared& sh, const GateUpArgs& a, int e, int jt0, int jt_end,
                                              const int (&slot)[kBlock], const uint16_t* xs, int c_lo, int cpw,
                                              int k_chunks, TileRegs (&t)[2], int w, int lane, int col) {
  int buf = 0;
#pragma unroll
  for (int i = 0; i < kTpw; i++) {
    if (i + 1 < kTpw) {
      const int jn = jt0 + i + 1 < jt_end ? jt0 + i + 1 : jt_end - 1;
      load_tile(t[(i + 1) & 1], a, e, jn, c_lo, cpw, k_chunks, lane, col);
    }
    if (jt0 + i < jt_end)   // uniform
      tile_step<kSingle>(sh, buf, a, jt0 + i, slot, xs, c_lo, cpw, k_chunks, t[i & 1], w, lane);
  }
}

template <bool kSingle>
__device__ __forceinline__ void gate_up_dispatch(GateUpShared& sh, const GateUpArgs& a, int e, int jt0, int jt_end,
                                                 const int (&slot)[kBlock], const uint16_t* xs, int c_lo, int cpw,
                                                 int k_chunks, TileRegs (&t)[2], int w, int lane, int col) {
  switch (a.tiles_per_wg) {
    case 1: gate_up_tiles<kSingle, 1>(sh, a, e, jt0, jt_end, slot, xs, c_lo, cpw, k_chunks, t, w, lane, col); break;
    case 2: gate_up_tiles<kSingle, 2>(sh, a, e, jt0, jt_end, slot, xs, c_lo, cpw, k_chunks, t, w, lane, col); break;
    case 4: gate_up_tiles<kSingle, 4>(sh, a, e, jt0, jt_end, slot, xs, c_lo, cpw, k_chunks, t, w, lane, col); break;
    default: gate_up_tiles<kSingle, 8>(sh, a, e, jt0, jt_end, slot, xs, c_lo, cpw, k_chunks, t, w, lane, col); break;
  }
}

// kSelfAlign: the workgroup derives its aligner block (expert and 8 slots)
// from the routes itself, with the aligner's ballots, instead of loading
// sorted_ids / expert_ids: one launch and one dependent load fewer.
// Workgroup (b, g) computes tiles [g * tiles_per_wg, +tiles_per_wg) of block b.
template <bool kSelfAlign>
__global__ __launch_bounds__(kThreads) void moe_w4a16_gate_up_kernel(const GateUpArgs a) {
  __shared__ GateUpShared sh;
  const int b = blockIdx.x;
  const int n_half = a.n_inter / kTileN;
  const int jt0 = blockIdx.y * a.tiles_per_wg;
  const int jt_end = jt0 + a.tiles_per_wg < n_half ? jt0 + a.tiles_per_wg : n_half;
  if (jt0 >= n_half) return;
  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int q = lane >> 4, col = lane & 15;
  const int R = a.num_routes;

  int slot[kBlock];   // route of each slot of the block (R = padding); wave-uniform
  int e;
  if (kSelfAlign) {
    const bool in = lane < R;
    const RoutePos rp = align_routes(in ? load_route_id(a.topk_ids, a.ids_i64, lane) : -1, in);
#pragma unroll
    for (int m = 0; m < kBlock; m++) {
      const uint64_t hit = __ballot(rp.valid && rp.pos == kBlock * b + m);
      slot[m] = hit ? __builtin_ctzll(hit) : R;
    }
    e = slot[0] < R ? __builtin_amdgcn_readlane(rp.key, slot[0]) : -1;
  } else {
    e = a.expert_ids[b];
#pragma unroll
    for (int m = 0; m < kBlock; m++) slot[m] = a.sorted_ids[kBlock * b + m];
  }
  if (e < 0 || e >= a.num_experts) return;   // unused block (uniform over the workgroup)

  // Wave w owns chunks [cpw*w, cpw*w + cpw) of K (cpw <= kBatch) and stages
  // the block's activation rows over that range into LDS once; the MFMA loop
  // reads only what this wave wrote, so no barrier is needed before it.
  // Slot 0 (always routed) is loaded before the first tile's weights and
  // stored after them, so its latency hides under theirs; further routed
  // slots (blocks shared by several tokens) follow one by one.  (Plain loads,
  // not global->LDS DMA: pending DMA makes the compiler wait for every
  // outstanding load before each LDS access, which would drain the weight
  // prefetch at every tile.)
  const int k_chunks = a.hidden / kChunkK;
  const int cpw = (k_chunks + kWaves - 1) / kWaves;
  const int c_lo = cpw * w;
  // A wave whose range starts at or past the end of the row (hidden sizes
  // that do not fill all waves, e.g. 640 = 5 chunks over 8 waves) computes
  // nothing and stages nothing: its activation offset would lie past the row.
  const int kbase = kChunkK * c_lo;                 // first feature of this wave
  const bool stage = kbase < a.hidden;              // uniform over the wave
  const int xo = kbase + 8 * (8 * lane < kChunkK * cpw && kbase + 8 * lane < a.hidden ? lane : 0);
  auto x_row = [&](int route) {
    const unsigned r = static_cast<unsigned>(route);
    const unsigned tok = a.topk_log2 >= 0 ? r >> a.topk_log2 : r / static_cast<unsigned>(a.topk);
    return reinterpret_cast<const uint4*>(a.x + static_cast<int64_t>(tok) * a.sx + xo);
  };
  const uint4 x0 = stage ? *x_row(slot[0]) : make_uint4(0, 0, 0, 0);
  TileRegs t[2];
  load_tile(t[0], a, e, jt0, c_lo, cpw, k_chunks, lane, col);
  if (stage) {
    *reinterpret_cast<uint4*>(&sh.x[0][xo]) = x0;
#pragma unroll
    for (int m = 1; m < kBlock; m++)
      if (slot[m] < R) *reinterpret_cast<uint4*>(&sh.x[m][xo]) = *x_row(slot[m]);
  }

  // A-operand row of this lane (m = col): padding slots and m >= 8 read row 0
  // (their D rows are discarded), so a block with one route reads one row.
  int xrow = 0;
#pragma unroll
  for (int m = 1; m < kBlock; m++)
    if ((col & 7) == m && slot[m] < R) xrow = m;
  const uint16_t* xs = &sh.x[xrow][8 * q];

  bool single = true;                   // only slot 0 routed: D row 0 is the only one kept
#pragma unroll
  for (int m = 1; m < kBlock; m++) single = single && slot[m] >= R;
  if (single)
    gate_up_dispatch<true>(sh, a, e, jt0, jt_end, slot, xs, c_lo, cpw, k_chunks, t, w, lane, col);
  else
    gate_up_dispatch<false>(sh, a, e, jt0, jt_end, slot, xs, c_lo, cpw, k_chunks, t, w, lane, col);
}

// Weight codes and scales are read once per call: the decode kernels load
// them non-temporally (nt), which streams faster than plain loads (layer over
// a 4-layer weight rotation, gate/up and down both nt: B=8 44.8 -> 41.6 us,
// B=4 27.4 -> 25.1, B=2 16.9 -> 15.8, B=1 12.2 -> 11.6; bit-identical).
__device__ __forceinline__ uint4 load_once(const uint4* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 load_once(const uint2* p) {
  const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
  return make_uint2(v.x, v.y);
}

// ------------------------------------------------------------------ gate/up, streaming
// For K = 4096 (1..8 tokens at the decode shape): the waves of workgroup
// (b, g) are kTiles tile pairs x kKSplit parts of K, chosen so that about one
// workgroup per CU covers all tile pairs (8 x 1 at 8 tokens, 4 x 1 at 4, 2 x 4
// at 2, 1 x 8 at 1).  Wave (tile, part)
// computes its gate/up tile pair over its 32 / kKSplit chunks of K, streaming
// codes and scales through a ring of kStreamDepth chunks in registers (one
// chunk is computed while the next kStreamDepth - 1 are in flight) at its own
// memory pace: no barrier between the activation staging and the end.  With
// kKSplit > 1 the parts meet once in LDS and are added in part order.  A
// shallow ring streams best: B=8 layer 49.3 us (split-K kernel) -> 44.4 /
// 45.1 / 46.5 us with depth 4 / 6 / 8, and 12 or 15 slower again; depths 2-4
// are within 2 %.  Same arithmetic per group as the split-K kernel (all four
// D rows always kept: one code path, so the compiler has no shared
// conversions to hoist above a branch); a wave adds its chunks in order.
constexpr int kStreamChunks = kMaxHidden / kChunkK;   // 32
constexpr int kStreamDepth = 3;

struct StreamRing {
  uint4 kg[kStreamDepth], ku[kStreamDepth];
  uint2 scg[kStreamDepth], scu[kStreamDepth];
};

// Chunks [c0, c0 + kCpw) of one tile pair; the ring holds chunks c0.. on entry.
// Per chunk: the four groups' MFMAs back to back (their activations read
// from LDS one chunk ahead), the ring slot refilled, then the scale FMAs in
// group order -- the same arithmetic as one group at a time, with fewer
// waits on LDS reads and MFMA results (B=8 layer 41.19 -> 40.84 us, B=2
// 15.87 -> 15.63 in an interleaved A/B; bit-identical).
template <int kCpw>
__device__ __forceinline__ void stream_chunks(const uint16_t* xs, const uint4* wg, const uint4* wu, const uint2* sg,
                                              const uint2* su, StreamRing& ring, int c0, int lane, f32x4& acc_g,
                                              f32x4& acc_u) {
  const bf16x8 minus136 = __builtin_bit_cast(bf16x8, make_uint4(kMinus136, kMinus136, kMinus136, kMinus136));
  const uint32_t mask = nibble_mask();
  const int col = lane & 15;
  bf16x8 xn[4];   // the next chunk's activations, read from LDS one chunk ahead
#pragma unroll
  for (int i = 0; i < 4; i++) xn[i] = *reinterpret_cast<const bf16x8*>(xs + kChunkK * c0 + kGroup * i);
#pragma unroll
  for (int c = 0; c < kCpw; c++) {
    const int r = c % kStreamDepth;
    bf16x8 xv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) xv[i] = xn[i];
    if (c + 1 < kCpw) {
#pragma unroll
      for (int i = 0; i < 4; i++) xn[i] = *reinterpret_cast<const bf16x8*>(xs + kChunkK * (c0 + c + 1) + kGroup * i);
    }
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 corr[4], dg[4], du[4];
#pragma unroll
    for (int i = 0; i < 4; i++) corr[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xv[i], minus136, zero, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      dg[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xv[i], codes_to_bf16(word_of(ring.kg[r], i), mask), corr[i], 0, 0, 0);
      du[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xv[i], codes_to_bf16(word_of(ring.ku[r], i), mask), corr[i], 0, 0, 0);
    }
    const uint2 pgs = ring.scg[r], pus = ring.scu[r];
    if (c + kStreamDepth < kCpw) {   // refill the slot just used (static condition)
      const int cn = c0 + c + kStreamDepth;
      ring.kg[r] = load_once(&wg[64 * cn + lane]);
      ring.ku[r] = load_once(&wu[64 * cn + lane]);
      ring.scg[r] = load_once(&sg[16 * cn + col]);
      ring.scu[r] = load_once(&su[16 * cn + col]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t pg = i < 2 ? pgs.x : pgs.y;
      const uint32_t pu = i < 2 ? pus.x : pus.y;
      const float s_g = __uint_as_float((i & 1) ? (pg & 0xFFFF0000u) : (pg << 16));
      const float s_u = __uint_as_float((i & 1) ? (pu & 0xFFFF0000u) : (pu << 16));
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        acc_g[rr] = __builtin_fmaf(s_g, dg[i][rr], acc_g[rr]);
        acc_u[rr] = __builtin_fmaf(s_u, du[i][rr], acc_u[rr]);
      }
    }
    // one chunk per scheduling region, its accumulation included: the
    // accumulators are otherwise only needed at the end, and the instruction
    // selector would defer every chunk's FMAs there (keeping all MFMA results
    // live)
    asm volatile("" : "+v"(acc_g), "+v"(acc_u));
    __builtin_amdgcn_sched_barrier(0);
  }
}

// bf16 gate/up, clamp, SiLU-and-multiply and the c2 store of one tile pair.
__device__ __forceinline__ void stream_finish(const GateUpArgs& a, const f32x4& acc_g, const f32x4& acc_u, int jt,
                                              const int (&slot)[kBlock], int lane) {
  // lane (q, col) holds column col of rows 4q + rr: slots 0..7 sit in q < 2
  const int q = lane >> 4, col = lane & 15;
#pragma unroll
  for (int rr = 0; rr < 4; rr++) {
    const int m = 4 * q + rr;
    int route = a.num_routes;
#pragma unroll
    for (int mm = 0; mm < kBlock; mm++)
      if (m == mm) route = slot[mm];
    if (q < 2 && route < a.num_routes) {
      // compare-and-select clamp: a NaN stays NaN (as torch.clamp keeps it)
      float g = bf16_round(acc_g[rr]);
      float up = bf16_round(acc_u[rr]);
      g = g > a.clamp ? a.clamp : g;
      up = up > a.clamp ? a.clamp : up < -a.clamp ? -a.clamp : up;
      const float v = g / (1.0f + expf(-g)) * up;
      a.act[static_cast<int64_t>(route) * a.n_inter + kTileN * jt + col] = static_cast<uint16_t>(f32_to_bf16_bits(v));
    }
  }
}

// one_token (with kSelfAlign): the call has a single token, so no block can
// hold routes of two tokens and the workgroup takes route b as its block --
// one uniform load of the route's expert, no ballots (B=1 layer 11.76 ->
// 11.17 us over the 4-layer rotation, bit-identical: a block's rows are
// computed independently, so a token routed twice to one expert gets the
// same c2 rows from two one-slot blocks as from one two-slot block).
template <bool kSelfAlign, int kTiles, int kKSplit>
__global__ __launch_bounds__(64 * kTiles * kKSplit) void moe_w4a16_gate_up_stream_kernel(
    const void* topk_ids, int ids_i64, int num_routes, const uint4* w13, const uint16_t* s13, const uint16_t* x,
    int64_t sx, int n_inter, int num_experts, int one_token, const GateUpArgs a) {
  constexpr int kW = kTiles * kKSplit;             // waves
  constexpr int kCpw = kStreamChunks / kKSplit;    // chunks per wave
  constexpr int kXPer = kWaves / kW;               // 512-feature activation pieces staged per wave
  static_assert(kCpw >= kStreamDepth, "the ring must fit a wave's chunks");
  static_assert(kW <= kWaves && kWaves % kW == 0, "1, 2, 4 or 8 waves");
  __shared__ __attribute__((aligned(16))) uint16_t xsh[kBlock][kXStride];
  __shared__ f32x4 red[kKSplit > 1 ? kW : 1][2][64];
  const int b = blockIdx.x;
  const int n_half = n_inter / kTileN;
  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int col = lane & 15;
  const int R = num_routes;

  int slot[kBlock];   // route of each slot of the block (R = padding); wave-uniform
  int e;
  if (kSelfAlign && one_token) {
    const int64_t raw = load_route_id(topk_ids, ids_i64, b);
    e = raw >= 0 && raw < num_experts ? static_cast<int>(raw) : -1;
    slot[0] = b;
#pragma unroll
    for (int m = 1; m < kBlock; m++) slot[m] = R;
  } else if (kSelfAlign) {
    const bool in = lane < R;
    const RoutePos rp = align_routes(in ? load_route_id(topk_ids, ids_i64, lane) : -1, in);
#pragma unroll
    for (int m = 0; m < kBlock; m++) {
      const uint64_t hit = __ballot(rp.valid && rp.pos == kBlock * b + m);
      slot[m] = hit ? __builtin_ctzll(hit) : R;
    }
    e = slot[0] < R ? __builtin_amdgcn_readlane(rp.key, slot[0]) : -1;
  } else {
    e = a.expert_ids[b];
#pragma unroll
    for (int m = 0; m < kBlock; m++) slot[m] = a.sorted_ids[kBlock * b + m];
  }
  if (e < 0 || e >= num_experts) return;   // unused block (uniform over the workgroup)

  // Activation rows: wave w stages features 512 (w + kW p) + [0, 512) of
  // every routed slot with direct global->LDS loads (no registers held while
  // the weights stream in).  They go out before the weight ring, so waiting
  // for them is vmcnt(ring loads).
#pragma unroll
  for (int m = 0; m < kBlock; m++) {
    if (slot[m] < R) {   // uniform
      const unsigned r = static_cast<unsigned>(slot[m]);
      const unsigned tok = a.topk_log2 >= 0 ? r >> a.topk_log2 : r / static_cast<unsigned>(a.topk);
      const uint16_t* xr = x + static_cast<int64_t>(tok) * sx;
#pragma unroll
      for (int p = 0; p < kXPer; p++)
        __builtin_amdgcn_global_load_lds(xr + 512 * (w + kW * p) + 8 * lane, &xsh[m][512 * (w + kW * p)], 16, 0, 0);
    }
  }

  const int part = w % kKSplit;
  const int jt = uniform(static_cast<int>(blockIdx.y) * kTiles + w / kKSplit);
  const int jtc = jt < n_half ? jt : n_half - 1;   // waves past the end load a real tile, store nothing
  const int64_t tg = (static_cast<int64_t>(e) * 2 * n_half + jtc) * kStreamChunks;
  const int64_t tu = tg + static_cast<int64_t>(n_half) * kStreamChunks;
  // uniform tile bases (SGPRs); each access adds the lane's 32-bit offset
  const uint4* wg = w13 + tg * 64;
  const uint4* wu = w13 + tu * 64;
  const uint2* sg = reinterpret_cast<const uint2*>(s13 + tg * 64);
  const uint2* su = reinterpret_cast<const uint2*>(s13 + tu * 64);
  const int c0 = part * kCpw;
  StreamRing ring;
#pragma unroll
  for (int c = 0; c < kStreamDepth; c++) {
    ring.kg[c] = load_once(&wg[64 * (c0 + c) + lane]);
    ring.ku[c] = load_once(&wu[64 * (c0 + c) + lane]);
    ring.scg[c] = load_once(&sg[16 * (c0 + c) + col]);
    ring.scu[c] = load_once(&su[16 * (c0 + c) + col]);
  }
  __builtin_amdgcn_sched_barrier(0);
  // vmcnt(4 * kStreamDepth): this wave's activation rows have landed in LDS
  static_assert(4 * kStreamDepth < 64, "vmcnt is 6 bits");
  constexpr int kRingLoads = 4 * kStreamDepth;
  __builtin_amdgcn_s_waitcnt((kRingLoads & 15) | ((kRingLoads >> 4) << 14) | (7 << 4) | (15 << 8));
  lds_barrier();

  int xrow = 0;   // A-operand row of this lane (m = col): unrouted slots and m >= 8 read row 0
#pragma unroll
  for (int m = 1; m < kBlock; m++)
    if ((col & 7) == m && slot[m] < R) xrow = m;
  const uint16_t* xs = &xsh[xrow][8 * (lane >> 4)];
  f32x4 acc_g = {0.f, 0.f, 0.f, 0.f}, acc_u = {0.f, 0.f, 0.f, 0.f};
  stream_chunks<kCpw>(xs, wg, wu, sg, su, ring, c0, lane, acc_g, acc_u);
  if (kKSplit > 1) {   // every wave reaches this barrier, also those past the last tile
    red[w][0][lane] = acc_g;
    red[w][1][lane] = acc_u;
    lds_barrier();
    if (part != 0) return;
#pragma unroll
    for (int k = 1; k < kKSplit; k++) {
      const f32x4 vg = red[w + k][0][lane], vu = red[w + k][1][lane];
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        acc_g[rr] += vg[rr];
        acc_u[rr] += vu[rr];
      }
    }
  }
  if (jt < n_half) stream_finish(a, acc_g, acc_u, jt, slot, lane);
}

// ------------------------------------------------------------------ down
struct DownArgs {
  const uint16_t* act;      // bf16 [T * topk][N]
  const uint4* w2;          // repacked [E][K/16][N/128][64] uint4
  const uint16_t* s2;       // bf16 scales in tile order [E][K/16][N/128][16][4]
  const void* topk_ids;     // [T][topk] int32 / int64, row stride sid_t
  int ids_i64;
  int64_t sid_t;
  const float* topk_w;      // fp32 [T][topk], row stride sw_t
  int64_t sw_t;
  int topk;
  int num_experts;
  int n_inter;              // N (the reduction length here)
  int hidden;               // K (output features)
  uint16_t* out;            // bf16 [T][K], row stride so
  int64_t so;
};

// Weight words and scales of chunks [c0, c0 + kBatch) of a down tile.
__device__ __forceinline__ void load_down_batch(const uint4* wp, const uint16_t* sp, int c0, int k_chunks,
                                                uint4 (&kw)[kBatch], uint2 (&sc)[kBatch]) {
#pragma unroll
  for (int u = 0; u < kBatch; u++) {   // chunks past N re-read the last one (not used)
    const int c = c0 + u < k_chunks ? c0 + u : k_chunks - 1;
    kw[u] = load_once(&wp[static_cast<int64_t>(c) * 64]);
    sc[u] = load_once(reinterpret_cast<const uint2*>(sp + 64 * c));
  }
}

struct __align__(16) DownShared {
  uint16_t act[kWaves][kActStride];   // the token's c2 rows
  float part[kWaves][kTileN];
};

__global__ __launch_bounds__(kThreads) void moe_w4a16_down_kernel(
    const void* topk_ids, int ids_i64, int topk, int64_t sid_t, const uint4* w2, const uint16_t* s2,
    const uint16_t* act, int n_inter, int hidden, const DownArgs a) {
  __shared__ DownShared sh;
  const int nt = blockIdx.x;
  const int t = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int q = lane >> 4, col = lane & 15;
  const int k_chunks = n_inter / kChunkK;
  const int n_tiles2 = hidden / kTileN;
  const bool has_route = w < topk;   // wave w computes route slot w (topk <= 8)

  // Route of this wave (the same id in every lane).
  int e = -1;
  if (has_route) {
    const int64_t raw = load_route_id(topk_ids, ids_i64, static_cast<int>(t * sid_t + w));
    e = uniform(raw >= 0 && raw < a.num_experts ? static_cast<int>(raw) : -1);
  }
  const uint4* wp = w2 + ((static_cast<int64_t>(e < 0 ? 0 : e) * n_tiles2 + nt) * k_chunks) * 64 + lane;
  const uint16_t* sp = s2 + ((static_cast<int64_t>(e < 0 ? 0 : e) * n_tiles2 + nt) * k_chunks) * 64 + 4 * col;
  // The wave's own c2 row into LDS with direct global->LDS loads (lane i ->
  // 16 bytes at i*16), then the first weight batch; only this wave reads the
  // row, so no workgroup barrier is needed before the MFMA loop.
  const uint16_t* act_r = act + (static_cast<int64_t>(t) * topk + w) * n_inter;
  if (e >= 0) {
    for (int k0 = 0; k0 < n_inter; k0 += 8 * 64)
      if (k0 + 8 * lane < n_inter)
        __builtin_amdgcn_global_load_lds(act_r + k0 + 8 * lane, &sh.act[w][k0], 16, 0, 0);
  }
  uint4 kw[kBatch];
  uint2 sc[kBatch];
  if (e >= 0) load_down_batch(wp, sp, 0, k_chunks, kw, sc);
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): the staged row is in LDS

  float y = 0.f;
  if (e >= 0) {
    const uint16_t* xs = &sh.act[w][8 * q];   // D row 0 is the route; the other rows repeat it
    const bf16x8 minus136 = __builtin_bit_cast(bf16x8, make_uint4(kMinus136, kMinus136, kMinus136, kMinus136));
    const uint32_t mask = nibble_mask();
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < k_chunks; c0 += kBatch) {
      if (c0 > 0) load_down_batch(wp, sp, c0, k_chunks, kw, sc);
#pragma unroll
      for (int u = 0; u < kBatch; u++) {
        const int c = c0 + u;
        if (c >= k_chunks) break;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const bf16x8 xv = *reinterpret_cast<const bf16x8*>(xs + kChunkK * c + kGroup * i);
          const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
          const f32x4 corr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xv, minus136, zero, 0, 0, 0);
          const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xv, codes_to_bf16(word_of(kw[u], i), mask), corr, 0, 0, 0);
          const uint32_t p = i < 2 ? sc[u].x : sc[u].y;
          const float s = __uint_as_float((i & 1) ? (p & 0xFFFF0000u) : (p << 16));
          acc[0] = __builtin_fmaf(s, d[0], acc[0]);   // D row 0: lanes 0..15, element 0
        }
      }
    }
    y = bf16_round(a.topk_w[t * a.sw_t + w] * acc[0]);
  }
  if (has_route && lane < kTileN) sh.part[w][lane] = y;
  __syncthreads();
  if (threadIdx.x < kTileN) {
    float s = 0.f;
    for (int ww = 0; ww < topk; ww++) s += sh.part[ww][threadIdx.x];
    a.out[t * a.so + kTileN * nt + threadIdx.x] = static_cast<uint16_t>(f32_to_bf16_bits(s));
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace glm53

using namespace glm53;

extern "C" int glm53_moe_w4a16_repack(const void* w_packed, const void* w_scale, int64_t num_experts,
                                      int64_t n_out, int64_t k, void* out, void* out_scale, void* stream) {
  if (!w_packed || !w_scale || !out || !out_scale) return GLM53_ERR_NULL_POINTER;
  if (num_experts < 1 || n_out < kTileN || n_out % kTileN || k < kChunkK || k % kChunkK)
    return GLM53_ERR_BAD_SHAPE;
  if (!aligned16(out) || (reinterpret_cast<uintptr_t>(w_packed) & 3) || (reinterpret_cast<uintptr_t>(w_scale) & 1) ||
      (reinterpret_cast<uintptr_t>(out_scale) & 7))
    return GLM53_ERR_MISALIGNED;
  const int64_t total = num_experts * n_out * (k / 8);
  (void)hipGetLastError();
  hipLaunchKernelGGL(moe_w4a16_repack_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint32_t*>(w_packed),
                     static_cast<const uint16_t*>(w_scale), static_cast<uint32_t*>(out),
                     static_cast<uint16_t*>(out_scale), total, static_cast<int>(k / kChunkK));
  return static_cast<int>(hipGetLastError());
}

namespace {

// Compute units of the current device (cached per device).
int num_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

int launch_gate_up(bool self_align, const void* x, int64_t sx, const void* w13, const void* s13,
                   const int32_t* sorted_ids, const int32_t* expert_ids, const void* topk_ids, int ids_is_i64,
                   int64_t num_routes, int64_t topk, int64_t num_experts, int64_t n_inter, int64_t hidden,
                   float clamp_limit, void* act, void* stream) {
  if (!x || !w13 || !s13 || !act) return GLM53_ERR_NULL_POINTER;
  if (self_align ? !topk_ids : (!sorted_ids || !expert_ids)) return GLM53_ERR_NULL_POINTER;
  if (num_routes < 1 || num_routes > (self_align ? kAlignMaxRoutes : (1 << 24)) || topk < 1 || num_experts < 1 ||
      n_inter < kTileN || n_inter % kTileN || hidden < kChunkK || hidden % kChunkK || hidden > kMaxHidden ||
      sx < hidden || !(clamp_limit > 0.f))
    return GLM53_ERR_BAD_SHAPE;
  if (!aligned16(x) || sx % 8 || !aligned16(w13) || (reinterpret_cast<uintptr_t>(s13) & 7) ||
      (reinterpret_cast<uintptr_t>(act) & 1))
    return GLM53_ERR_MISALIGNED;
  // Enough tiles per workgroup that the blocks' workgroups about fill the
  // CUs once (each block has n_inter / 16 tiles; at most num_routes blocks).
  const int64_t n_half = n_inter / kTileN;
  const int64_t want = (n_half * num_routes + num_cus() - 1) / num_cus();
  int64_t tpw = 1;                       // a power of two up to 8 (the kernel's unrolled variants)
  while (tpw < want && tpw < 8) tpw *= 2;
  GateUpArgs a{static_cast<const uint16_t*>(x), sx, static_cast<const uint4*>(w13),
               static_cast<const uint16_t*>(s13), sorted_ids, expert_ids, topk_ids, ids_is_i64,
               static_cast<int>(num_routes), static_cast<int>(topk),
               (topk & (topk - 1)) ? -1 : __builtin_ctzll(static_cast<uint64_t>(topk)), static_cast<int>(tpw),
               static_cast<int>(num_experts), static_cast<int>(n_inter), static_cast<int>(hidden), clamp_limit,
               static_cast<uint16_t*>(act)};
  (void)hipGetLastError();
  // Streaming variant at K = 4096: kTiles tile pairs per workgroup so that
  // about one workgroup per CU covers them; at 1 and 2 tokens 8 and 4 waves
  // split each pair's K (interleaved A/B against the split-K kernel: B=1
  // layer 12.1 -> 11.7 us, B=2 18.7 -> 16.8 us; at 4 tokens the 4 x 2 form
  // was 0.8 us slower than 4 x 1).
  const int64_t pairs = n_half * num_routes;
  if (hidden == kMaxHidden && pairs >= num_cus()) {
    const int tiles = pairs >= 8 * num_cus() ? 8 : pairs >= 4 * num_cus() ? 4 : pairs >= 2 * num_cus() ? 2 : 1;
    const dim3 gs(static_cast<unsigned>(num_routes), static_cast<unsigned>((n_half + tiles - 1) / tiles));
    hipStream_t st = static_cast<hipStream_t>(stream);
    // the fields the first loads need lead, as scalars (preloaded into SGPRs)
    const int one_token = self_align && num_routes == topk ? 1 : 0;
    auto go = [&](auto kernel, int waves) {
      hipLaunchKernelGGL(kernel, gs, dim3(64 * waves), 0, st, a.topk_ids, a.ids_i64, a.num_routes, a.w13, a.s13,
                         a.x, a.sx, a.n_inter, a.num_experts, one_token, a);
    };
    if (tiles == 8)
      self_align ? go(moe_w4a16_gate_up_stream_kernel<true, 8, 1>, 8) : go(moe_w4a16_gate_up_stream_kernel<false, 8, 1>, 8);
    else if (tiles == 4)
      self_align ? go(moe_w4a16_gate_up_stream_kernel<true, 4, 1>, 4) : go(moe_w4a16_gate_up_stream_kernel<false, 4, 1>, 4);
    else if (tiles == 2)
      self_align ? go(moe_w4a16_gate_up_stream_kernel<true, 2, 4>, 8) : go(moe_w4a16_gate_up_stream_kernel<false, 2, 4>, 8);
    else
      self_align ? go(moe_w4a16_gate_up_stream_kernel<true, 1, 8>, 8) : go(moe_w4a16_gate_up_stream_kernel<false, 1, 8>, 8);
    return static_cast<int>(hipGetLastError());
  }
  const dim3 grid(static_cast<unsigned>(num_routes), static_cast<unsigned>((n_half + tpw - 1) / tpw));
  if (self_align)
    hipLaunchKernelGGL(moe_w4a16_gate_up_kernel<true>, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(moe_w4a16_gate_up_kernel<false>, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), a);
  return static_cast<int>(hipGetLastError());
}

}  // namespace

extern "C" int glm53_moe_w4a16_gate_up(const void* x, int64_t sx, const void* w13, const void* s13,
                                       const int32_t* sorted_ids, const int32_t* expert_ids,
                                       int64_t num_routes, int64_t topk, int64_t num_experts,
                                       int64_t n_inter, int64_t hidden, float clamp_limit, void* act,
                                       void* stream) {
  return launch_gate_up(false, x, sx, w13, s13, sorted_ids, expert_ids, nullptr, 0, num_routes, topk, num_experts,
                        n_inter, hidden, clamp_limit, act, stream);
}

extern "C" int glm53_moe_w4a16_down(const void* act, const void* w2, const void* s2, const void* topk_ids,
                                    int ids_is_i64, int64_t sid_t, const float* topk_weights, int64_t sw_t,
                                    int64_t num_tokens, int64_t topk, int64_t num_experts, int64_t n_inter,
                                    int64_t hidden, void* out, int64_t so, void* stream) {
  if (!act || !w2 || !s2 || !topk_ids || !topk_weights || !out) return GLM53_ERR_NULL_POINTER;
  if (num_tokens < 1 || num_tokens > 65535 || topk < 1 || topk > kWaves || num_experts < 1 ||
      n_inter < kChunkK || n_inter % kChunkK || n_inter > kMaxInter || hidden < kTileN || hidden % kTileN ||
      sid_t < topk || sw_t < topk || so < hidden)
    return GLM53_ERR_BAD_SHAPE;
  if (!aligned16(act) || !aligned16(w2) || (reinterpret_cast<uintptr_t>(s2) & 7) || (reinterpret_cast<uintptr_t>(out) & 1))
    return GLM53_ERR_MISALIGNED;
  DownArgs a{static_cast<const uint16_t*>(act), static_cast<const uint4*>(w2), static_cast<const uint16_t*>(s2),
             topk_ids, ids_is_i64, sid_t, topk_weights, sw_t, static_cast<int>(topk),
             static_cast<int>(num_experts), static_cast<int>(n_inter), static_cast<int>(hidden),
             static_cast<uint16_t*>(out), so};
  (void)hipGetLastError();
  hipLaunchKernelGGL(moe_w4a16_down_kernel, dim3(static_cast<unsigned>(hidden / kTileN), static_cast<unsigned>(num_tokens)),
                     dim3(kThreads), 0, static_cast<hipStream_t>(stream), a.topk_ids, a.ids_i64, a.topk, a.sid_t,
                     a.w2, a.s2, a.act, a.n_inter, a.hidden, a);
  return static_cast<int>(hipGetLastError());
}

// Workspace of glm53_fused_moe_w4a16: the c2 activations.
namespace {
constexpr int64_t kAlignBytes = 256;
int64_t fused_ws_bytes(int64_t routes, int64_t n_inter) {
  return (routes * n_inter * 2 + kAlignBytes - 1) / kAlignBytes * kAlignBytes;
}
constexpr int64_t kFusedTopk = 8;
constexpr int64_t kFusedMaxTokens = 8;
}  // namespace

extern "C" int64_t glm53_fused_moe_w4a16_workspace_bytes(int64_t num_tokens, int64_t topk, int64_t n_inter) {
  if (num_tokens < 1 || topk < 1 || n_inter < 1) return 0;
  return fused_ws_bytes(num_tokens * topk, n_inter);
}

extern "C" int glm53_fused_moe_w4a16(const void* x, int64_t sx, const void* w13, const void* s13,
                                     const void* w2, const void* s2, const void* topk_ids, int ids_is_i64,
                                     const float* topk_weights, int64_t num_tokens, int64_t topk,
                                     int64_t num_experts, int64_t n_inter, int64_t hidden, float clamp_limit,
                                     void* workspace, int64_t workspace_bytes, void* out, int64_t so,
                                     void* stream) {
  if (!x || !w13 || !s13 || !w2 || !s2 || !topk_ids || !topk_weights || !out || !workspace)
    return GLM53_ERR_NULL_POINTER;
  if (num_tokens < 1 || num_tokens > kFusedMaxTokens || topk != kFusedTopk || num_experts != kAlignExperts)
    return GLM53_ERR_BAD_SHAPE;
  const int64_t routes = num_tokens * topk;
  if (workspace_bytes < fused_ws_bytes(routes, n_inter)) return GLM53_ERR_WORKSPACE;
  if (!aligned16(workspace)) return GLM53_ERR_MISALIGNED;
  // The gate/up kernel aligns the routes itself (the aligner's layout), so
  // the aligner's launch and its outputs' round trip through memory go away.
  int rc = launch_gate_up(true, x, sx, w13, s13, nullptr, nullptr, topk_ids, ids_is_i64, routes, topk, num_experts,
                          n_inter, hidden, clamp_limit, workspace, stream);
  if (rc) return rc;
  return glm53_moe_w4a16_down(workspace, w2, s2, topk_ids, ids_is_i64, topk, topk_weights, topk, num_tokens, topk,
                              num_experts, n_inter, hidden, out, so, stream);
}
