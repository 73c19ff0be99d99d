// Per-token symmetric INT8 latent writer for gfx950.
//
// Behaviour of kernels/titan_kv.py:7-21: for each slot row, s = max(max|x| /
// 127, 1e-12) in fp32, q = clamp(rint(x / s), -127, 127), and the 528-byte
// row [q(512 x int8) | s (fp32) | 12 zero bytes] goes to the cache at
// (slot / block) * stride_block + (slot % block) * stride_slot; slot < 0 is
// skipped, and so is a slot at or beyond the cache capacity (the reference
// leaves that case undefined).
//
// Layout: a wavefront handles 2 rows, both loaded before either is reduced.
// Lane i loads bf16 elements [8i, 8i+8) of a row as one 16-byte
// non-temporal load (the latents stream through once) and stores their 8
// int8 codes as one 8-byte store; lane 0 stores the 16-byte tail
// [s, 0, 0, 0].  Calls of at least kStreamRows rows store non-temporally
// too (bulk fills: 262144 rows over rotating sets 73.31 -> 71.39 us, 16384
// rows 6.35 -> 6.25 us); fewer rows -- a decode step's, a short prefill
// chunk's -- keep plain stores, which leave them in the caches for the
// attention that reads them next (2048 scattered rows 3.31 us plain, 3.77 us
// non-temporal).  max|x| is taken on the bf16 bit patterns (|x| = bits &
// 0x7fff orders like the values for finite inputs) and reduced across the
// wave with DPP and permlane swaps (no LDS traffic).
//
// Quotient: the reference rounds the IEEE quotient fl(x / s) to an integer.
// Instead of a full division per element the kernel takes y = fl(1 / s) once
// per row and per element q0 = fl(x * y), r = fma(-q0, s, x),
// q1 = fma(r, y, q0) (Markstein's correction step), then adds 1.5 * 2^23:
// that rounds q1 to the nearest integer with ties to even and leaves it, as
// two's complement, in the low byte of the sum's bit pattern.
// tests/native/quotient_check.c walks the whole input domain (every finite
// bf16 amax, every bf16 x with |x| <= amax: 1,065,369,600 pairs): the code
// equals int8(clamp(nearbyint(x / s), -127, 127)) for every pair, and
// q1 == fl(x / s) whenever |x / s| >= 1e-20 (below that intermediates
// underflow and both round to 0).  |x / s| <= 127 * (1 + 2^-23) on that
// domain, so the reference's clamp never changes a value.
#include "glm53_common.h"

namespace glm53 {
namespace {

constexpr int kLatent = 512;
constexpr int kWavesPerBlock = 4;
constexpr float kRoundMagic = 12582912.0f;  // 1.5 * 2^23
constexpr int64_t kStreamRows = 16384;      // calls from this many rows store non-temporally

__device__ __forceinline__ uint32_t quant_bits(float x, float s, float y) {
  float q0 = x * y;
  float r = __builtin_fmaf(-q0, s, x);
  float q1 = __builtin_fmaf(r, y, q0);
  return __float_as_uint(q1 + kRoundMagic);
}

// Four int8 codes (low bytes of a..d) packed into one dword.
__device__ __forceinline__ uint32_t pack4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  uint32_t lo = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);  // [a0, b0, 0, 0]
  uint32_t hi = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);  // [c0, d0, 0, 0]
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);       // [a0, b0, c0, d0]
}

__device__ __forceinline__ uint32_t absmax_bf16x2(uint32_t m, uint32_t w) {
  uint32_t a = w & 0x7fffu, b = (w >> 16) & 0x7fffu;
  m = m > a ? m : a;
  return m > b ? m : b;
}

// Scale s and its correctly rounded reciprocal from the bf16 bit pattern of
// max|x| (titan_kv.py:16).
__device__ __forceinline__ void row_scale(uint32_t amax_bits, float& s, float& y) {
  float amax = bf16_bits_to_f32(amax_bits);
  s = amax / 127.0f;
  s = s > 1.0e-12f ? s : 1.0e-12f;
  y = 1.0f / s;
}

__device__ __forceinline__ int64_t load_slot(const void* slots, int slots_i64, int64_t row) {
  return slots_i64 ? static_cast<const int64_t*>(slots)[row]
                   : static_cast<int64_t>(static_cast<const int32_t*>(slots)[row]);
}

// Fast path: x rows 16-byte aligned, destination rows 16-byte aligned.
// ROWS rows per wave are loaded before any is reduced, so each lane keeps
// ROWS independent 16-byte loads in flight.
// The arguments of the first loads (latents, slots) lead: the library is
// built to preload the leading 14 dwords of kernel arguments into SGPRs.
template <int ROWS, bool kStream>
__global__ __launch_bounds__(256) void store_int8_vec(const uint16_t* __restrict__ x, int64_t xs,
                                                      const void* __restrict__ slots, int64_t n,
                                                      int slots_i64, uint8_t* __restrict__ cache, int64_t cs0,
                                                      int64_t cs1, int64_t block, int64_t capacity) {
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave) * ROWS;
  // The rows' latents are requested before their slots and without waiting
  // for them (a row past n re-reads row n - 1, a skipped row is read and
  // dropped): behind each slot's scalar load the wave paid a memory round
  // trip per row before its latents were even requested.
  uint4 v[ROWS];
  int64_t slot[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) {
    const int64_t row = row0 + r < n ? row0 + r : n - 1;
    const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + row * xs) + lane);
    v[r] = make_uint4(t[0], t[1], t[2], t[3]);
  }
  // every slot load issued before any is waited for (clamped rows, masked after)
  if (slots_i64) {
#pragma unroll
    for (int r = 0; r < ROWS; r++) slot[r] = static_cast<const int64_t*>(slots)[row0 + r < n ? row0 + r : n - 1];
  } else {
#pragma unroll
    for (int r = 0; r < ROWS; r++) slot[r] = static_cast<const int32_t*>(slots)[row0 + r < n ? row0 + r : n - 1];
  }
#pragma unroll
  for (int r = 0; r < ROWS; r++)
    if (row0 + r >= n || slot[r] >= capacity) slot[r] = -1;
#pragma unroll
  for (int r = 0; r < ROWS; r++) {
    if (slot[r] < 0) continue;  // wave-uniform
    uint32_t m = absmax_bf16x2(0u, v[r].x);
    m = absmax_bf16x2(m, v[r].y);
    m = absmax_bf16x2(m, v[r].z);
    m = absmax_bf16x2(m, v[r].w);
    m = wave_max_u32(m);
    float s, y;
    row_scale(m, s, y);
    const uint32_t w[4] = {v[r].x, v[r].y, v[r].z, v[r].w};
    uint32_t b[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      b[2 * k] = quant_bits(__uint_as_float(w[k] << 16), s, y);
      b[2 * k + 1] = quant_bits(__uint_as_float(w[k] & 0xffff0000u), s, y);
    }
    uint8_t* dst = cache + (slot[r] / block) * cs0 + (slot[r] % block) * cs1;
    const u32x2 codes = {pack4(b[0], b[1], b[2], b[3]), pack4(b[4], b[5], b[6], b[7])};
    const u32x4 tail = {__float_as_uint(s), 0u, 0u, 0u};
    if (kStream) {
      __builtin_nontemporal_store(codes, reinterpret_cast<u32x2*>(dst) + lane);
      if (lane == 0) __builtin_nontemporal_store(tail, reinterpret_cast<u32x4*>(dst + kLatent));
    } else {
      reinterpret_cast<u32x2*>(dst)[lane] = codes;
      if (lane == 0) *reinterpret_cast<u32x4*>(dst + kLatent) = tail;
    }
  }
}

// Generic path for rows that are only 2-byte (x) / 1-byte (cache) aligned:
// the same arithmetic with element-wise loads and byte stores.
__global__ __launch_bounds__(256) void store_int8_any(const uint16_t* __restrict__ x, int64_t xs,
                                                      uint8_t* __restrict__ cache, int64_t cs0,
                                                      int64_t cs1, int64_t block, int64_t capacity,
                                                      const void* __restrict__ slots,
                                                      int slots_i64, int64_t n) {
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave;
  if (row >= n) return;
  const int64_t slot = load_slot(slots, slots_i64, row);
  if (slot < 0 || slot >= capacity) return;
  uint32_t e[8];
  uint32_t m = 0;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    e[k] = x[row * xs + lane * 8 + k];
    uint32_t a = e[k] & 0x7fffu;
    m = m > a ? m : a;
  }
  m = wave_max_u32(m);
  float s, y;
  row_scale(m, s, y);
  uint8_t* dst = cache + (slot / block) * cs0 + (slot % block) * cs1;
#pragma unroll
  for (int k = 0; k < 8; k++)
    dst[lane * 8 + k] = static_cast<uint8_t>(quant_bits(bf16_bits_to_f32(e[k]), s, y) & 0xffu);
  if (lane < 16) {
    const uint32_t sb = __float_as_uint(s);
    dst[kLatent + lane] = lane < 4 ? static_cast<uint8_t>(sb >> (8 * lane)) : 0;
  }
}

}  // namespace
}  // namespace glm53

using namespace glm53;

extern "C" int glm53_store_int8(const void* x, int64_t x_row_stride, void* cache,
                                int64_t cache_stride_block, int64_t cache_stride_slot,
                                int64_t block_size, int64_t capacity, const void* slots,
                                int slots_is_i64, int64_t n_slots, void* stream) {
  if (n_slots < 0 || block_size <= 0) return GLM53_ERR_BAD_SHAPE;
  if (n_slots == 0) return 0;
  if (!x || !cache || !slots) return GLM53_ERR_NULL_POINTER;
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  const uintptr_t xa = reinterpret_cast<uintptr_t>(x), ca = reinterpret_cast<uintptr_t>(cache);
  const bool aligned = (xa % 16 == 0) && (x_row_stride % 8 == 0) && (ca % 16 == 0) &&
                       (cache_stride_block % 16 == 0) && (cache_stride_slot % 16 == 0);
  const auto* xp = static_cast<const uint16_t*>(x);
  auto* cp = static_cast<uint8_t*>(cache);
  if (aligned) {
    constexpr int kRows = 2;   // measured best of 1/2/4/8 rows per wave on MI355X
    const int64_t rows_per_block = kWavesPerBlock * kRows;
    const int64_t grid = (n_slots + rows_per_block - 1) / rows_per_block;
    if (grid > 0x7fffffff) return GLM53_ERR_BAD_SHAPE;
    hipLaunchKernelGGL((n_slots >= kStreamRows ? store_int8_vec<kRows, true> : store_int8_vec<kRows, false>),
                       dim3(static_cast<unsigned>(grid)), dim3(256), 0, st, xp, x_row_stride, slots, n_slots,
                       slots_is_i64, cp, cache_stride_block, cache_stride_slot, block_size, capacity);
  } else {
    const int64_t grid = (n_slots + kWavesPerBlock - 1) / kWavesPerBlock;
    if (grid > 0x7fffffff) return GLM53_ERR_BAD_SHAPE;
    hipLaunchKernelGGL(store_int8_any, dim3(static_cast<unsigned>(grid)), dim3(256), 0, st, xp,
                       x_row_stride, cp, cache_stride_block, cache_stride_slot, block_size,
                       capacity, slots, slots_is_i64, n_slots);
  }
  return static_cast<int>(hipGetLastError());
}
