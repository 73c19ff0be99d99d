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
//   * 4 wavefronts; wavefront w owns latent columns [128w, 128w + 128).
//   * Keys are processed in tiles of 32.  Lane (g = lane / 16, c = lane % 16)
//     loads 32 bytes of the wave's slice from keys c and 16 + c, so every
//     lane issues four independent 16-byte gathers per tile.
//   * S^T = K Q^T on v_mfma_f32_16x16x32_bf16: A = 16 keys x 32 latents
//     (the gathered int8 converted to bf16 in registers), B = Q^T, 4 K-steps
//     per wave; the four partial S^T tiles of the waves are summed through
//     LDS in a fixed order, so every wave holds the same full scores.
//   * The C layout of S^T gives lane (g, c) head c and keys {4g+i, 16+4g+i};
//     that is exactly the B operand P^T of O^T = V^T P^T, so the online
//     softmax runs per lane without any shuffle of P.
//   * V^T comes from the same gathered rows: each wave stores its bf16 slice
//     row-major in LDS and reads it back transposed with ds_read_b64_tr_b16
//     (two reads per 16x32 operand).  O^T accumulates in 8 MFMA tiles
//     (16 latents x 16 heads each) per wave.
#include "glm53_common.h"

namespace glm53 {
namespace {

constexpr int kLatent = 512;
constexpr int kHeads = 16;       // heads per workgroup (one MFMA M/N tile)
constexpr int kTile = 32;        // keys per tile
constexpr int kWaves = 4;        // latent slices of 128
constexpr int kSlice = kLatent / kWaves;
constexpr int kVStride = kSlice + 16;  // bf16 per LDS row: 288 bytes, rows 8 banks apart
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
  float* part;    // [T][S][Hp][512] fp32 (num_splits > 1)
  float* lse;     // [T][S][Hp]
  int heads_padded;
  uint16_t* out;
  int64_t so_t, so_h;
};

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

__global__ __launch_bounds__(256) void sparse_mla_kernel(const MlaArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t vbuf[kWaves][kTile][kVStride];
  __shared__ float red[2][kWaves][8][64];

  const int split = blockIdx.x;
  const int t = blockIdx.y;
  const int hg = blockIdx.z;
  const int w = uniform(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int start = split * a.split_len;
  const int end = min(start + a.split_len, a.topk);
  const int head = hg * kHeads + c;
  const bool head_ok = head < a.num_heads;
  const int32_t* idx_t = a.idx + t * a.si_t;

  // Q^T fragment (B operand of S^T = K Q^T): head c, latents
  // [128w + 32g, +32) -> four K-steps of 8.
  bf16x8 qf[4];
  {
    uint4 z = make_uint4(0, 0, 0, 0);
    uint4 q0 = z, q1 = z, q2 = z, q3 = z;
    if (head_ok) {
      const uint4* qp = reinterpret_cast<const uint4*>(a.q + t * a.sq_t + head * a.sq_h +
                                                       kSlice * w + 32 * g);
      q0 = qp[0]; q1 = qp[1]; q2 = qp[2]; q3 = qp[3];
    }
    qf[0] = __builtin_bit_cast(bf16x8, q0);
    qf[1] = __builtin_bit_cast(bf16x8, q1);
    qf[2] = __builtin_bit_cast(bf16x8, q2);
    qf[3] = __builtin_bit_cast(bf16x8, q3);
  }

  f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegLarge, l_run = 0.f;

  int buf = 0;
  for (int k0 = start; k0 < end; k0 += kTile, buf ^= 1) {
    // Indices of the tile: lane l holds key (l & 31).
    const int pos = k0 + (lane & 31);
    int id = pos < end ? idx_t[pos] : -1;
    if (id < 0 || static_cast<int64_t>(id) >= a.seq_kv) id = -1;

    // Gather: keys c and 16 + c, bytes [128w + 32g, +32).
    uint4 kd[2][2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int kid = __shfl(id, 16 * u + c, 64);
      kd[u][0] = make_uint4(0, 0, 0, 0);
      kd[u][1] = make_uint4(0, 0, 0, 0);
      if (kid >= 0) {
        const uint4* rp = reinterpret_cast<const uint4*>(a.kv + static_cast<int64_t>(kid) * a.skv +
                                                         kSlice * w + 32 * g);
        kd[u][0] = rp[0];
        kd[u][1] = rp[1];
      }
    }
    // Scales of the keys this lane scores: 16u + 4g + i.
    float sc[8];
    int kvalid = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int key = 16 * (j >> 2) + 4 * g + (j & 3);
      const int kid = __shfl(id, key, 64);
      sc[j] = 0.f;
      if (kid >= 0) {
        sc[j] = *reinterpret_cast<const float*>(a.kv + static_cast<int64_t>(kid) * a.skv + kLatent);
        kvalid |= 1 << j;
      }
    }

    // bf16 K fragments; partial S^T over this wave's slice.
    f32x4 s_part[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
      bf16x8 k01, k23, k45, k67;
      i8x16_to_bf16(kd[u][0], k01, k23);
      i8x16_to_bf16(kd[u][1], k45, k67);
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k01, qf[0], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k23, qf[1], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k45, qf[2], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k67, qf[3], s, 0, 0, 0);
      s_part[u] = s;
      // V slice for the PV product: row 16u + c, latents [32g, +32) of the slice.
      uint4* vp = reinterpret_cast<uint4*>(&vbuf[w][16 * u + c][32 * g]);
      vp[0] = __builtin_bit_cast(uint4, k01);
      vp[1] = __builtin_bit_cast(uint4, k23);
      vp[2] = __builtin_bit_cast(uint4, k45);
      vp[3] = __builtin_bit_cast(uint4, k67);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      red[buf][w][i][lane] = s_part[0][i];
      red[buf][w][4 + i][lane] = s_part[1][i];
    }
    __syncthreads();

    // Full scores (fixed summation order over the four slices).
    float s[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      float v = red[buf][0][j][lane];
      v += red[buf][1][j][lane];
      v += red[buf][2][j][lane];
      v += red[buf][3][j][lane];
      v *= sc[j];
      v *= a.scale_log2;
      s[j] = (kvalid >> j) & 1 ? v : kNegLarge;
    }
    float mx = s[0];
#pragma unroll
    for (int j = 1; j < 8; j++) mx = fmaxf(mx, s[j]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = exp2f(m_run - m_new);
    float p[8];
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      p[j] = (kvalid >> j) & 1 ? exp2f(s[j] - m_new) : 0.f;
      psum += p[j];
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;

    // P^T operand: k-slot 8g + j <-> key 16(j/4) + 4g + (j%4).
    uint4 pw = make_uint4(pack_bf16x2(p[0] * sc[0], p[1] * sc[1]), pack_bf16x2(p[2] * sc[2], p[3] * sc[3]),
                          pack_bf16x2(p[4] * sc[4], p[5] * sc[5]), pack_bf16x2(p[6] * sc[6], p[7] * sc[7]));
    const bf16x8 pb = __builtin_bit_cast(bf16x8, pw);

    // O^T += V^T P^T for the 8 latent tiles of this wave.
    // ds_read_b64_tr_b16: in each 16-lane group, lane 4r + q addresses row r,
    // columns [4q, 4q + 4); lane c receives column c of the 4 rows.
    const int tr_row = 4 * g + (c >> 2);
    const int tr_col = 4 * (c & 3);
#pragma unroll
    for (int dt = 0; dt < 8; dt++) {
      const i16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          GLM53_LDS(i16x4, &vbuf[w][tr_row][16 * dt + tr_col]));
      const i16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          GLM53_LDS(i16x4, &vbuf[w][16 + tr_row][16 * dt + tr_col]));
      const i32x2 v0i = __builtin_bit_cast(i32x2, v0);
      const i32x2 v1i = __builtin_bit_cast(i32x2, v1);
      const uint4 vv = make_uint4(v0i[0], v0i[1], v1i[0], v1i[1]);
      f32x4 o = acc[dt];
      o[0] *= alpha; o[1] *= alpha; o[2] *= alpha; o[3] *= alpha;
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vv), pb, o, 0, 0, 0);
    }
  }

  if (!head_ok) return;
  const float l_safe = l_run > 0.f ? l_run : 1.f;
  if (a.num_splits == 1) {
    uint16_t* op = a.out + t * a.so_t + head * a.so_h + kSlice * w + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 8; dt++) {
      uint2 o;
      o.x = pack_bf16x2(acc[dt][0] / l_safe, acc[dt][1] / l_safe);
      o.y = pack_bf16x2(acc[dt][2] / l_safe, acc[dt][3] / l_safe);
      *reinterpret_cast<uint2*>(op + 16 * dt) = o;
    }
  } else {
    const int64_t row = (static_cast<int64_t>(t) * a.num_splits + split) * a.heads_padded + head;
    float* pp = a.part + row * kLatent + kSlice * w + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 8; dt++) {
      float4 o = make_float4(acc[dt][0] / l_safe, acc[dt][1] / l_safe, acc[dt][2] / l_safe,
                             acc[dt][3] / l_safe);
      *reinterpret_cast<float4*>(pp + 16 * dt) = o;
    }
    if (w == 0 && g == 0) a.lse[row] = (m_run + log2f(l_run)) * kLn2;
  }
}

// N-way LSE merge (kernels/titan_mla.py:403-429): one workgroup per (t, h),
// 128 threads x 4 latents.
__global__ __launch_bounds__(128) void sparse_mla_merge_kernel(const float* __restrict__ part,
                                                               const float* __restrict__ lse,
                                                               int num_splits, int heads_padded,
                                                               int num_heads,
                                                               uint16_t* __restrict__ out,
                                                               int64_t so_t, int64_t so_h) {
  const int t = blockIdx.x / num_heads;
  const int h = blockIdx.x % num_heads;
  const int d = threadIdx.x * 4;
  float e_max = kNegLarge, e_sum = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s = 0; s < num_splits; s++) {
    const int64_t row = (static_cast<int64_t>(t) * num_splits + s) * heads_padded + h;
    const float tl = lse[row];
    const float4 v = *reinterpret_cast<const float4*>(part + row * kLatent + d);
    const float n_max = fmaxf(tl, e_max);
    const float old_scale = expf(e_max - n_max);
    const float e = expf(tl - n_max);
    acc.x = acc.x * old_scale + e * v.x;
    acc.y = acc.y * old_scale + e * v.y;
    acc.z = acc.z * old_scale + e * v.z;
    acc.w = acc.w * old_scale + e * v.w;
    e_sum = e_sum * old_scale + e;
    e_max = n_max;
  }
  const float es = e_sum > 0.f ? e_sum : 1.f;
  uint2 o;
  o.x = pack_bf16x2(acc.x / es, acc.y / es);
  o.y = pack_bf16x2(acc.z / es, acc.w / es);
  *reinterpret_cast<uint2*>(out + t * so_t + h * so_h + d) = o;
}

}  // namespace
}  // namespace glm53

using namespace glm53;

extern "C" int64_t glm53_sparse_mla_workspace_bytes(int64_t num_tokens, int64_t num_heads,
                                                    int64_t num_splits) {
  if (num_tokens < 0 || num_heads < 1 || num_splits < 1) return -1;
  if (num_splits == 1) return 0;
  const int64_t hp = (num_heads + kHeads - 1) / kHeads * kHeads;
  const int64_t rows = num_tokens * num_splits * hp;
  return rows * kLatent * 4 + rows * 4;
}

extern "C" int glm53_sparse_mla(const void* q, int64_t sq_t, int64_t sq_h, const void* kv,
                                int64_t skv_t, int64_t seq_kv, const int32_t* indices,
                                int64_t si_t, int64_t num_tokens, int64_t num_heads, int64_t topk,
                                double sm_scale, int64_t num_splits, void* workspace,
                                int64_t workspace_bytes, void* out, int64_t so_t, int64_t so_h,
                                void* stream) {
  if (num_tokens < 0 || num_heads < 1 || topk < 0 || num_splits < 1 || seq_kv < 0)
    return GLM53_ERR_BAD_SHAPE;
  if (num_tokens == 0) return 0;
  if (!q || !out || (!kv && seq_kv > 0) || (!indices && topk > 0)) return GLM53_ERR_NULL_POINTER;
  if (topk > 0x7fffffff || num_tokens > 0x7fffffff || num_splits > 65535 ||
      (num_heads + kHeads - 1) / kHeads > 65535)
    return GLM53_ERR_BAD_SHAPE;
  if (reinterpret_cast<uintptr_t>(q) % 16 || sq_t % 8 || sq_h % 8 ||
      reinterpret_cast<uintptr_t>(kv) % 16 || skv_t % 16 || reinterpret_cast<uintptr_t>(out) % 8 ||
      so_t % 4 || so_h % 4)
    return GLM53_ERR_MISALIGNED;
  const int64_t need = glm53_sparse_mla_workspace_bytes(num_tokens, num_heads, num_splits);
  if (num_splits > 1 && (!workspace || workspace_bytes < need)) return GLM53_ERR_WORKSPACE;

  MlaArgs a;
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
  const int64_t rows = num_tokens * num_splits * a.heads_padded;
  a.part = num_splits > 1 ? static_cast<float*>(workspace) : nullptr;
  a.lse = num_splits > 1 ? static_cast<float*>(workspace) + rows * kLatent : nullptr;
  a.out = static_cast<uint16_t*>(out);
  a.so_t = so_t;
  a.so_h = so_h;

  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  const dim3 grid(static_cast<unsigned>(num_splits), static_cast<unsigned>(num_tokens),
                  static_cast<unsigned>(a.heads_padded / kHeads));
  hipLaunchKernelGGL(sparse_mla_kernel, grid, dim3(256), 0, st, a);
  if (num_splits > 1) {
    hipLaunchKernelGGL(sparse_mla_merge_kernel, dim3(static_cast<unsigned>(num_tokens * num_heads)),
                       dim3(128), 0, st, a.part, a.lse, a.num_splits, a.heads_padded, a.num_heads,
                       a.out, so_t, so_h);
  }
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
    default: return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "unknown error";
  }
}
