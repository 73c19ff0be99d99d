/*
 * CPU oracle for the GLM-5.3 decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates the reference algorithms in
 * plain C so that tests/, __graft_entry__.smoke() and bench.py's CPU baseline
 * can check the HIP kernels.  Nothing in the product path links or calls it.
 *
 * Functions and the reference lines they follow (paths relative to the
 * reference checkout):
 *   oracle_store_int8      kernels/titan_kv.py:7-21   (per-token INT8 row writer)
 *   oracle_moe_align       benchmarks/moe_align.py:23-31 (stable counting sort,
 *                          the baseline the Triton aligner must equal,
 *                          kernels/titan_moe_align.py:12-46)
 *   oracle_moe_align_pairwise  benchmarks/moe_align.py:34-46 (pairwise form)
 *   oracle_sparse_mla      kernels/titan_mla.py:59-182 (tile loop), :245-255
 *                          (single pass), :330-354 (split partials), :403-429
 *                          (LSE merge)
 *   oracle_sparse_mla_f64  tests/verify_mla.py:79-84 (textbook softmax
 *                          attention), here over the dequantised rows in double
 *
 * Arithmetic follows IEEE-754 binary32 with round-to-nearest-even; build with
 * -ffp-contract=off and without -ffast-math so every rounding point is the
 * one written here.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ROW_BYTES 528
#define LATENT 512
#define N_EXPERTS 288

static inline float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* fp32 -> bf16, round to nearest even (the conversion `.to(tl.bfloat16)`). */
static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

static inline float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

/* ------------------------------------------------------------------------ */
/* store_int8: kernels/titan_kv.py:10-21                                     */
/* ------------------------------------------------------------------------ */

/* One 528-byte row from 512 bf16 latents: bytes [0,512) = int8 quantised
 * values, [512,516) = fp32 scale (little endian), [516,528) = 0. */
void oracle_quantize_row(const uint16_t* x, uint8_t* dst) {
  float amax = 0.0f;
  for (int d = 0; d < LATENT; d++) {            /* tl.max(tl.abs(x))         :16 */
    float a = fabsf(bf16_to_f32(x[d]));
    if (a > amax) amax = a;
  }
  float scale = amax / 127.0f;                  /* tl.maximum(amax/127, 1e-12) :16 */
  if (!(scale > 1.0e-12f)) scale = 1.0e-12f;
  for (int d = 0; d < LATENT; d++) {
    float q = nearbyintf(bf16_to_f32(x[d]) / scale);   /* nearbyint(x / scale) :17 */
    q = fminf(fmaxf(q, -127.0f), 127.0f);              /* clamp to +-127       :18 */
    dst[d] = (uint8_t)(int8_t)(int)q;
  }
  memcpy(dst + LATENT, &scale, 4);              /* [scale, 0, 0, 0] at byte 512 :21 */
  memset(dst + LATENT + 4, 0, ROW_BYTES - LATENT - 4);
}

/* x: bf16 rows with row stride x_stride (elements); cache: byte base with
 * strides cs0 (per block) and cs1 (per slot in a block), both in bytes;
 * slots: int64, a negative slot leaves the cache untouched (:11). */
void oracle_store_int8(const uint16_t* x, int64_t x_stride, uint8_t* cache,
                       int64_t cs0, int64_t cs1, int64_t block,
                       const int64_t* slots, int64_t n, int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static) if (nthreads != 1)
#endif
  for (int64_t r = 0; r < n; r++) {
    int64_t slot = slots[r];
    if (slot < 0) continue;
    uint8_t* dst = cache + (slot / block) * cs0 + (slot % block) * cs1;  /* :19 */
    oracle_quantize_row(x + r * x_stride, dst);
  }
}

/* ------------------------------------------------------------------------ */
/* MoE align: benchmarks/moe_align.py:23-46                                   */
/* ------------------------------------------------------------------------ */

/* Stable counting sort of flat route ids by expert, each expert padded to a
 * multiple of 8 with the value R; expert_ids lists the expert of every
 * 8-block, remaining entries -1; postpad = padded length.  Routes outside
 * [0, 288) are dropped.  sorted has R*8 entries, experts R entries. */
void oracle_moe_align(const int64_t* ids, int64_t R, int32_t* sorted,
                      int32_t* experts, int32_t* postpad) {
  int64_t out = 0, nb = 0;
  for (int64_t e = 0; e < N_EXPERTS; e++) {     /* for expert in range(288) :25 */
    int64_t members = 0;
    for (int64_t i = 0; i < R; i++)
      if (ids[i] == e) { sorted[out++] = (int32_t)i; members++; }
    int64_t padded = (members + 7) / 8 * 8;     /* :27 */
    for (int64_t k = members; k < padded; k++) sorted[out++] = (int32_t)R;
    for (int64_t b = 0; b < padded / 8; b++) experts[nb++] = (int32_t)e;
  }
  *postpad = (int32_t)out;                      /* :30 */
  for (int64_t k = out; k < R * 8; k++) sorted[k] = (int32_t)R;
  for (int64_t b = nb; b < R; b++) experts[b] = -1;
}

/* The CPU baseline's timing loop: oracle_moe_align `iters` times over the
 * same routes (one call through ctypes costs about as much as the work). */
void oracle_moe_align_repeat(const int64_t* ids, int64_t R, int32_t* sorted,
                             int32_t* experts, int32_t* postpad, int64_t iters) {
  for (int64_t it = 0; it < iters; it++) oracle_moe_align(ids, R, sorted, experts, postpad);
}

/* Independent pairwise formulation (rank = earlier routes with the same
 * expert, offset = padded sizes of smaller experts). */
void oracle_moe_align_pairwise(const int64_t* ids, int64_t R, int32_t* sorted,
                               int32_t* experts, int32_t* postpad) {
  int64_t* rank = (int64_t*)calloc((size_t)R, sizeof(int64_t));
  int64_t* count = (int64_t*)calloc((size_t)R, sizeof(int64_t));
  int64_t* offset = (int64_t*)calloc((size_t)R, sizeof(int64_t));
  for (int64_t j = 0; j < R; j++) {
    int valid_j = ids[j] >= 0 && ids[j] < N_EXPERTS;
    for (int64_t k = 0; k < R; k++) {
      int valid_k = ids[k] >= 0 && ids[k] < N_EXPERTS;
      if (valid_k && ids[k] == ids[j]) { count[j]++; if (k < j) rank[j]++; }
    }
    (void)valid_j;
  }
  int64_t total = 0;
  for (int64_t j = 0; j < R; j++) {
    for (int64_t k = 0; k < R; k++) {
      int valid_k = ids[k] >= 0 && ids[k] < N_EXPERTS;
      if (valid_k && rank[k] == 0 && ids[k] < ids[j]) offset[j] += (count[k] + 7) / 8 * 8;
    }
  }
  for (int64_t k = 0; k < R * 8; k++) sorted[k] = (int32_t)R;
  for (int64_t b = 0; b < R; b++) experts[b] = -1;
  for (int64_t j = 0; j < R; j++) {
    int valid = ids[j] >= 0 && ids[j] < N_EXPERTS;
    if (!valid) continue;
    sorted[offset[j] + rank[j]] = (int32_t)j;
    if (rank[j] == 0) {
      int64_t padded = (count[j] + 7) / 8 * 8;
      for (int64_t b = 0; b < padded / 8; b++) experts[offset[j] / 8 + b] = (int32_t)ids[j];
      total += padded;
    }
  }
  *postpad = (int32_t)total;
  free(rank); free(count); free(offset);
}

/* ------------------------------------------------------------------------ */
/* Sparse NoPE MLA: kernels/titan_mla.py                                      */
/* ------------------------------------------------------------------------ */

#define NEG_LARGE (-1.0e30f)
#define LOGE2_F ((float)0.6931471805599453)

/* One head, one contiguous range [start, end) of the top-k axis, processed in
 * tiles of block_n keys exactly as _sparse_mla_compute_tile (:117-180).
 * acc (512 floats) / *m / *l receive the running accumulators.
 * With groups > 1 the tiles are dealt round-robin (tile i -> stream i % groups)
 * to independent online-softmax streams that are combined at the end with
 * base-2 rescaling to the largest stream max m (acc = sum_g acc_g 2^(m_g - m),
 * l likewise, summed in stream order): the reduction structure of the HIP
 * kernel's wavefronts.  groups = 1 is the reference's single stream.
 * lazy > 0: a stream moves its reference max only when a tile's max exceeds
 * it by more than `lazy` (base-2 units), to that tile's max; p = 2^(s - m_ref)
 * can then reach 2^lazy.  lazy = 0 is the reference (:171-174). */
static void mla_stream(const float* qf, const uint8_t* kv, int64_t skv,
                       int64_t seq_kv, const int32_t* idx, int64_t start,
                       int64_t end, float sm_scale_log2, int64_t block_n,
                       int64_t groups, int64_t gsel, float lazy, float* acc,
                       float* m_out, float* l_out, float* qk, float* kscale,
                       int32_t* kid) {
  float e_max = NEG_LARGE, e_sum = 0.0f;
  for (int d = 0; d < LATENT; d++) acc[d] = 0.0f;
  int64_t tile = 0;
  for (int64_t s0 = start; s0 < end; s0 += block_n, tile++) {
    if (tile % groups != gsel) continue;
    float tile_max = NEG_LARGE;
    for (int64_t j = 0; j < block_n; j++) {
      int64_t pos = s0 + j;
      int32_t id = pos < end ? idx[pos] : -1;           /* mask_indice, other=-1 :119-127 */
      int valid = id >= 0 && id < seq_kv;               /* mask_kv :128 */
      kid[j] = valid ? id : -1;
      float s = 0.0f, sc = 0.0f;
      if (valid) {
        const int8_t* row = (const int8_t*)(kv + (int64_t)id * skv);
        for (int d = 0; d < LATENT; d++) s += qf[d] * (float)row[d];  /* tl.dot(q, k) :140 */
        memcpy(&sc, kv + (int64_t)id * skv + LATENT, 4);              /* scale at byte 512 :138-139 */
      }
      s *= sc;                                          /* qk *= kv_scale :156 */
      s *= sm_scale_log2;                               /* qk *= sm_scale*log2e :157 */
      if (!valid) s = NEG_LARGE;                        /* :158 */
      qk[j] = s;
      kscale[j] = sc;
      if (s > tile_max) tile_max = s;
    }
    float n_e_max = tile_max > e_max + lazy ? tile_max : e_max;  /* :171 */
    float re_scale = exp2f(e_max - n_e_max);              /* :172 */
    for (int d = 0; d < LATENT; d++) acc[d] *= re_scale;  /* :174 */
    float psum = 0.0f;
    for (int64_t j = 0; j < block_n; j++) {
      float p = kid[j] >= 0 ? exp2f(qk[j] - n_e_max) : 0.0f;   /* :173 */
      psum += p;
      if (kid[j] < 0) continue;
      float pw = round_bf16(p * kscale[j]);                     /* bf16(p * kv_scale) :176 */
      const int8_t* row = (const int8_t*)(kv + (int64_t)kid[j] * skv);
      for (int d = 0; d < LATENT; d++) acc[d] += pw * (float)row[d];
    }
    e_sum = e_sum * re_scale + psum;                      /* :179 */
    e_max = n_e_max;
  }
  *m_out = e_max;
  *l_out = e_sum;
}

static void mla_range(const uint16_t* qh, const uint8_t* kv, int64_t skv,
                      int64_t seq_kv, const int32_t* idx, int64_t start,
                      int64_t end, float sm_scale_log2, int64_t block_n,
                      int64_t groups, float lazy, float* acc, float* m_out,
                      float* l_out, float* qk, float* kscale, int32_t* kid) {
  float qf[LATENT];
  for (int d = 0; d < LATENT; d++) qf[d] = bf16_to_f32(qh[d]);
  if (groups <= 1) {
    mla_stream(qf, kv, skv, seq_kv, idx, start, end, sm_scale_log2, block_n, 1, 0, lazy, acc,
               m_out, l_out, qk, kscale, kid);
    return;
  }
  float* gacc = (float*)malloc((size_t)groups * LATENT * sizeof(float));
  float* gm = (float*)malloc((size_t)groups * sizeof(float));
  float* gl = (float*)malloc((size_t)groups * sizeof(float));
  for (int64_t gsel = 0; gsel < groups; gsel++)
    mla_stream(qf, kv, skv, seq_kv, idx, start, end, sm_scale_log2, block_n, groups, gsel, lazy,
               gacc + gsel * LATENT, gm + gsel, gl + gsel, qk, kscale, kid);
  /* flat merge: m = max m_g, acc = sum_g acc_g 2^(m_g - m), l likewise, g in order */
  float mm = NEG_LARGE;
  for (int64_t i = 0; i < groups; i++) mm = gm[i] > mm ? gm[i] : mm;
  float ll = 0.0f;
  float* out = (float*)calloc(LATENT, sizeof(float));
  for (int64_t i = 0; i < groups; i++) {
    float f = exp2f(gm[i] - mm);
    for (int d = 0; d < LATENT; d++) out[d] += gacc[i * LATENT + d] * f;
    ll += gl[i] * f;
  }
  memcpy(gacc, out, LATENT * sizeof(float));
  free(out);
  gm[0] = mm;
  gl[0] = ll;
  memcpy(acc, gacc, LATENT * sizeof(float));
  *m_out = gm[0];
  *l_out = gl[0];
  free(gacc); free(gm); free(gl);
}

/* q: bf16 [T, H, 512] with strides sq_t, sq_h (elements); kv: byte base of
 * rows with stride skv (bytes), seq_kv rows; idx: int32 [T, topk] with stride
 * si_t; out: bf16 [T, H, 512] with strides so_t, so_h.  n_splits >= 1 follows
 * the split-KV + merge path (:258-429) when > 1, the single pass (:185-255)
 * when 1.  block_n is the tile width of the online softmax; groups > 1 deals
 * the tiles of each split to that many streams and lazy > 0 delays max
 * updates (see mla_stream / mla_range). */
void oracle_sparse_mla(const uint16_t* q, int64_t sq_t, int64_t sq_h,
                       const uint8_t* kv, int64_t skv, int64_t seq_kv,
                       const int32_t* idx, int64_t si_t, int64_t T, int64_t H,
                       int64_t topk, float sm_scale_log2, int64_t n_splits,
                       int64_t block_n, int64_t groups, float lazy,
                       uint16_t* out, int64_t so_t, int64_t so_h,
                       int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for collapse(2) schedule(dynamic) if (nthreads != 1)
#endif
  for (int64_t t = 0; t < T; t++) {
    for (int64_t h = 0; h < H; h++) {
      float acc[LATENT], macc[LATENT];
      float* qk = (float*)malloc((size_t)block_n * sizeof(float));
      float* ks = (float*)malloc((size_t)block_n * sizeof(float));
      int32_t* kid = (int32_t*)malloc((size_t)block_n * sizeof(int32_t));
      const uint16_t* qh = q + t * sq_t + h * sq_h;
      const int32_t* it = idx + t * si_t;
      uint16_t* oh = out + t * so_t + h * so_h;
      if (n_splits <= 1) {
        float m, l;
        mla_range(qh, kv, skv, seq_kv, it, 0, topk, sm_scale_log2, block_n, groups, lazy, acc, &m, &l, qk, ks, kid);
        float ls = l > 0.0f ? l : 1.0f;                   /* :246 */
        for (int d = 0; d < LATENT; d++) oh[d] = f32_to_bf16(acc[d] / ls);
      } else {
        int64_t split_topk = (topk + n_splits - 1) / n_splits;   /* :301 */
        float g_max = NEG_LARGE, g_sum = 0.0f;                   /* merge state :392-394 */
        for (int d = 0; d < LATENT; d++) macc[d] = 0.0f;
        for (int64_t s = 0; s < n_splits; s++) {
          int64_t start = s * split_topk;
          int64_t end = start + split_topk < topk ? start + split_topk : topk;
          float m = NEG_LARGE, l = 0.0f;
          if (start < end) {
            mla_range(qh, kv, skv, seq_kv, it, start, end, sm_scale_log2, block_n, groups, lazy, acc, &m, &l, qk, ks, kid);
          } else {
            for (int d = 0; d < LATENT; d++) acc[d] = 0.0f;
          }
          float ls = l > 0.0f ? l : 1.0f;                        /* :334 */
          float lse = (m + log2f(l)) * LOGE2_F;                  /* :354 */
          float n_max = lse > g_max ? lse : g_max;               /* :414 */
          float old_scale = expf(g_max - n_max);                 /* :415 */
          float exp_logic = expf(lse - n_max);                   /* :416 */
          for (int d = 0; d < LATENT; d++)
            macc[d] = macc[d] * old_scale + exp_logic * (acc[d] / ls);   /* :417 */
          g_sum = g_sum * old_scale + exp_logic;                 /* :418 */
          g_max = n_max;
        }
        float gs = g_sum > 0.0f ? g_sum : 1.0f;                  /* :421 */
        for (int d = 0; d < LATENT; d++) oh[d] = f32_to_bf16(macc[d] / gs);
      }
      free(qk); free(ks); free(kid);
    }
  }
}

/* Textbook attention in double over the dequantised rows: out[t,h] =
 * sum_j softmax_j(sm_scale * q.k_j) k_j with k_j = int8_j * scale_j; rows
 * with an index outside [0, seq_kv) are excluded; no valid row gives 0. */
void oracle_sparse_mla_f64(const uint16_t* q, int64_t sq_t, int64_t sq_h,
                           const uint8_t* kv, int64_t skv, int64_t seq_kv,
                           const int32_t* idx, int64_t si_t, int64_t T,
                           int64_t H, int64_t topk, double sm_scale,
                           double* out, int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for collapse(2) schedule(dynamic) if (nthreads != 1)
#endif
  for (int64_t t = 0; t < T; t++) {
    for (int64_t h = 0; h < H; h++) {
      const uint16_t* qh = q + t * sq_t + h * sq_h;
      const int32_t* it = idx + t * si_t;
      double* oh = out + (t * H + h) * LATENT;
      double* logit = (double*)malloc((size_t)topk * sizeof(double));
      double mx = -INFINITY;
      for (int64_t j = 0; j < topk; j++) {
        int32_t id = it[j];
        if (id < 0 || id >= seq_kv) { logit[j] = -INFINITY; continue; }
        const int8_t* row = (const int8_t*)(kv + (int64_t)id * skv);
        float sc;
        memcpy(&sc, kv + (int64_t)id * skv + LATENT, 4);
        double s = 0.0;
        for (int d = 0; d < LATENT; d++) s += (double)bf16_to_f32(qh[d]) * ((double)row[d] * (double)sc);
        logit[j] = s * sm_scale;
        if (logit[j] > mx) mx = logit[j];
      }
      for (int d = 0; d < LATENT; d++) oh[d] = 0.0;
      if (mx == -INFINITY) { free(logit); continue; }
      double den = 0.0;
      for (int64_t j = 0; j < topk; j++) {
        if (logit[j] == -INFINITY) continue;
        double w = exp(logit[j] - mx);
        den += w;
        int32_t id = it[j];
        const int8_t* row = (const int8_t*)(kv + (int64_t)id * skv);
        float sc;
        memcpy(&sc, kv + (int64_t)id * skv + LATENT, 4);
        for (int d = 0; d < LATENT; d++) oh[d] += w * ((double)row[d] * (double)sc);
      }
      for (int d = 0; d < LATENT; d++) oh[d] /= den;
      free(logit);
    }
  }
}

/* Version tag so Python can check it loaded the intended build. */
int oracle_abi_version(void) { return 3; }
