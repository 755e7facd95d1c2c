/*
 * oracle/paged_attention.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * CPU restatement of vflorence's decode-step attention path, used only by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the reference results
 * the tests compare against and as the timed CPU baseline.  Nothing in vflorence_amd/ links or calls it.
 *
 * The reference's arithmetic lives in the external package vllm-cpu-attn 0.1.0
 * (git 79b2eb02549b3e047bc80df51321bc7281f851c9, uv.lock:1091-1093), which is not
 * in /root/reference.  What is restated here is what its call sites require:
 *   - oracle_reshape_and_cache: vllm_cpu_attn.reshape_and_cache as called at
 *     vflorence/layers/attention.py:55-57 and vflorence/engine/model_runner.py:252-259,
 *     cache[slot / bs][h][slot % bs][:] = key[t][h][:]  (logical layout
 *     [num_blocks][H][bs][D], vflorence/engine/model_runner.py:66-77).
 *   - oracle_copy_blocks: ModelRunner._copy_blocks, vflorence/engine/model_runner.py:162-167
 *     (index_select of all sources, then index_copy_ into the destinations).
 *   - oracle_paged_attention: vllm_cpu_attn.attention_with_kv_cache as called at
 *     vflorence/layers/attention.py:61-72 (self) and :98-109 (cross): one query per
 *     sequence, softmax(scale * q K^T) V over the first seq_lens[r] tokens of the
 *     pages block_table[r] lists; fp32 accumulation, two-pass softmax.
 * Pinning: tests/test_oracle.py checks these against torch's scaled_dot_product_attention
 * on densely gathered tensors, closed forms (one token, constant keys), block-permutation
 * invariance, pure-Python brute force, and the copy-on-write known answer of
 * tests/test_engine.py:382-405 in the reference.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { OR_F32 = 0, OR_BF16 = 1, OR_F16 = 2 };

static inline float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  uint32_t u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else { /* subnormal: renormalise */
      exp = 127 - 15 + 1;
      while (!(man & 0x400)) {
        man <<= 1;
        exp--;
      }
      man &= 0x3ff;
      u = sign | (exp << 23) | (man << 13);
    }
  } else if (exp == 0x1f) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline float load_elem(const void *base, int64_t idx, int dtype) {
  if (dtype == OR_F32) return ((const float *)base)[idx];
  const uint16_t h = ((const uint16_t *)base)[idx];
  return dtype == OR_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

/* <q, row> and acc += p * row over one head_dim row, with the dtype switch outside
 * the loops so each loop vectorises (omp simd permits the reassociated sum). */
static float row_dot(const float *q, const void *base, int64_t off, int n, int dtype) {
  float s = 0.f;
  if (dtype == OR_F32) {
    const float *r = (const float *)base + off;
#pragma omp simd reduction(+ : s)
    for (int d = 0; d < n; ++d) s += q[d] * r[d];
  } else if (dtype == OR_BF16) {
    const uint16_t *r = (const uint16_t *)base + off;
#pragma omp simd reduction(+ : s)
    for (int d = 0; d < n; ++d) s += q[d] * bf16_to_f32(r[d]);
  } else {
    const uint16_t *r = (const uint16_t *)base + off;
    for (int d = 0; d < n; ++d) s += q[d] * f16_to_f32(r[d]);
  }
  return s;
}

static void row_axpy(float *acc, float p, const void *base, int64_t off, int n, int dtype) {
  if (dtype == OR_F32) {
    const float *r = (const float *)base + off;
#pragma omp simd
    for (int d = 0; d < n; ++d) acc[d] += p * r[d];
  } else if (dtype == OR_BF16) {
    const uint16_t *r = (const uint16_t *)base + off;
#pragma omp simd
    for (int d = 0; d < n; ++d) acc[d] += p * bf16_to_f32(r[d]);
  } else {
    const uint16_t *r = (const uint16_t *)base + off;
    for (int d = 0; d < n; ++d) acc[d] += p * f16_to_f32(r[d]);
  }
}

void oracle_reshape_and_cache(const void *key, const void *value, int64_t k_st, int64_t k_sh,
                              int64_t v_st, int64_t v_sh, void *k_cache, void *v_cache,
                              const int64_t *slots, int64_t num_tokens, int num_heads,
                              int head_dim, int block_size, int64_t num_blocks,
                              int elem_bytes) {
  const size_t row = (size_t)head_dim * elem_bytes;
  for (int64_t t = 0; t < num_tokens; ++t) {
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= num_blocks * block_size) continue;
    const int64_t blk = slot / block_size, off = slot % block_size;
    for (int h = 0; h < num_heads; ++h) {
      const int64_t dst = ((blk * num_heads + h) * block_size + off) * head_dim;
      memcpy((char *)k_cache + dst * elem_bytes,
             (const char *)key + (t * k_st + h * k_sh) * elem_bytes, row);
      memcpy((char *)v_cache + dst * elem_bytes,
             (const char *)value + (t * v_st + h * v_sh) * elem_bytes, row);
    }
  }
}

/* Returns 0, or -1 when the staging buffer cannot be allocated. */
int oracle_copy_blocks(void **caches, int num_caches, const int64_t *src, const int64_t *dst,
                       int64_t num_pairs, int64_t block_bytes, int64_t num_blocks) {
  char *tmp = (char *)malloc((size_t)(num_pairs > 0 ? num_pairs : 1) * block_bytes);
  if (!tmp) return -1;
  for (int c = 0; c < num_caches; ++c) {
    char *base = (char *)caches[c];
    for (int64_t p = 0; p < num_pairs; ++p) /* gather every source first */
      if (src[p] >= 0 && src[p] < num_blocks && dst[p] >= 0 && dst[p] < num_blocks)
        memcpy(tmp + p * block_bytes, base + src[p] * block_bytes, block_bytes);
    for (int64_t p = 0; p < num_pairs; ++p) /* then scatter */
      if (src[p] >= 0 && src[p] < num_blocks && dst[p] >= 0 && dst[p] < num_blocks)
        memcpy(base + dst[p] * block_bytes, tmp + p * block_bytes, block_bytes);
  }
  free(tmp);
  return 0;
}

/*
 * out: float32 [num_rows][H][D].  Rows with seq_lens <= 0 get zeros; lengths are
 * clamped to max_blocks * block_size (the table width); block ids outside
 * [0, num_blocks) contribute nothing.  Returns 0, or -1 on allocation failure.
 */
int oracle_paged_attention(const void *q, int64_t q_st, int64_t q_sh, const void *k_cache,
                           const void *v_cache, float *out, const int32_t *seq_lens,
                           const int32_t *block_table, int64_t bt_stride, int max_blocks,
                           int64_t num_rows, int num_heads, int head_dim, int block_size,
                           int64_t num_blocks, float scale, int dtype, int num_threads) {
  const int64_t pairs = num_rows * num_heads;
  int failed = 0;
#ifdef _OPENMP
  if (num_threads > 0) omp_set_num_threads(num_threads);
#pragma omp parallel reduction(| : failed)
#endif
  {
    const int64_t cap = (int64_t)max_blocks * block_size;
    float *scores = (float *)malloc((size_t)(cap > 0 ? cap : 1) * sizeof(float));
    unsigned char *ok = (unsigned char *)malloc((size_t)(cap > 0 ? cap : 1));
    float *qf = (float *)malloc((size_t)head_dim * sizeof(float));
    float *acc = (float *)malloc((size_t)head_dim * sizeof(float));
    if (!scores || !ok || !qf || !acc) failed = 1;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
    for (int64_t ph = 0; ph < pairs; ++ph) {
      if (failed) continue;
      const int64_t r = ph / num_heads;
      const int h = (int)(ph % num_heads);
      float *o = out + ph * head_dim;
      int64_t L = seq_lens[r];
      if (L > cap) L = cap;
      for (int d = 0; d < head_dim; ++d) o[d] = 0.f;
      if (L <= 0) continue;
      for (int d = 0; d < head_dim; ++d) qf[d] = load_elem(q, r * q_st + h * q_sh + d, dtype);
      const int32_t *row = block_table + r * bt_stride;
      float mx = -INFINITY;
      for (int64_t j = 0; j < L; ++j) {
        const int32_t blk = row[j / block_size];
        ok[j] = blk >= 0 && blk < num_blocks;
        if (!ok[j]) continue;
        const int64_t base = (((int64_t)blk * num_heads + h) * block_size + j % block_size) *
                             head_dim;
        scores[j] = row_dot(qf, k_cache, base, head_dim, dtype) * scale;
        if (scores[j] > mx) mx = scores[j];
      }
      if (mx == -INFINITY) continue;
      float sum = 0.f;
      for (int d = 0; d < head_dim; ++d) acc[d] = 0.f;
      for (int64_t j = 0; j < L; ++j) {
        if (!ok[j]) continue;
        const int32_t blk = row[j / block_size];
        const int64_t base = (((int64_t)blk * num_heads + h) * block_size + j % block_size) *
                             head_dim;
        const float p = expf(scores[j] - mx);
        sum += p;
        row_axpy(acc, p, v_cache, base, head_dim, dtype);
      }
      for (int d = 0; d < head_dim; ++d) o[d] = acc[d] / sum;
    }
    free(scores);
    free(ok);
    free(qf);
    free(acc);
  }
  return failed ? -1 : 0;
}
