/*
 * CPU oracle for the paged-KV hot path -- TEST INFRASTRUCTURE ONLY (see
 * oxide_oracle.h).  Plain C restatement of the reference semantics; each
 * function cites the reference lines it follows.  Pinning, per function:
 *   half/float conversions   numpy float16 and torch bfloat16 casts, all
 *                            special values (tests/test_oracle.py)
 *   compute_slot_mapping     the reference's known answers,
 *                            kv_cache_manager.rs:254-322 (tests/golden)
 *   build_decode_metadata    the reference's known answers, metadata.rs:82-161
 *   pad_block_table          closed form (rows copied, tail zero) on ragged rows
 *   reshape_and_cache        the reference's GPU known answer,
 *                            attention/mod.rs:161-230, plus numpy fancy-index
 *                            scatter on random inputs and the -1 invariant
 *   copy_blocks / gather     numpy fancy-index copy; src == dst idempotence
 *   paged_decode_attention   numpy fp64 softmax(QK^T)V over the gathered
 *                            contiguous K/V; closed forms (constant V, L = 1,
 *                            q = 0 -> mean V, one-hot q against orthogonal keys);
 *                            invariance under block placement; window >= L
 *   prefill_attention        numpy fp64 masked softmax over dense score
 *                            matrices; every query row equals a decode-oracle
 *                            call over its causal prefix; Lq = 1 equals the
 *                            decode oracle; the FlashAttention 2 bottom-right
 *                            mask on a hand-worked Lq = 2, Lk = 5 case; paged
 *                            equals contiguous; rows with no keys give zeros
 *   rope_cos_sin_cache       numpy float32 restatement of the formula; the
 *                            reference's own tests (position 0 row = [1.., 0..],
 *                            shape, base changes the cache)
 *   qk_norm_rope_and_cache   numpy fp64 RMSNorm + complex-multiplication RoPE
 *                            with the same rounding points; position 0 is the
 *                            identity after the norm (the reference's test);
 *                            constant rows normalise to +-1; the rotation keeps
 *                            each (x1_i, x2_i) pair's length; v copied bitwise
 *   xxh64                    python-xxhash digests and the spec's empty-input
 *                            vector
 */
#include "oxide_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- formats */

float oracle_half_to_float(uint16_t h, int dtype) {
  uint32_t bits;
  if (dtype == 1) {
    bits = (uint32_t)h << 16;
  } else {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    if (exp == 0x1f) {
      bits = sign | 0x7f800000u | (mant << 13);
    } else if (exp != 0) {
      bits = sign | ((exp + 112u) << 23) | (mant << 13);
    } else if (mant == 0) {
      bits = sign;
    } else {
      /* subnormal: value = mant * 2^-24; normalise. */
      int e = 113;
      while ((mant & 0x400u) == 0) {
        mant <<= 1;
        --e;
      }
      bits = sign | ((uint32_t)e << 23) | ((mant & 0x3ffu) << 13);
    }
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t oracle_float_to_half(float f, int dtype) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if (dtype == 1) {
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  }
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu)); /* NaN */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520: inf */
  if (a >= 0x38800000u) {
    /* normal f16: rebias exponent, round 13 dropped bits to nearest even. */
    const uint32_t r = a - 0x38000000u;
    return (uint16_t)(sign | ((r + 0xfffu + ((r >> 13) & 1u)) >> 13));
  }
  if (a < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to zero */
  /* subnormal f16: value / 2^-24, rounded to nearest even. */
  const uint32_t e = a >> 23;
  const uint32_t m = (a & 0x7fffffu) | 0x800000u;
  const uint32_t shift = 126u - e; /* 14..24 bits dropped */
  const uint32_t q = m >> shift;
  const uint32_t rem = m & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1u);
  uint32_t out = q;
  if (rem > half || (rem == half && (q & 1u))) ++out;
  return (uint16_t)(sign | out);
}

/* ------------------------------------------------------------ host logic */

/* kv_cache_manager.rs:115-135: slot = table[(off+i)/bs]*bs + (off+i)%bs, or -1
 * past the end of the table. */
void oracle_compute_slot_mapping(const int64_t* block_table, int64_t table_len,
                                 int64_t block_size, int64_t token_offset, int64_t num_tokens,
                                 int64_t* slot_mapping) {
  for (int64_t i = 0; i < num_tokens; ++i) {
    const int64_t abs_idx = token_offset + i;
    const int64_t block_idx = abs_idx / block_size;
    const int64_t intra = abs_idx % block_size;
    slot_mapping[i] = block_idx < table_len ? block_table[block_idx] * block_size + intra : -1;
  }
}

/* metadata.rs:20-47. */
int64_t oracle_build_decode_metadata(const uint32_t* context_lens, int64_t batch,
                                     uint32_t* cu_seqlens_q, uint32_t* cu_seqlens_k) {
  int64_t max_k = 0;
  cu_seqlens_q[0] = 0;
  cu_seqlens_k[0] = 0;
  for (int64_t i = 0; i < batch; ++i) {
    cu_seqlens_q[i + 1] = cu_seqlens_q[i] + 1u;
    cu_seqlens_k[i + 1] = cu_seqlens_k[i] + context_lens[i];
    if ((int64_t)context_lens[i] > max_k) max_k = context_lens[i];
  }
  return max_k;
}

/* flash_attn.rs:74-86. */
int64_t oracle_pad_block_table(const int32_t* flat, const int64_t* row_lens, int64_t batch,
                               int32_t* out) {
  int64_t max_len = 0;
  for (int64_t b = 0; b < batch; ++b)
    if (row_lens[b] > max_len) max_len = row_lens[b];
  int64_t src = 0;
  for (int64_t b = 0; b < batch; ++b) {
    for (int64_t i = 0; i < max_len; ++i) out[b * max_len + i] = i < row_lens[b] ? flat[src + i] : 0;
    src += row_lens[b];
  }
  return max_len;
}

/* ---------------------------------------------------------- cache copies */

/* reshape_and_cache.cu:6-28: for each token, row t of key/value -> row slot. */
void oracle_reshape_and_cache(const void* key, const void* value, void* key_cache,
                              void* value_cache, const int64_t* slot_mapping, int64_t num_tokens,
                              int64_t num_kv_heads, int64_t head_dim, int esize) {
  const size_t row = (size_t)(num_kv_heads * head_dim) * (size_t)esize;
  for (int64_t t = 0; t < num_tokens; ++t) {
    const int64_t slot = slot_mapping[t];
    if (slot == -1) continue;
    memcpy((char*)key_cache + (size_t)slot * row, (const char*)key + (size_t)t * row, row);
    memcpy((char*)value_cache + (size_t)slot * row, (const char*)value + (size_t)t * row, row);
  }
}

/* copy_blocks.cu:8-28: cache[dst*S + e] = cache[src*S + e] for K and V. */
void oracle_copy_blocks(void* key_cache, void* value_cache, const int64_t* block_mapping,
                        int64_t num_pairs, int64_t block_stride, int esize) {
  const size_t blk = (size_t)block_stride * (size_t)esize;
  for (int64_t p = 0; p < num_pairs; ++p) {
    const int64_t src = block_mapping[2 * p], dst = block_mapping[2 * p + 1];
    memmove((char*)key_cache + (size_t)dst * blk, (const char*)key_cache + (size_t)src * blk, blk);
    memmove((char*)value_cache + (size_t)dst * blk, (const char*)value_cache + (size_t)src * blk,
            blk);
  }
}

void oracle_gather_blocks(void* key_dst, void* value_dst, const void* key_cache,
                          const void* value_cache, const int32_t* block_ids, int64_t num_blocks,
                          int64_t block_stride, int esize) {
  const size_t blk = (size_t)block_stride * (size_t)esize;
  for (int64_t i = 0; i < num_blocks; ++i) {
    memcpy((char*)key_dst + (size_t)i * blk, (const char*)key_cache + (size_t)block_ids[i] * blk,
           blk);
    if (value_dst)
      memcpy((char*)value_dst + (size_t)i * blk,
             (const char*)value_cache + (size_t)block_ids[i] * blk, blk);
  }
}

/* -------------------------------------------------------------- attention */

void oracle_paged_decode_attention(float* out, const uint16_t* q, const uint16_t* k_cache,
                                   const uint16_t* v_cache, const uint32_t* cu_seqlens_k,
                                   const int32_t* block_table, int64_t max_blocks, int64_t batch,
                                   int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                   int64_t block_size, int32_t window_left, float softmax_scale,
                                   int dtype, int use_f64, int threads) {
  const int64_t group = num_heads / num_kv_heads;
  const int64_t row_stride = num_kv_heads * head_dim;
  const int64_t units = batch * num_kv_heads;
  const int nthreads = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (int64_t u = 0; u < units; ++u) {
    const int64_t b = u / num_kv_heads;
    const int64_t kh = u % num_kv_heads;
    const int64_t L = (int64_t)cu_seqlens_k[b + 1] - (int64_t)cu_seqlens_k[b];
    const int64_t lo = (window_left < 0) ? 0 : (L - 1 - window_left > 0 ? L - 1 - window_left : 0);
    const int64_t n = L > lo ? L - lo : 0;
    double* sc = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
    float* qf = (float*)malloc(sizeof(float) * (size_t)head_dim);
    double* acc = (double*)malloc(sizeof(double) * (size_t)head_dim);
    for (int64_t g = 0; g < group; ++g) {
      const int64_t h = kh * group + g;
      float* o = out + (b * num_heads + h) * head_dim;
      if (n == 0) {
        for (int64_t d = 0; d < head_dim; ++d) o[d] = 0.f;
        continue;
      }
      for (int64_t d = 0; d < head_dim; ++d)
        qf[d] = oracle_half_to_float(q[(b * num_heads + h) * head_dim + d], dtype);
      /* scores */
      double mx = -INFINITY;
      for (int64_t i = 0; i < n; ++i) {
        const int64_t j = lo + i;
        const int64_t row = (int64_t)block_table[b * max_blocks + j / block_size] * block_size +
                            j % block_size;
        const uint16_t* kr = k_cache + row * row_stride + kh * head_dim;
        double s;
        if (use_f64) {
          double dot = 0.0;
          for (int64_t d = 0; d < head_dim; ++d)
            dot += (double)qf[d] * (double)oracle_half_to_float(kr[d], dtype);
          s = dot * (double)softmax_scale;
        } else {
          float dot = 0.f;
          for (int64_t d = 0; d < head_dim; ++d) dot += qf[d] * oracle_half_to_float(kr[d], dtype);
          s = (double)(dot * softmax_scale);
        }
        sc[i] = s;
        if (s > mx) mx = s;
      }
      /* probabilities and weighted V */
      for (int64_t d = 0; d < head_dim; ++d) acc[d] = 0.0;
      if (use_f64) {
        double l = 0.0;
        for (int64_t i = 0; i < n; ++i) {
          const int64_t j = lo + i;
          const int64_t row = (int64_t)block_table[b * max_blocks + j / block_size] * block_size +
                              j % block_size;
          const uint16_t* vr = v_cache + row * row_stride + kh * head_dim;
          const double p = exp(sc[i] - mx);
          l += p;
          for (int64_t d = 0; d < head_dim; ++d) acc[d] += p * (double)oracle_half_to_float(vr[d], dtype);
        }
        for (int64_t d = 0; d < head_dim; ++d) o[d] = (float)(acc[d] / l);
      } else {
        float l = 0.f;
        float* accf = (float*)acc; /* reuse storage: head_dim floats fit in head_dim doubles */
        for (int64_t d = 0; d < head_dim; ++d) accf[d] = 0.f;
        for (int64_t i = 0; i < n; ++i) {
          const int64_t j = lo + i;
          const int64_t row = (int64_t)block_table[b * max_blocks + j / block_size] * block_size +
                              j % block_size;
          const uint16_t* vr = v_cache + row * row_stride + kh * head_dim;
          const float p = expf((float)sc[i] - (float)mx);
          l += p;
          for (int64_t d = 0; d < head_dim; ++d) accf[d] += p * oracle_half_to_float(vr[d], dtype);
        }
        for (int64_t d = 0; d < head_dim; ++d) o[d] = accf[d] / l;
      }
    }
    free(sc);
    free(qf);
    free(acc);
  }
}

/* Prefill attention: one query row of one head, keys [lo, hi] of sequence b.
 * Follows attention/flash_attn.rs:15-37 (flash_attn_varlen, causal) and
 * :52-67 (flash_attn_varlen_paged_windowed) with the FlashAttention 2 mask. */
static int64_t prefill_key_row(const int32_t* block_table, int64_t max_blocks, int64_t block_size,
                               const uint32_t* cu_seqlens_k, int64_t b, int64_t j) {
  if (block_table == NULL) return (int64_t)cu_seqlens_k[b] + j;
  return (int64_t)block_table[b * max_blocks + j / block_size] * block_size + j % block_size;
}

void oracle_prefill_attention(float* out, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const uint32_t* cu_seqlens_q, const uint32_t* cu_seqlens_k,
                              const int32_t* block_table, int64_t max_blocks, int64_t batch,
                              int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                              int64_t block_size, int32_t window_left, float softmax_scale,
                              int dtype, int use_f64, int threads) {
  const int64_t group = num_heads / num_kv_heads;
  const int64_t row_stride = num_kv_heads * head_dim;
  const int64_t total_q = (int64_t)cu_seqlens_q[batch];
  const int nthreads = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel num_threads(nthreads)
  {
    int64_t cap = 0;
    double* sc = NULL;
    float* qf = (float*)malloc(sizeof(float) * (size_t)head_dim);
    double* acc = (double*)malloc(sizeof(double) * (size_t)head_dim);
    float* accf = (float*)malloc(sizeof(float) * (size_t)head_dim);
#pragma omp for schedule(dynamic, 4)
    for (int64_t tq = 0; tq < total_q * num_heads; ++tq) {
      const int64_t t = tq / num_heads, h = tq % num_heads, kh = h / group;
      int64_t b = 0;
      while (b + 1 < batch && (int64_t)cu_seqlens_q[b + 1] <= t) ++b;
      const int64_t Lq = (int64_t)cu_seqlens_q[b + 1] - (int64_t)cu_seqlens_q[b];
      const int64_t Lk = (int64_t)cu_seqlens_k[b + 1] - (int64_t)cu_seqlens_k[b];
      const int64_t i = t - (int64_t)cu_seqlens_q[b];
      int64_t hi = i + Lk - Lq;
      if (hi > Lk - 1) hi = Lk - 1;
      int64_t lo = window_left < 0 ? 0 : i + Lk - Lq - window_left;
      if (lo < 0) lo = 0;
      const int64_t n = hi >= lo ? hi - lo + 1 : 0;
      float* o = out + tq * head_dim;
      if (n == 0) {
        for (int64_t d = 0; d < head_dim; ++d) o[d] = 0.f;
        continue;
      }
      if (n > cap) {
        free(sc);
        cap = n;
        sc = (double*)malloc(sizeof(double) * (size_t)cap);
      }
      for (int64_t d = 0; d < head_dim; ++d) qf[d] = oracle_half_to_float(q[tq * head_dim + d], dtype);
      double mx = -INFINITY;
      for (int64_t x = 0; x < n; ++x) {
        const uint16_t* kr = k + prefill_key_row(block_table, max_blocks, block_size, cu_seqlens_k, b,
                                                 lo + x) * row_stride + kh * head_dim;
        double s;
        if (use_f64) {
          double dot = 0.0;
          for (int64_t d = 0; d < head_dim; ++d) dot += (double)qf[d] * (double)oracle_half_to_float(kr[d], dtype);
          s = dot * (double)softmax_scale;
        } else {
          float dot = 0.f;
          for (int64_t d = 0; d < head_dim; ++d) dot += qf[d] * oracle_half_to_float(kr[d], dtype);
          s = (double)(dot * softmax_scale);
        }
        sc[x] = s;
        if (s > mx) mx = s;
      }
      if (use_f64) {
        double l = 0.0;
        for (int64_t d = 0; d < head_dim; ++d) acc[d] = 0.0;
        for (int64_t x = 0; x < n; ++x) {
          const uint16_t* vr = v + prefill_key_row(block_table, max_blocks, block_size, cu_seqlens_k, b,
                                                   lo + x) * row_stride + kh * head_dim;
          const double p = exp(sc[x] - mx);
          l += p;
          for (int64_t d = 0; d < head_dim; ++d) acc[d] += p * (double)oracle_half_to_float(vr[d], dtype);
        }
        for (int64_t d = 0; d < head_dim; ++d) o[d] = (float)(acc[d] / l);
      } else {
        float l = 0.f;
        for (int64_t d = 0; d < head_dim; ++d) accf[d] = 0.f;
        for (int64_t x = 0; x < n; ++x) {
          const uint16_t* vr = v + prefill_key_row(block_table, max_blocks, block_size, cu_seqlens_k, b,
                                                   lo + x) * row_stride + kh * head_dim;
          const float p = expf((float)sc[x] - (float)mx);
          l += p;
          for (int64_t d = 0; d < head_dim; ++d) accf[d] += p * oracle_half_to_float(vr[d], dtype);
        }
        for (int64_t d = 0; d < head_dim; ++d) o[d] = accf[d] / l;
      }
    }
    free(sc);
    free(qf);
    free(acc);
    free(accf);
  }
}

/* ------------------------------------------------------ norm + rope prologue */

void oracle_rope_cos_sin_cache(float* cache, int64_t max_position, int64_t rotary_dim, float base) {
  const int64_t half = rotary_dim / 2;
  for (int64_t t = 0; t < max_position; ++t) {
    for (int64_t i = 0; i < half; ++i) {
      const float inv_freq = 1.0f / powf(base, (float)(2 * i) / (float)rotary_dim);
      const float f = (float)t * inv_freq;
      cache[t * rotary_dim + i] = cosf(f);
      cache[t * rotary_dim + half + i] = sinf(f);
    }
  }
}

static float round_to(float x, int dtype) { return oracle_half_to_float(oracle_float_to_half(x, dtype), dtype); }

/* layers/rmsnorm.rs:52-87 (residual None) on one head of D values. */
static void rms_norm_head(float* x, const uint16_t* w, int64_t d, double eps, int dtype) {
  double ss = 0.0;
  for (int64_t i = 0; i < d; ++i) ss += (double)x[i] * (double)x[i];
  const float var = (float)ss / (float)d;
  const float s = sqrtf(var + (float)eps);
  for (int64_t i = 0; i < d; ++i) {
    const float n = round_to(x[i] / s, dtype);
    x[i] = round_to(n * oracle_half_to_float(w[i], dtype), dtype);
  }
}

/* layers/rope.rs:150-163 on one head (x holds dtype-rounded values). */
static void rope_head(float* x, const float* cs, int64_t d, int dtype) {
  const int64_t h = d / 2;
  for (int64_t i = 0; i < h; ++i) {
    const float x1 = x[i], x2 = x[h + i], c = cs[i], s = cs[h + i];
    /* each product and sum rounded to fp32 (built with -ffp-contract=off) */
    x[i] = round_to(x1 * c - x2 * s, dtype);
    x[h + i] = round_to(x2 * c + x1 * s, dtype);
  }
}

void oracle_qk_norm_rope_and_cache(uint16_t* q_out, uint16_t* k_out, const uint16_t* qkv,
                                   int64_t qkv_stride, const uint16_t* q_norm_weight,
                                   const uint16_t* k_norm_weight, double eps,
                                   const float* cos_sin_cache, int64_t max_position,
                                   const int32_t* positions, uint16_t* key_cache,
                                   uint16_t* value_cache, const int64_t* slot_mapping,
                                   int64_t num_tokens, int64_t num_heads, int64_t num_kv_heads,
                                   int64_t head_dim, int dtype) {
  const int64_t D = head_dim;
  float* x = (float*)malloc(sizeof(float) * (size_t)D);
  for (int64_t t = 0; t < num_tokens; ++t) {
    int64_t pos = positions[t];
    if (pos < 0) pos = 0;
    if (pos >= max_position) pos = max_position - 1;
    const float* cs = cos_sin_cache + pos * D;
    const uint16_t* row = qkv + t * qkv_stride;
    const int64_t slot = slot_mapping ? slot_mapping[t] : -1;
    for (int64_t h = 0; h < num_heads + num_kv_heads; ++h) {
      const int is_q = h < num_heads;
      for (int64_t i = 0; i < D; ++i) x[i] = oracle_half_to_float(row[h * D + i], dtype);
      const uint16_t* w = is_q ? q_norm_weight : k_norm_weight;
      if (w) rms_norm_head(x, w, D, eps, dtype);
      rope_head(x, cs, D, dtype);
      if (is_q) {
        for (int64_t i = 0; i < D; ++i) q_out[(t * num_heads + h) * D + i] = oracle_float_to_half(x[i], dtype);
      } else {
        const int64_t kh = h - num_heads;
        for (int64_t i = 0; i < D; ++i) {
          const uint16_t bits = oracle_float_to_half(x[i], dtype);
          if (k_out) k_out[(t * num_kv_heads + kh) * D + i] = bits;
          if (slot >= 0) key_cache[(slot * num_kv_heads + kh) * D + i] = bits;
        }
      }
    }
    if (slot >= 0)
      memcpy(value_cache + slot * num_kv_heads * D, row + (num_heads + num_kv_heads) * D,
             sizeof(uint16_t) * (size_t)(num_kv_heads * D));
  }
  free(x);
}

/* ------------------------------------------------------------------ XXH64 */

#define P64_1 0x9E3779B185EBCA87ULL
#define P64_2 0xC2B2AE3D27D4EB4FULL
#define P64_3 0x165667B19E3779F9ULL
#define P64_4 0x85EBCA77C2B2AE63ULL
#define P64_5 0x27D4EB2F165667C5ULL

static uint64_t rotl64(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
static uint64_t rd64(const uint8_t* p) {
  uint64_t v;
  memcpy(&v, p, 8); /* little-endian host */
  return v;
}
static uint32_t rd32(const uint8_t* p) {
  uint32_t v;
  memcpy(&v, p, 4);
  return v;
}
static uint64_t xxh_round(uint64_t acc, uint64_t in) {
  acc += in * P64_2;
  acc = rotl64(acc, 31);
  return acc * P64_1;
}
static uint64_t xxh_merge(uint64_t acc, uint64_t v) {
  acc ^= xxh_round(0, v);
  return acc * P64_1 + P64_4;
}

uint64_t oracle_xxh64(const void* data, size_t len, uint64_t seed) {
  const uint8_t* p = (const uint8_t*)data;
  const uint8_t* end = p + len;
  uint64_t h;
  if (len >= 32) {
    uint64_t v1 = seed + P64_1 + P64_2, v2 = seed + P64_2, v3 = seed, v4 = seed - P64_1;
    const uint8_t* limit = end - 32;
    do {
      v1 = xxh_round(v1, rd64(p));
      v2 = xxh_round(v2, rd64(p + 8));
      v3 = xxh_round(v3, rd64(p + 16));
      v4 = xxh_round(v4, rd64(p + 24));
      p += 32;
    } while (p <= limit);
    h = rotl64(v1, 1) + rotl64(v2, 7) + rotl64(v3, 12) + rotl64(v4, 18);
    h = xxh_merge(h, v1);
    h = xxh_merge(h, v2);
    h = xxh_merge(h, v3);
    h = xxh_merge(h, v4);
  } else {
    h = seed + P64_5;
  }
  h += (uint64_t)len;
  while (p + 8 <= end) {
    h ^= xxh_round(0, rd64(p));
    h = rotl64(h, 27) * P64_1 + P64_4;
    p += 8;
  }
  if (p + 4 <= end) {
    h ^= (uint64_t)rd32(p) * P64_1;
    h = rotl64(h, 23) * P64_2 + P64_3;
    p += 4;
  }
  while (p < end) {
    h ^= (uint64_t)(*p) * P64_5;
    h = rotl64(h, 11) * P64_1;
    ++p;
  }
  h ^= h >> 33;
  h *= P64_2;
  h ^= h >> 29;
  h *= P64_3;
  h ^= h >> 32;
  return h;
}
