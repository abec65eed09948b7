/*
 * tmc_oracle.c — CPU restatement of the reference decode path.
 *
 * TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg as the checker.  Nothing in the product library
 * links or calls this file.
 *
 * Pinning status (which check fixes each function) is listed per function;
 * "golden" means tests/golden vectors written from the compiled reference
 * GraphReference (oracle/_ref), "closed form" means a mathematical identity
 * test in tests/test_oracle.py.
 */
#include "tmc_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* Scalar conversions                                                         */
/* ------------------------------------------------------------------------- */

/* Host fp32 -> fp16 with round-to-nearest, ties away from zero; NaN keeps its
 * sign and becomes 0x7e00, overflow saturates to inf, values below half the
 * smallest subnormal flush to signed zero.  Follows the host rule of
 * GraphReference.cpp:39-60 and MetalRuntime.mm:42-67.  Pinned: golden. */
uint16_t tmco_f32_to_f16(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof bits);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t biased = (bits >> 23) & 0xffu;
  const uint32_t fraction = bits & 0x7fffffu;
  if (biased == 0xffu) return (uint16_t)(sign | (fraction ? 0x7e00u : 0x7c00u));
  const int exponent = (int)biased - 112; /* rebias 127 -> 15 */
  if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
  if (exponent <= 0) {
    if (exponent < -10) return (uint16_t)sign;
    const uint32_t significand = fraction | 0x800000u;
    const int shift = 14 - exponent;
    return (uint16_t)(sign | ((significand + (1u << (shift - 1))) >> shift));
  }
  const uint32_t rounded = fraction + 0x1000u; /* add half an fp16 ulp */
  if (rounded & 0x800000u) {
    if (exponent + 1 >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)(exponent + 1) << 10));
  }
  return (uint16_t)(sign | ((uint32_t)exponent << 10) | (rounded >> 13));
}

/* GraphReference.cpp:62-80.  Pinned: golden + exhaustive round trip. */
float tmco_f16_to_f32(uint16_t half) {
  const uint32_t sign = (uint32_t)(half & 0x8000u) << 16;
  uint32_t exponent = (half >> 10) & 0x1fu;
  uint32_t mantissa = half & 0x3ffu;
  uint32_t bits;
  if (exponent == 0) {
    if (mantissa == 0) {
      bits = sign;
    } else {
      int shift = 0;
      while ((mantissa & 0x400u) == 0) {
        mantissa <<= 1;
        ++shift;
      }
      mantissa &= 0x3ffu;
      bits = sign | ((uint32_t)(113 - shift) << 23) | (mantissa << 13);
    }
  } else if (exponent == 31) {
    bits = sign | 0x7f800000u | (mantissa << 13);
  } else {
    bits = sign | ((exponent + 112) << 23) | (mantissa << 13);
  }
  float result;
  memcpy(&result, &bits, sizeof result);
  return result;
}

/* MetalRuntime.mm:92-97 (round to nearest even on the raw bits).  Pinned:
 * closed form against numpy/torch bf16 for finite values. */
uint16_t tmco_f32_to_bf16(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof bits);
  return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

float tmco_bf16_to_f32(uint16_t half) {
  const uint32_t bits = (uint32_t)half << 16;
  float result;
  memcpy(&result, &bits, sizeof result);
  return result;
}

/* storeValue, GraphReference.cpp:82-87: fp16 rounds through the host rule,
 * int32 truncates, fp32 and bf16 keep the float value (bf16 is not rounded by
 * the reference oracle).  Pinned: golden. */
float tmco_store(double value, int dtype) {
  const float as_float = (float)value;
  if (dtype == TMCO_F16) return tmco_f16_to_f32(tmco_f32_to_f16(as_float));
  if (dtype == TMCO_I32) return (float)(int32_t)as_float;
  return as_float;
}

static float g_half_table[65536];
static int g_half_table_ready = 0;

static void half_table_init(void) {
  if (g_half_table_ready) return;
  for (uint32_t i = 0; i < 65536u; ++i) g_half_table[i] = tmco_f16_to_f32((uint16_t)i);
  g_half_table_ready = 1;
}

double tmco_load(const void *data, int dtype, size_t index) {
  switch (dtype) {
  case TMCO_F16: return tmco_f16_to_f32(((const uint16_t *)data)[index]);
  case TMCO_BF16: return tmco_bf16_to_f32(((const uint16_t *)data)[index]);
  case TMCO_I32: return (double)((const int32_t *)data)[index];
  default: return (double)((const float *)data)[index];
  }
}

/* Decode a storage-typed array into floats (values exactly representable). */
static float *decode_array(const void *data, int dtype, size_t count) {
  float *out = (float *)malloc((count ? count : 1) * sizeof(float));
  if (!out) abort();
  if (dtype == TMCO_F16) {
    half_table_init();
    const uint16_t *src = (const uint16_t *)data;
    for (size_t i = 0; i < count; ++i) out[i] = g_half_table[src[i]];
  } else {
    for (size_t i = 0; i < count; ++i) out[i] = (float)tmco_load(data, dtype, i);
  }
  return out;
}

/* MetalRuntime.mm:515-592: createBuffer / writeBuffer host conversion. */
void tmco_encode(const float *src, size_t count, int dtype, void *dst) {
  for (size_t i = 0; i < count; ++i) {
    switch (dtype) {
    case TMCO_F16: ((uint16_t *)dst)[i] = tmco_f32_to_f16(src[i]); break;
    case TMCO_BF16: ((uint16_t *)dst)[i] = tmco_f32_to_bf16(src[i]); break;
    case TMCO_I32: ((int32_t *)dst)[i] = (int32_t)src[i]; break;
    default: ((float *)dst)[i] = src[i]; break;
    }
  }
}

/* MetalRuntime.mm:171-186: MetalBuffer::read. */
void tmco_decode(const void *src, size_t count, int dtype, float *dst) {
  for (size_t i = 0; i < count; ++i) dst[i] = (float)tmco_load(src, dtype, i);
}

/* ------------------------------------------------------------------------- */
/* Validator                                                                  */
/* ------------------------------------------------------------------------- */

/* Validator.cpp:11-38: |actual - ref| <= atol + rtol*|ref|, non-finite fails. */
int tmco_compare(const float *actual, const double *reference, size_t count, double atol,
                 double rtol, double *max_abs_error, size_t *mismatch_count,
                 size_t *first_mismatch) {
  double worst = 0.0;
  size_t mismatches = 0, first = (size_t)-1;
  if (count == 0) {
    if (max_abs_error) *max_abs_error = 0.0;
    if (mismatch_count) *mismatch_count = 0;
    if (first_mismatch) *first_mismatch = first;
    return 0;
  }
  for (size_t i = 0; i < count; ++i) {
    const double expected = reference[i];
    const double value = actual[i];
    const int finite = isfinite(value) && isfinite(expected);
    const double error = finite ? fabs(value - expected) : INFINITY;
    if (error > worst) worst = error;
    if (!finite || error > atol + rtol * fabs(expected)) {
      if (mismatches == 0) first = i;
      ++mismatches;
    }
  }
  if (max_abs_error) *max_abs_error = worst;
  if (mismatch_count) *mismatch_count = mismatches;
  if (first_mismatch) *first_mismatch = first;
  return mismatches == 0;
}

/* Validator.cpp:40-66: double sum of squares, inverse = 1/sqrt(mean + eps),
 * out = x * inverse * w.  Pinned: golden ([1,4096], [3,4097], fp16 [1,257]). */
void tmco_rmsnorm_reference(const float *input, const float *weight, size_t rows, size_t width,
                            float epsilon, double *out) {
  for (size_t row = 0; row < rows; ++row) {
    const float *x = input + row * width;
    double squares = 0.0;
    for (size_t c = 0; c < width; ++c) squares += (double)x[c] * (double)x[c];
    const double inverse = 1.0 / sqrt(squares / (double)width + (double)epsilon);
    for (size_t c = 0; c < width; ++c)
      out[row * width + c] = (double)x[c] * inverse * (double)weight[c];
  }
}

/* ------------------------------------------------------------------------- */
/* Op-level oracles                                                           */
/* ------------------------------------------------------------------------- */

/* RMSNorm node of evaluateGraph (GraphReference.cpp:171-176) on storage-typed
 * operands.  Pinned: golden. */
void tmco_rmsnorm(const void *x, const void *w, int dtype, size_t rows, size_t width,
                  float epsilon, double *out) {
  float *xv = decode_array(x, dtype, rows * width);
  float *wv = decode_array(w, dtype, width);
  tmco_rmsnorm_reference(xv, wv, rows, width, epsilon, out);
  free(xv);
  free(wv);
}

/* Add -> RMSNorm graph (GraphReference.cpp:126-136 then :171-176): the sum is
 * stored in the graph dtype (storeValue) before it is normalized, matching the
 * rounding point of DecoderLLMMetalEmitter.cpp:451-453.  Pinned: golden. */
void tmco_add_rmsnorm(const void *residual, const void *update, const void *w, int dtype,
                      size_t rows, size_t width, float epsilon, float *sum_stored,
                      double *normalized) {
  const size_t count = rows * width;
  float *a = decode_array(residual, dtype, count);
  float *b = decode_array(update, dtype, count);
  float *wv = decode_array(w, dtype, width);
  for (size_t i = 0; i < count; ++i)
    sum_stored[i] = tmco_store((double)a[i] + (double)b[i], dtype);
  tmco_rmsnorm_reference(sum_stored, wv, rows, width, epsilon, normalized);
  free(a);
  free(b);
  free(wv);
}

/* y[r,n] = sum_k x[r,k] * W[n,k] in double, W stored [out,in] (nn.Linear).
 * Same sum as GraphReference MatMul (GraphReference.cpp:150-170) on W^T and
 * the DecodeGEMVTuner reference (DecodeGEMVTuner.cpp:98-118) before its
 * output rounding.  Pinned: golden (MatMul on W^T) + identity/basis tests. */
void tmco_linear(const void *x, const void *weight, int dtype, size_t rows, size_t in_features,
                 size_t out_features, double *y) {
  float *xv = decode_array(x, dtype, rows * in_features);
  float *row = (float *)malloc(in_features * sizeof(float));
  if (!row) abort();
  half_table_init();
  for (size_t n = 0; n < out_features; ++n) {
    if (dtype == TMCO_F16) {
      const uint16_t *src = (const uint16_t *)weight + n * in_features;
      for (size_t k = 0; k < in_features; ++k) row[k] = g_half_table[src[k]];
    } else {
      for (size_t k = 0; k < in_features; ++k)
        row[k] = (float)tmco_load(weight, dtype, n * in_features + k);
    }
    for (size_t r = 0; r < rows; ++r) {
      const float *xr = xv + r * in_features;
      double sum = 0.0;
      for (size_t k = 0; k < in_features; ++k) sum += (double)xr[k] * (double)row[k];
      y[r * out_features + n] = sum;
    }
  }
  free(row);
  free(xv);
}

/* Sign-stable SiLU of GraphReference.cpp:143-149. */
static double silu(double x) {
  const double e = exp(x >= 0.0 ? -x : x);
  return x >= 0.0 ? x / (1.0 + e) : x * e / (1.0 + e);
}

/* SiLU -> Mul graph: the activation is stored, the product is precise
 * (rounding points of DecoderLLMMetalEmitter.cpp:410-411).  Pinned: golden. */
void tmco_silu_mul(const void *gate, const void *up, int dtype, size_t count, double *out) {
  for (size_t i = 0; i < count; ++i) {
    const double activated = tmco_store(silu(tmco_load(gate, dtype, i)), dtype);
    out[i] = activated * tmco_load(up, dtype, i);
  }
}

/* Gated MLP (DecoderLLMMetalEmitter.cpp:479-536): gate and up projections are
 * stored, SiLU(gate) is stored, the product is precise.  Pinned: composition
 * of golden-pinned linear and silu_mul. */
void tmco_gated_mlp(const void *x, const void *gate_w, const void *up_w, int dtype, size_t rows,
                    size_t hidden, size_t intermediate, double *out) {
  const size_t count = rows * intermediate;
  double *g = (double *)malloc(count * sizeof(double));
  double *u = (double *)malloc(count * sizeof(double));
  if (!g || !u) abort();
  tmco_linear(x, gate_w, dtype, rows, hidden, intermediate, g);
  tmco_linear(x, up_w, dtype, rows, hidden, intermediate, u);
  for (size_t i = 0; i < count; ++i) {
    const double gs = tmco_store(g[i], dtype);
    const double us = tmco_store(u[i], dtype);
    const double activated = tmco_store(silu(gs), dtype);
    out[i] = activated * us;
  }
  free(g);
  free(u);
}

/* Interleaved-pair RoPE (GraphReference.cpp:218-228) with fp32 tables
 * [position, head_dim/2]; x is token-major [rows, heads, head_dim], the
 * result uses the same layout.  positions[row] selects the table row
 * (decoder: valid - S + t, DecoderLLMMetalEmitter.cpp:110-158; serving:
 * valid - 1, :260-312).  Pinned: golden + rotation-norm invariant. */
void tmco_rope(const void *x, const float *cosine, const float *sine, int dtype, size_t rows,
               size_t heads, size_t head_dim, const int32_t *positions, double *out) {
  const size_t pairs = head_dim / 2;
  for (size_t r = 0; r < rows; ++r) {
    const size_t position = (size_t)positions[r];
    for (size_t h = 0; h < heads; ++h) {
      for (size_t p = 0; p < pairs; ++p) {
        const size_t base = (r * heads + h) * head_dim + 2 * p;
        const double c = cosine[position * pairs + p];
        const double s = sine[position * pairs + p];
        const double even = tmco_load(x, dtype, base);
        const double odd = tmco_load(x, dtype, base + 1);
        out[base] = even * c - odd * s;
        out[base + 1] = even * s + odd * c;
      }
    }
  }
}

/* softmax(q K^T * scale) V over positions [0, valid) for one (query, kv) head
 * pair: the GraphReference chain MatMul -> Mul(scale) -> Softmax -> MatMul
 * (GraphReference.cpp:150-170, :196-207) evaluated in double.  The scale is
 * the fp32 literal 1/sqrt(D) baked into KVCacheMetalEmitter.cpp:119-208. */
static void attend(const float *q, const float *keys, const float *values, size_t valid,
                   size_t head_dim, double scale, double *scores, double *out) {
  double maximum = -INFINITY;
  for (size_t j = 0; j < valid; ++j) {
    double dot = 0.0;
    for (size_t d = 0; d < head_dim; ++d) dot += (double)q[d] * (double)keys[j * head_dim + d];
    scores[j] = dot * scale;
    if (scores[j] > maximum) maximum = scores[j];
  }
  double denominator = 0.0;
  for (size_t j = 0; j < valid; ++j) denominator += exp(scores[j] - maximum);
  for (size_t d = 0; d < head_dim; ++d) out[d] = 0.0;
  for (size_t j = 0; j < valid; ++j) {
    const double p = exp(scores[j] - maximum) / denominator;
    for (size_t d = 0; d < head_dim; ++d) out[d] += p * (double)values[j * head_dim + d];
  }
}

static double attention_scale(size_t head_dim) {
  return (double)(float)(1.0 / sqrt((double)head_dim));
}

/* Contiguous decode attention, caches [batch, kv_heads, capacity, head_dim],
 * q [batch, q_heads, head_dim]; out [batch, q_heads*head_dim].  Query head h
 * reads kv head h / (q_heads / kv_heads).  Pinned: closed forms (valid = 1
 * gives V0; equal keys give the mean of V) + golden attention chain. */
void tmco_decode_attention(const void *q, const void *key_cache, const void *value_cache,
                           int dtype, size_t batch, size_t q_heads, size_t kv_heads,
                           size_t head_dim, size_t capacity, size_t valid, double *out) {
  const size_t group = q_heads / kv_heads;
  const double scale = attention_scale(head_dim);
  float *qv = (float *)malloc(head_dim * sizeof(float));
  float *kv = (float *)malloc(valid * head_dim * sizeof(float) + 1);
  float *vv = (float *)malloc(valid * head_dim * sizeof(float) + 1);
  double *scores = (double *)malloc((valid + 1) * sizeof(double));
  if (!qv || !kv || !vv || !scores) abort();
  for (size_t b = 0; b < batch; ++b) {
    for (size_t h = 0; h < q_heads; ++h) {
      const size_t kh = h / group;
      for (size_t d = 0; d < head_dim; ++d)
        qv[d] = (float)tmco_load(q, dtype, (b * q_heads + h) * head_dim + d);
      const size_t base = (b * kv_heads + kh) * capacity * head_dim;
      for (size_t i = 0; i < valid * head_dim; ++i) {
        kv[i] = (float)tmco_load(key_cache, dtype, base + i);
        vv[i] = (float)tmco_load(value_cache, dtype, base + i);
      }
      attend(qv, kv, vv, valid, head_dim, scale, scores, out + (b * q_heads + h) * head_dim);
    }
  }
  free(qv);
  free(kv);
  free(vv);
  free(scores);
}

/* Paged decode attention over per-request block tables
 * (KVCacheMetalEmitter.cpp:312-406 semantics, generalised to kv_heads <=
 * q_heads): element (page, kv head, offset, d) lives at
 * page*page_stride + kvh*head_stride + offset*head_dim + d.  A request at or
 * beyond active_count, with valid <= 0 or valid > max_pages*page_size, or
 * with a negative page among the first ceil(valid/page_size) table entries
 * is skipped (written = 0), as the reference kernel returns before writing.
 * Returns the number of (request, head) outputs written.  Pinned: golden
 * Gather->attention chain + identity-table equivalence to the contiguous
 * oracle. */
int tmco_paged_attention(const void *q, const void *key_pool, const void *value_pool, int dtype,
                         size_t batch, size_t q_heads, size_t kv_heads, size_t head_dim,
                         size_t page_size, size_t page_stride, size_t head_stride,
                         const int32_t *block_tables, size_t max_pages,
                         const int32_t *valid_lengths, size_t active_count, double *out,
                         uint8_t *written) {
  const size_t group = q_heads / kv_heads;
  const double scale = attention_scale(head_dim);
  const size_t capacity = max_pages * page_size;
  float *qv = (float *)malloc(head_dim * sizeof(float));
  float *kv = (float *)malloc(capacity * head_dim * sizeof(float) + 1);
  float *vv = (float *)malloc(capacity * head_dim * sizeof(float) + 1);
  double *scores = (double *)malloc((capacity + 1) * sizeof(double));
  if (!qv || !kv || !vv || !scores) abort();
  int count = 0;
  for (size_t b = 0; b < batch; ++b) {
    const int32_t valid = valid_lengths[b];
    int skip = b >= active_count || valid <= 0 || (size_t)valid > capacity;
    const size_t pages = skip ? 0 : ((size_t)valid + page_size - 1) / page_size;
    for (size_t lp = 0; lp < pages && !skip; ++lp)
      if (block_tables[b * max_pages + lp] < 0) skip = 1;
    for (size_t h = 0; h < q_heads; ++h) {
      written[b * q_heads + h] = (uint8_t)!skip;
      if (skip) continue;
      const size_t kh = h / group;
      for (size_t d = 0; d < head_dim; ++d)
        qv[d] = (float)tmco_load(q, dtype, (b * q_heads + h) * head_dim + d);
      for (size_t pos = 0; pos < (size_t)valid; ++pos) {
        const size_t page = (size_t)block_tables[b * max_pages + pos / page_size];
        const size_t base =
            page * page_stride + kh * head_stride + (pos % page_size) * head_dim;
        for (size_t d = 0; d < head_dim; ++d) {
          kv[pos * head_dim + d] = (float)tmco_load(key_pool, dtype, base + d);
          vv[pos * head_dim + d] = (float)tmco_load(value_pool, dtype, base + d);
        }
      }
      attend(qv, kv, vv, (size_t)valid, head_dim, scale, scores,
             out + (b * q_heads + h) * head_dim);
      ++count;
    }
  }
  free(qv);
  free(kv);
  free(vv);
  free(scores);
  return count;
}

/* Greedy token per row, ties to the lowest index, NaN never selected, an
 * all-NaN row yields -1 (TransformerDecodeMetalEmitter.cpp:198-256).
 * Pinned: exact special cases in tests. */
void tmco_argmax(const float *logits, size_t rows, size_t vocabulary, int32_t *tokens) {
  for (size_t r = 0; r < rows; ++r) {
    float best = -INFINITY;
    int32_t selected = -1;
    for (size_t t = 0; t < vocabulary; ++t) {
      const float candidate = logits[r * vocabulary + t];
      if (candidate > best || (candidate == best && (selected < 0 || (int32_t)t < selected))) {
        best = candidate;
        selected = (int32_t)t;
      }
    }
    tokens[r] = selected;
  }
}

/* ------------------------------------------------------------------------- */
/* KV append index maps (DecoderLLMMetalEmitter.cpp:160-373)                  */
/* ------------------------------------------------------------------------- */

void tmco_append_contiguous(const uint16_t *input, size_t batch, size_t heads, size_t head_dim,
                            size_t seq_len, size_t capacity, int input_head_major, int32_t valid,
                            uint16_t *cache) {
  if (valid < (int32_t)seq_len || valid > (int32_t)capacity) return;
  const size_t hidden = heads * head_dim;
  for (size_t b = 0; b < batch; ++b)
    for (size_t t = 0; t < seq_len; ++t)
      for (size_t f = 0; f < hidden; ++f) {
        const size_t h = f / head_dim, c = f % head_dim;
        const size_t position = (size_t)valid - seq_len + t;
        const size_t src = input_head_major ? ((b * heads + h) * seq_len + t) * head_dim + c
                                            : (b * seq_len + t) * hidden + f;
        cache[((b * heads + h) * capacity + position) * head_dim + c] = input[src];
      }
}

void tmco_append_paged(const uint16_t *input, size_t batch, size_t heads, size_t head_dim,
                       size_t seq_len, size_t capacity, size_t page_size, int input_head_major,
                       int32_t valid, const int32_t *block_table, uint16_t *cache) {
  if (valid < (int32_t)seq_len || valid > (int32_t)capacity) return;
  const size_t hidden = heads * head_dim;
  for (size_t b = 0; b < batch; ++b)
    for (size_t t = 0; t < seq_len; ++t)
      for (size_t f = 0; f < hidden; ++f) {
        const size_t h = f / head_dim, c = f % head_dim;
        const size_t position = (size_t)valid - seq_len + t;
        const int32_t page = block_table[position / page_size];
        if (page < 0) continue;
        const size_t src = input_head_major ? ((b * heads + h) * seq_len + t) * head_dim + c
                                            : (b * seq_len + t) * hidden + f;
        const size_t dst =
            ((((size_t)page * batch + b) * heads + h) * page_size + position % page_size) *
                head_dim + c;
        cache[dst] = input[src];
      }
}

void tmco_append_serving(const uint16_t *input, size_t max_batch, size_t heads, size_t head_dim,
                         size_t capacity, size_t page_size, int input_head_major,
                         const int32_t *valid_lengths, const int32_t *block_tables,
                         int32_t active_count, uint16_t *cache) {
  const size_t hidden = heads * head_dim;
  const size_t max_pages = (capacity + page_size - 1) / page_size;
  for (size_t r = 0; r < max_batch; ++r) {
    if ((int32_t)r >= active_count) return;
    const int32_t valid = valid_lengths[r];
    if (valid <= 0 || valid > (int32_t)capacity) continue;
    const size_t position = (size_t)valid - 1;
    const int32_t page = block_tables[r * max_pages + position / page_size];
    if (page < 0) continue;
    for (size_t f = 0; f < hidden; ++f) {
      const size_t h = f / head_dim, c = f % head_dim;
      const size_t src = input_head_major ? (r * heads + h) * head_dim + c : r * hidden + f;
      cache[(((size_t)page * heads + h) * page_size + position % page_size) * head_dim + c] =
          input[src];
    }
  }
}

/* ------------------------------------------------------------------------- */
/* Decode step composition                                                   */
/* ------------------------------------------------------------------------- */

static void store_array(const double *src, size_t count, float *dst) {
  for (size_t i = 0; i < count; ++i) dst[i] = tmco_store(src[i], TMCO_F16);
}

/* Threads of the decode-step composition (tmco_set_threads; 1 by default,
 * so the CPU baseline stays single-threaded).  Work is split over output
 * features and heads only: every sum keeps its own order, so the results do
 * not depend on the thread count. */
static int g_threads = 1;

void tmco_set_threads(int threads) { g_threads = threads > 0 ? threads : 1; }

/* Sixteen rows against two weight rows: the inputs are k-major
 * (xt[k*16 + j] = x[row j][k], storage values as float) and every
 * (row, weight row) pair keeps its own double sum in k order, so a
 * vectorised build computes exactly the scalar sums. */
__attribute__((target_clones("avx512f", "avx2", "default")))
static void dot16x2(const float *xt, const float *w0, const float *w1, size_t in_features,
                    double *sums0, double *sums1) {
  double s0[16] = {0.0}, s1[16] = {0.0};
  for (size_t k = 0; k < in_features; ++k) {
    const double a = (double)w0[k], b = (double)w1[k];
    const float *xk = xt + k * 16;
    for (int j = 0; j < 16; ++j) {
      const double xv = (double)xk[j];
      s0[j] += xv * a;
      s1[j] += xv * b;
    }
  }
  for (int j = 0; j < 16; ++j) {
    sums0[j] = s0[j];
    sums1[j] = s1[j];
  }
}

/* y[r,n] = sum_k x[r,k]*W[n,k] with x already float (storage values) and W
 * fp16 bits; double accumulation in k order for every (r, n).  Rows go in
 * blocks of 16 through dot16x2 (two output features at a time), a few
 * blocks per pass over the weights so that their inputs stay in cache; the
 * last rows % 16 go one at a time. */
static void linear_f16(const float *x, const uint16_t *w, size_t rows, size_t in_features,
                       size_t out_features, double *y) {
  enum { kBlocksPerPass = 4 };
  const size_t blocks = rows / 16;
  const size_t passes = (blocks + kBlocksPerPass - 1) / kBlocksPerPass + (rows % 16 ? 1 : 0);
  float *xt = NULL;
  if (blocks) {
    xt = (float *)malloc(blocks * in_features * 16 * sizeof(float));
    if (!xt) abort();
    for (size_t b = 0; b < blocks; ++b)
      for (size_t k = 0; k < in_features; ++k)
        for (size_t j = 0; j < 16; ++j)
          xt[(b * in_features + k) * 16 + j] = x[(b * 16 + j) * in_features + k];
  }
  const size_t pairs = (out_features + 1) / 2;
#pragma omp parallel num_threads(g_threads) if (g_threads > 1)
  {
    float *row = (float *)malloc(2 * in_features * sizeof(float));
    if (!row) abort();
    for (size_t pass = 0; pass < passes; ++pass) {
      const size_t b0 = pass * kBlocksPerPass;
      const size_t b1 = b0 + kBlocksPerPass < blocks ? b0 + kBlocksPerPass : blocks;
      const int tail = b0 >= blocks; /* the pass over the last rows % 16 */
#pragma omp for schedule(static)
      for (size_t pair = 0; pair < pairs; ++pair) {
        const size_t n0 = 2 * pair, count = n0 + 1 < out_features ? 2 : 1;
        for (size_t i = 0; i < count; ++i) {
          const uint16_t *src = w + (n0 + i) * in_features;
          for (size_t k = 0; k < in_features; ++k) row[i * in_features + k] = g_half_table[src[k]];
        }
        if (tail) {
          for (size_t i = 0; i < count; ++i) {
            const float *wr = row + i * in_features;
            for (size_t r = blocks * 16; r < rows; ++r) {
              const float *xr = x + r * in_features;
              double sum = 0.0;
              for (size_t k = 0; k < in_features; ++k) sum += (double)xr[k] * (double)wr[k];
              y[r * out_features + n0 + i] = sum;
            }
          }
          continue;
        }
        const float *w1 = row + (count - 1) * in_features;
        double sums0[16], sums1[16];
        for (size_t b = b0; b < b1; ++b) {
          dot16x2(xt + b * in_features * 16, row, w1, in_features, sums0, sums1);
          for (size_t j = 0; j < 16; ++j) {
            y[(b * 16 + j) * out_features + n0] = sums0[j];
            if (count == 2) y[(b * 16 + j) * out_features + n0 + 1] = sums1[j];
          }
        }
      }
    }
    free(row);
  }
  free(xt);
}

/* The decode step's linear on its own: x holds storage values as floats, W
 * fp16 bits [out, in]; the same double sums, in the same k order, as
 * tmco_linear (which decodes x itself), split over tmco_set_threads threads.
 * Pinned: equality with tmco_linear (tests/test_oracle_decoder.py). */
void tmco_linear_values(const float *x, const uint16_t *weight, size_t rows, size_t in_features,
                        size_t out_features, double *y) {
  half_table_init();
  linear_f16(x, weight, rows, in_features, out_features, y);
}

static void rmsnorm_f16(const float *x, const uint16_t *w, size_t rows, size_t width,
                        float epsilon, double *out) {
  for (size_t r = 0; r < rows; ++r) {
    double squares = 0.0;
    for (size_t c = 0; c < width; ++c) squares += (double)x[r * width + c] * x[r * width + c];
    const double inverse = 1.0 / sqrt(squares / (double)width + (double)epsilon);
    for (size_t c = 0; c < width; ++c)
      out[r * width + c] = (double)x[r * width + c] * inverse * (double)g_half_table[w[c]];
  }
}

/* One decode step of the decoder kernel sequence (DecoderLLMExecutor.cpp:
 * 322-849; ServingRuntime.cpp:233-407): every kernel output is stored in fp16
 * (storeValue) before the next kernel reads it; logits are returned as fp32.
 * Pinned: composition of the pinned op oracles (tests/test_oracle_decoder.py
 * rebuilds the step from the separately pinned ops and requires identical
 * logits and pool bits). */
int tmco_decoder_step(const tmco_model *m, uint16_t *const *key_pools,
                      uint16_t *const *value_pools, size_t page_size, size_t max_pages,
                      const int32_t *block_tables, const int32_t *tokens,
                      const int32_t *valid_lengths, size_t batch, size_t layer_limit,
                      size_t logits_from, float *logits, int32_t *next_tokens) {
  half_table_init();
  const size_t H = m->hidden, D = m->head_dim, NH = m->heads, I = m->intermediate;
  const size_t KVH = m->kv_heads ? m->kv_heads : NH, KV = KVH * D, group = NH / KVH;
  const size_t pairs = D / 2;
  if (KVH == 0 || NH % KVH != 0) return -3;
  const size_t layers = layer_limit && layer_limit < m->layers ? layer_limit : m->layers;
  /* acc holds one layer's widest output for every row, or the LM head's
   * logits for the rows from logits_from on. */
  const size_t layer_width = I > H ? I : H;
  const size_t head_rows = logits_from < batch ? batch - logits_from : 0;
  const size_t acc_size = batch * layer_width > head_rows * m->vocabulary
                              ? batch * layer_width : head_rows * m->vocabulary;
  for (size_t b = 0; b < batch; ++b) {
    if (tokens[b] < 0 || (size_t)tokens[b] >= m->vocabulary) return -1;
    if (valid_lengths[b] <= 0 || (size_t)valid_lengths[b] > m->capacity) return -2;
  }
  float *cur = (float *)malloc(batch * H * sizeof(float));
  float *nrm = (float *)malloc(batch * H * sizeof(float));
  float *q = (float *)malloc(batch * H * sizeof(float));
  float *k = (float *)malloc(batch * H * sizeof(float));
  float *v = (float *)malloc(batch * H * sizeof(float));
  float *ctx = (float *)malloc(batch * H * sizeof(float));
  float *after = (float *)malloc(batch * H * sizeof(float));
  float *gated = (float *)malloc(batch * I * sizeof(float));
  double *acc = (double *)malloc(acc_size * sizeof(double));
  double *acc2 = (double *)malloc(batch * I * sizeof(double));
  if (!cur || !nrm || !q || !k || !v || !ctx || !after || !gated || !acc || !acc2) abort();
  const double scale = attention_scale(D);

  for (size_t b = 0; b < batch; ++b)
    for (size_t f = 0; f < H; ++f)
      cur[b * H + f] = g_half_table[m->embedding[(size_t)tokens[b] * H + f]];

  for (size_t l = 0; l < layers; ++l) {
    const tmco_layer *L = &m->layer[l];
    const int32_t *table = block_tables + l * batch * max_pages;
    rmsnorm_f16(cur, L->input_norm, batch, H, m->epsilon, acc);
    store_array(acc, batch * H, nrm);
    linear_f16(nrm, L->wq, batch, H, H, acc);
    store_array(acc, batch * H, q);
    linear_f16(nrm, L->wk, batch, H, KV, acc);
    store_array(acc, batch * KV, k);
    linear_f16(nrm, L->wv, batch, H, KV, acc);
    store_array(acc, batch * KV, v);
    for (size_t b = 0; b < batch; ++b) {
      const size_t valid = (size_t)valid_lengths[b];
      const size_t position = valid - 1;
      /* RoPE on q and k, stored. */
      for (size_t p = 0; p < pairs; ++p) {
        const double c = m->rope_cos[position * pairs + p];
        const double s = m->rope_sin[position * pairs + p];
        for (size_t h = 0; h < NH; ++h) {
          const size_t base = b * H + h * D + 2 * p;
          const double qe = q[base], qo = q[base + 1];
          q[base] = tmco_store(qe * c - qo * s, TMCO_F16);
          q[base + 1] = tmco_store(qe * s + qo * c, TMCO_F16);
        }
        for (size_t h = 0; h < KVH; ++h) {
          const size_t base = b * KV + h * D + 2 * p;
          const double ke = k[base], ko = k[base + 1];
          k[base] = tmco_store(ke * c - ko * s, TMCO_F16);
          k[base + 1] = tmco_store(ke * s + ko * c, TMCO_F16);
        }
      }
      /* Append k, v at position valid-1 ([page][kv_head][page_size][D] pools). */
      const int32_t page = table[b * max_pages + position / page_size];
      if (page < 0) continue;
      for (size_t h = 0; h < KVH; ++h)
        for (size_t c = 0; c < D; ++c) {
          const size_t dst = (((size_t)page * KVH + h) * page_size + position % page_size) * D + c;
          key_pools[l][dst] = tmco_f32_to_f16(k[b * KV + h * D + c]);
          value_pools[l][dst] = tmco_f32_to_f16(v[b * KV + h * D + c]);
        }
      /* Attention over [0, valid), stored; query head h reads kv head h/group. */
#pragma omp parallel num_threads(g_threads) if (g_threads > 1)
      {
        float *keys = (float *)malloc(valid * D * sizeof(float));
        float *vals = (float *)malloc(valid * D * sizeof(float));
        double *scores = (double *)malloc((valid + 1) * sizeof(double));
        double *head_out = (double *)malloc(D * sizeof(double));
        if (!keys || !vals || !scores || !head_out) abort();
#pragma omp for schedule(static)
        for (size_t h = 0; h < NH; ++h) {
          for (size_t pos = 0; pos < valid; ++pos) {
            const size_t pg = (size_t)table[b * max_pages + pos / page_size];
            const size_t base = ((pg * KVH + h / group) * page_size + pos % page_size) * D;
            for (size_t c = 0; c < D; ++c) {
              keys[pos * D + c] = g_half_table[key_pools[l][base + c]];
              vals[pos * D + c] = g_half_table[value_pools[l][base + c]];
            }
          }
          attend(q + b * H + h * D, keys, vals, valid, D, scale, scores, head_out);
          for (size_t c = 0; c < D; ++c)
            ctx[b * H + h * D + c] = tmco_store(head_out[c], TMCO_F16);
        }
        free(keys); free(vals); free(scores); free(head_out);
      }
    }
    linear_f16(ctx, L->wo, batch, H, H, acc);
    for (size_t i = 0; i < batch * H; ++i) {
      const double attn = tmco_store(acc[i], TMCO_F16);
      after[i] = tmco_store((double)cur[i] + attn, TMCO_F16);
    }
    rmsnorm_f16(after, L->post_norm, batch, H, m->epsilon, acc);
    store_array(acc, batch * H, nrm);
    linear_f16(nrm, L->wg, batch, H, I, acc);
    linear_f16(nrm, L->wu, batch, H, I, acc2);
    for (size_t i = 0; i < batch * I; ++i) {
      const double g = tmco_store(acc[i], TMCO_F16);
      const double u = tmco_store(acc2[i], TMCO_F16);
      gated[i] = tmco_store(tmco_store(silu(g), TMCO_F16) * u, TMCO_F16);
    }
    linear_f16(gated, L->wd, batch, I, H, acc);
    for (size_t i = 0; i < batch * H; ++i) {
      const double mlp = tmco_store(acc[i], TMCO_F16);
      cur[i] = tmco_store((double)after[i] + mlp, TMCO_F16);
    }
  }

  if (layers == m->layers && logits_from < batch) {
    /* Rows before logits_from (prompt rows whose logits are not needed) skip
     * the LM head; their logits stay 0 and their next token -1. */
    const size_t rows = batch - logits_from, V = m->vocabulary;
    rmsnorm_f16(cur + logits_from * H, m->final_norm, rows, H, m->epsilon, acc);
    store_array(acc, rows * H, nrm);
    linear_f16(nrm, m->lm_head, rows, H, V, acc);
    memset(logits, 0, logits_from * V * sizeof(float));
    for (size_t i = 0; i < rows * V; ++i) logits[logits_from * V + i] = (float)acc[i];
    for (size_t b = 0; b < logits_from; ++b) next_tokens[b] = -1;
    tmco_argmax(logits + logits_from * V, rows, V, next_tokens + logits_from);
  }

  free(cur); free(nrm); free(q); free(k); free(v); free(ctx); free(after); free(gated);
  free(acc); free(acc2);
  return 0;
}
