/*
 * tmc_oracle — CPU restatement of the reference decode path's numerics.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg.  The product path
 * (libtmc_hip.so) never links, loads or calls it.
 *
 * Every function restates, in plain C with double accumulation, the semantics
 * of a reference function (file:line in /root/reference cited per function):
 * values are decoded from their storage dtype, combined in double, and either
 * returned unrounded ("precise", as GraphReference returns graph outputs) or
 * re-rounded with the host storage rule where the reference kernels round an
 * intermediate (storeValue, GraphReference.cpp:82-87).
 *
 * Storage dtype codes follow tensor::metal::ElementType order
 * (MetalRuntime.hpp:12): 0 = fp16, 1 = fp32, 2 = bf16, 3 = int32.
 */
#ifndef TMC_ORACLE_H
#define TMC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { TMCO_F16 = 0, TMCO_F32 = 1, TMCO_BF16 = 2, TMCO_I32 = 3 };

/* ---- scalar conversions (GraphReference.cpp:39-87, MetalRuntime.mm:42-104) ---- */
uint16_t tmco_f32_to_f16(float value);   /* round to nearest, ties away from zero */
float tmco_f16_to_f32(uint16_t bits);
uint16_t tmco_f32_to_bf16(float value);  /* round to nearest even */
float tmco_bf16_to_f32(uint16_t bits);
float tmco_store(double value, int dtype);          /* storeValue */
double tmco_load(const void *data, int dtype, size_t index);

/* Host upload / readback conversion (MetalRuntime.mm:515-592, :171-186). */
void tmco_encode(const float *src, size_t count, int dtype, void *dst);
void tmco_decode(const void *src, size_t count, int dtype, float *dst);

/* ---- Validator (Validator.cpp:11-66) ---- */
int tmco_compare(const float *actual, const double *reference, size_t count,
                 double atol, double rtol, double *max_abs_error,
                 size_t *mismatch_count, size_t *first_mismatch);
void tmco_rmsnorm_reference(const float *input, const float *weight, size_t rows,
                            size_t width, float epsilon, double *out);

/* ---- op-level oracles (storage-typed inputs, double math) ---- */
void tmco_rmsnorm(const void *x, const void *w, int dtype, size_t rows, size_t width,
                  float epsilon, double *out);
void tmco_add_rmsnorm(const void *residual, const void *update, const void *w, int dtype,
                      size_t rows, size_t width, float epsilon, float *sum_stored,
                      double *normalized);
void tmco_linear(const void *x, const void *weight, int dtype, size_t rows, size_t in_features,
                 size_t out_features, double *y);
void tmco_silu_mul(const void *gate, const void *up, int dtype, size_t count, double *out);
void tmco_gated_mlp(const void *x, const void *gate_w, const void *up_w, int dtype, size_t rows,
                    size_t hidden, size_t intermediate, double *out);
void tmco_rope(const void *x, const float *cosine, const float *sine, int dtype, size_t rows,
               size_t heads, size_t head_dim, const int32_t *positions, double *out);
void tmco_decode_attention(const void *q, const void *key_cache, const void *value_cache,
                           int dtype, size_t batch, size_t q_heads, size_t kv_heads,
                           size_t head_dim, size_t capacity, size_t valid, double *out);
int tmco_paged_attention(const void *q, const void *key_pool, const void *value_pool, int dtype,
                         size_t batch, size_t q_heads, size_t kv_heads, size_t head_dim,
                         size_t page_size, size_t page_stride, size_t head_stride,
                         const int32_t *block_tables, size_t max_pages,
                         const int32_t *valid_lengths, size_t active_count, double *out,
                         uint8_t *written);
void tmco_argmax(const float *logits, size_t rows, size_t vocabulary, int32_t *tokens);

/* ---- KV append index mappings (bit-exact copies) ---- */
void tmco_append_contiguous(const uint16_t *input, size_t batch, size_t heads, size_t head_dim,
                            size_t seq_len, size_t capacity, int input_head_major, int32_t valid,
                            uint16_t *cache);
void tmco_append_paged(const uint16_t *input, size_t batch, size_t heads, size_t head_dim,
                       size_t seq_len, size_t capacity, size_t page_size, int input_head_major,
                       int32_t valid, const int32_t *block_table, uint16_t *cache);
void tmco_append_serving(const uint16_t *input, size_t max_batch, size_t heads, size_t head_dim,
                         size_t capacity, size_t page_size, int input_head_major,
                         const int32_t *valid_lengths, const int32_t *block_tables,
                         int32_t active_count, uint16_t *cache);

/* ---- full decode step (GraphReference-style composition of the decoder's
 *      kernel sequence, DecoderLLMExecutor.cpp:322-849 / ServingRuntime.cpp:233-407) ---- */
typedef struct tmco_layer {
  const uint16_t *input_norm, *wq, *wk, *wv, *wo, *post_norm, *wg, *wu, *wd;
} tmco_layer;

typedef struct tmco_model {
  size_t layers, hidden, heads, head_dim, intermediate, vocabulary, capacity;
  float epsilon;
  size_t kv_heads; /* key/value heads (grouped-query attention); 0 = heads.
                      wk, wv are [kv_heads*head_dim, hidden]; query head h
                      reads kv head h / (heads / kv_heads). */
  const uint16_t *embedding, *final_norm, *lm_head;
  const float *rope_cos, *rope_sin;  /* [capacity, head_dim/2] */
  const tmco_layer *layer;
} tmco_model;

/* One decode step for `batch` requests over fp16 paged pools laid out
 * [page][kv_heads][page_size][head_dim] (one pool pair per layer).  The new
 * token of request b lands at position valid_lengths[b]-1.  Writes K/V into
 * the pools, fp32 logits [batch, vocabulary] (rounded from double) and the
 * greedy tokens.  Rows b < logits_from skip the final norm and LM head
 * (logits 0, token -1); layer_limit > 0 and below the layer count stops
 * after that many layers with no LM head at all. */
/* y[r,n] = sum_k x[r,k] W[n,k] (double, k order) with x as float storage
 * values and W fp16 bits; threaded by tmco_set_threads, same sums as
 * tmco_linear. */
void tmco_linear_values(const float *x, const uint16_t *weight, size_t rows, size_t in_features,
                        size_t out_features, double *y);

/* Threads used by tmco_decoder_step (default 1).  Results do not depend on
 * it: the work is split over output features and heads, never inside a sum. */
void tmco_set_threads(int threads);

int tmco_decoder_step(const tmco_model *model, uint16_t *const *key_pools,
                      uint16_t *const *value_pools, size_t page_size, size_t max_pages,
                      const int32_t *block_tables, const int32_t *tokens,
                      const int32_t *valid_lengths, size_t batch, size_t layer_limit,
                      size_t logits_from, float *logits, int32_t *next_tokens);

#ifdef __cplusplus
}
#endif

#endif
