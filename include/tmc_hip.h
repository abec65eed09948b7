/*
 * tmc_hip.h — C ABI of the MI355X (gfx950) decode backend, libtmc_hip.so.
 *
 * This is the drop-in boundary for the reference's Metal backend
 * (/root/reference/src/backend/metal): plain pointers and sizes, no C++ or
 * torch types.  Every function returns 0 on success and a nonzero status on
 * failure; the failure text is then available from tmc_last_error() (a
 * thread-local string, the counterpart of the reference's
 * `std::string errorMessage` results, MetalRuntime.hpp:33-44,74-77,91-99).
 *
 * Two layers:
 *  1. Runtime objects (tmc_rt_*, tmc_buf_*, tmc_kernel_*, tmc_prepare,
 *     tmc_exec_*, tmc_seq_*) replace MetalRuntime / MetalBuffer /
 *     PreparedExecution / PreparedSequence (MetalRuntime.hpp:56-208).
 *  2. Typed kernel entry points (tmc_gemv_f16 ... tmc_argmax_f32) replace the
 *     MSL emitters of DecodeGEMVMetalEmitter / DecoderLLMMetalEmitter /
 *     KVCacheMetalEmitter / TransformerDecodeMetalEmitter.  They take device
 *     pointers, shapes and a hipStream_t passed as `void *stream` (NULL =
 *     the default stream) and enqueue asynchronously.
 *
 * Paged K/V writes (every *append* entry point and the q.k.v projections
 * with a RoPE + append epilogue) skip a block-table entry < 0 and trust
 * every other entry: the caller guarantees that each page id it stores in a
 * block table is below the number of pages of the pool it passes (the
 * KVPagePool / KVCacheState host layer only stores ids it allocated).  The
 * paged attention reads take `pool_pages` and treat an id past it as
 * missing, so a stale table can spoil reads but never read out of bounds.
 *
 * Storage dtype codes follow tensor::metal::ElementType (MetalRuntime.hpp:12).
 * Weights are [out_features, in_features] row-major (nn.Linear layout, as in
 * DecodeGEMVMetalEmitter.cpp:97-103).
 */
#ifndef TMC_HIP_H
#define TMC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum tmc_dtype { TMC_F16 = 0, TMC_F32 = 1, TMC_BF16 = 2, TMC_I32 = 3 } tmc_dtype;

/* Thread-local text of the last failure on this thread ("" when none). */
const char *tmc_last_error(void);

/* ===================================================================== */
/* 1. Runtime objects                                                     */
/* ===================================================================== */

typedef struct tmc_runtime tmc_runtime;
typedef struct tmc_buffer tmc_buffer;
typedef struct tmc_kernel tmc_kernel;
typedef struct tmc_exec tmc_exec;
typedef struct tmc_seq tmc_seq;

/* tensor::metal::HardwareInfo (MetalRuntime.hpp:14-19). */
typedef struct tmc_hardware_info {
  size_t max_threads_per_threadgroup;
  size_t max_threadgroup_memory_length; /* LDS bytes per workgroup */
  size_t max_buffer_length;
  int supports_bfloat16;
  int compute_units;
  int wave_size;
} tmc_hardware_info;

/* MetalRuntime::MetalRuntime / ~MetalRuntime / isAvailable / deviceName /
 * initializationError / hardwareInfo (MetalRuntime.hpp:151-166). */
int tmc_rt_create(tmc_runtime **out);
void tmc_rt_destroy(tmc_runtime *rt);
int tmc_rt_is_available(const tmc_runtime *rt);
const char *tmc_rt_device_name(const tmc_runtime *rt);
const char *tmc_rt_init_error(const tmc_runtime *rt);
int tmc_rt_device_info(const tmc_runtime *rt, tmc_hardware_info *info);
/* The stream every prepared execution and sequence of this runtime uses. */
void *tmc_rt_stream(const tmc_runtime *rt);
/* Wait for all work enqueued on that stream (the reference's execute() is
 * synchronous; this is the wait for work enqueued with tmc_seq_launch). */
int tmc_rt_synchronize(tmc_runtime *rt);

/* MetalRuntime::createBuffer (MetalRuntime.hpp:186-188; .mm:515-561): host
 * floats converted per dtype (fp16 ties away from zero, bf16 RNE, int32
 * truncation); without data the buffer is filled with NaN (float types) or 0
 * (int32). */
int tmc_buf_create(tmc_runtime *rt, size_t count, int dtype, const float *init,
                   tmc_buffer **out);
/* Wrap existing device memory (not owned, never freed by the runtime). */
int tmc_buf_wrap(tmc_runtime *rt, void *device_ptr, size_t count, int dtype, tmc_buffer **out);
/* MetalRuntime::writeBuffer (MetalRuntime.hpp:189-192; .mm:563-592). */
int tmc_buf_write(tmc_buffer *buf, const float *data, size_t count, size_t offset);
/* Raw storage copies (no conversion); bytes/offsets in elements of the dtype. */
int tmc_buf_write_raw(tmc_buffer *buf, const void *data, size_t count, size_t offset);
int tmc_buf_read_raw(const tmc_buffer *buf, void *data, size_t count, size_t offset);
/* tmc_buf_write_raw without the wait: `data` is copied into the runtime's
 * pinned staging area and the host-to-device copy is queued on the runtime
 * stream, ordered before later launches on it; the caller may reuse `data`
 * on return.  No counterpart in the reference (its writes are synchronous):
 * it is for per-step metadata uploads that precede a graph launch.  Copies
 * larger than the staging area (4 MiB) fall back to tmc_buf_write_raw.
 * Refused while the runtime stream is being captured. */
int tmc_buf_write_raw_async(tmc_buffer *buf, const void *data, size_t count, size_t offset);
/* Sparse form of tmc_buf_write_raw_async for a TMC_I32 buffer: `pairs` holds
 * `count` (element index, value) pairs, indices increasing and inside the
 * buffer.  The pairs are copied into the same pinned staging area and a
 * kernel on the runtime stream stores each value at its index, reading the
 * pairs from the pinned host memory (no DMA transfer is queued; one of
 * 512 KiB cost about 80 us between two graph launches on MI355X, the kernel
 * about 6 us).  No counterpart in the reference: it is for the per-step
 * block-table changes of a batched decode, one entry per layer for each
 * request that enters a new page.  At most 524288 pairs; refused while the
 * runtime stream is being captured. */
int tmc_buf_write_sparse_async(tmc_buffer *buf, const int32_t *pairs, size_t count);
/* Device-to-device copy of `count` elements (same dtype, same runtime),
 * queued on the runtime stream.  No counterpart in the reference: the
 * chained decode loop uses it to feed each step's greedy tokens to the next
 * step and into a history buffer without a host round trip. */
int tmc_buf_copy_async(tmc_buffer *dst, size_t dst_offset, const tmc_buffer *src,
                       size_t src_offset, size_t count);
/* MetalBuffer::read (MetalRuntime.hpp:66; .mm:171-186). */
int tmc_buf_read(const tmc_buffer *buf, float *out);
size_t tmc_buf_count(const tmc_buffer *buf);
int tmc_buf_dtype(const tmc_buffer *buf);
void *tmc_buf_device_ptr(const tmc_buffer *buf);
void tmc_buf_release(tmc_buffer *buf);

/* The host conversions behind tmc_buf_create / tmc_buf_write / tmc_buf_read,
 * on host memory only (no device, no runtime): the reference's floatToHalf /
 * halfToFloat / floatToBFloat16 / bfloat16ToFloat (MetalRuntime.mm:42-104)
 * and its int32 truncating cast (.mm:545-547,585-589).  fp32 -> fp16 rounds
 * to nearest with ties away from zero, NaN -> 0x7e00 with its sign, overflow
 * -> inf; fp32 -> bf16 rounds to nearest even on the raw bits.  dst holds
 * `count` elements of the storage dtype (encode) or floats (decode). */
int tmc_host_encode(const float *src, size_t count, int dtype, void *dst);
int tmc_host_decode(const void *src, size_t count, int dtype, float *dst);

/* Replaces MetalRuntime::createComputePipeline(source, functionName)
 * (MetalRuntime.hpp:168-170; .mm:397-513).  `key` names a built-in gfx950
 * kernel and its specialization as "name?k=v&k=v" (the string an emitter
 * returns in GeneratedKernel::source, MetalEmitter.hpp:13-18).  On success
 * `*bindings` receives the binding count and `types`/`writable` (each of
 * length >= 32) describe every buffer binding in ABI order: inputs, outputs,
 * then an optional uint32 constants binding (type TMC_I32, writable 0). */
int tmc_kernel_resolve(tmc_runtime *rt, const char *key, tmc_kernel **out, int *bindings,
                       int *types, int *writable);
/* Grid the resolved kernel needs (DispatchSize, MetalRuntime.hpp:87-90). */
int tmc_kernel_dispatch(const tmc_kernel *kernel, size_t *groups, size_t *threads);
void tmc_kernel_release(tmc_kernel *kernel);

/* MetalRuntime::prepareBuffers (MetalRuntime.hpp:193-201; .mm:594-648):
 * inputs [0,n_in), outputs [n_in, n_in+n_out), u32 constants last.  Outputs
 * must be distinct and must not alias inputs; at most 31 bindings and 1024
 * constants. */
int tmc_prepare(tmc_runtime *rt, const tmc_kernel *kernel, tmc_buffer *const *inputs,
                size_t n_in, tmc_buffer *const *outputs, size_t n_out, size_t groups,
                size_t threads, const uint32_t *constants, size_t n_constants, tmc_exec **out);
/* PreparedExecution::run / execute (MetalRuntime.hpp:110-115): with
 * `reset_outputs` the outputs are first filled with sentinels (NaN, 0x7e00,
 * 0x7fc0, INT32_MIN; .mm:200-215).  Synchronous; times are optional outputs
 * (gpu_us from hipEvents, cpu_us from submit to completion). */
int tmc_exec_run(tmc_exec *exec, int reset_outputs, double *gpu_us, double *cpu_us);
void tmc_exec_release(tmc_exec *exec);

/* MetalRuntime::prepareSequence / PreparedSequence::execute
 * (MetalRuntime.hpp:130-142,202-203; .mm:292-341,751-781): the steps are
 * captured once into a HIP graph and replayed with one hipGraphLaunch.  A
 * sequence that holds a step kept out of graphs replays its steps eagerly,
 * in order, on the runtime's stream instead.  Either way the steps and their
 * buffers must outlive the sequence. */
int tmc_seq_create(tmc_runtime *rt, tmc_exec *const *steps, size_t n, tmc_seq **out);
int tmc_seq_run(tmc_seq *seq, double *gpu_us, double *cpu_us);
/* Enqueue one replay on the runtime stream without waiting. */
int tmc_seq_launch(tmc_seq *seq);
void tmc_seq_release(tmc_seq *seq);

/* Test hook: make the next `count` executions (exec or sequence) fail before
 * they launch, so host rollback paths can be exercised without a GPU fault. */
void tmc_rt_fail_next(tmc_runtime *rt, int count);

/* ===================================================================== */
/* 2. Typed kernel entry points                                           */
/* ===================================================================== */

/* Decode GEMV, emitDecodeGEMV (DecodeGEMVMetalEmitter.cpp:68-132):
 * y[r,n] = sum_k x[r,k] * W[n,k] with fp16 x and W, fp32 accumulation, y in
 * y_dtype (TMC_F16 or TMC_F32).  Batch 1 runs the wave64 split-K dot
 * GEMV; larger batches run the MFMA skinny GEMM (see tmc_gemv_config). */
int tmc_gemv_f16(const void *x, const void *w, void *y, int y_dtype, int64_t batch,
                 int64_t in_features, int64_t out_features, void *stream);

/* Launch configuration of the GEMV family (the decode GEMV tuner's
 * candidates; DecodeGEMVConfig, DecodeGEMVMetalEmitter.hpp:11-16, retargeted
 * to gfx950).  algorithm 0 = default for the shape, 1 = wave64 split-K dot
 * (rows_per_wave 1|2 rows per wave, unroll 2|4 16-byte loads per row in
 * flight, k_split 1|2|4 waves sharing a row), 2 = MFMA (rows_per_wave =
 * 16-row output tiles per block, k_split waves per tile, n_tiles*k_split
 * <= 16, unroll 1|2 K tiles in flight), 3 = MFMA row tiles with buffer loads
 * (rows_per_wave 1|2|4 16-row tiles per wave, k_split 1..16 waves per block
 * each taking a contiguous K run, unroll 1|2|4 adjacent K tiles in flight,
 * 4 only with at most 2 tiles; batch handled 16 rows per pass), 4 = linear
 * baseline, one thread per output (emitLinearBaseline,
 * DecodeGEMVMetalEmitter.cpp:18-66; the tuners' baseline and fallback, other
 * fields ignored), 5 = persistent dot at batch 1 (no reference counterpart:
 * the resident blocks each stream a fixed share of row groups, rows_per_wave
 * 1|2 rows per group kept two groups deep; k_split must be 4 and unroll is
 * ignored; in_features <= 16384 and W below 4 GiB; results equal algorithm 1
 * at k_split 4 bit for bit).  Algorithms 1-3 and 5 need in_features % 8 == 0
 * and 16-byte aligned x and W; otherwise a scalar per-output kernel runs. */
typedef struct tmc_gemv_config {
  int algorithm;
  int rows_per_wave;
  int unroll;
  int k_split;
} tmc_gemv_config;

/* tmc_gemv_f16 with an explicit launch configuration. */
int tmc_gemv_f16_config(const void *x, const void *w, void *y, int y_dtype, int64_t batch,
                        int64_t in_features, int64_t out_features, const tmc_gemv_config *config,
                        void *stream);

/* The configuration tmc_gemv_f16 / tmc_gate_up_silu_f16 pick for a shape. */
int tmc_gemv_default_config(int64_t batch, int64_t in_features, int64_t out_features, int gated,
                            tmc_gemv_config *out);

/* Skinny GEMM with fp16 MFMA (v_mfma_f32_16x16x32_f16), any batch >= 1;
 * same semantics as tmc_gemv_f16.  No reference counterpart: the reference
 * batched decode runs emitDecodeGEMV per row (ServingRuntime.cpp:281-291). */
int tmc_skinny_gemm_f16_mfma(const void *x, const void *w, void *y, int y_dtype,
                             int64_t batch, int64_t in_features, int64_t out_features,
                             void *stream);

/* Gated MLP, emitDecoderGatedMLP (DecoderLLMMetalEmitter.cpp:479-536):
 * out[r,f] = h(h(silu(h(g))) * h(u)) with g = x.Wg[f], u = x.Wu[f] and h()
 * the fp16 rounding; Wg, Wu are [intermediate, hidden]. */
int tmc_gate_up_silu_f16(const void *x, const void *w_gate, const void *w_up, void *out,
                         int64_t batch, int64_t hidden, int64_t intermediate, void *stream);
int tmc_gate_up_silu_f16_config(const void *x, const void *w_gate, const void *w_up, void *out,
                                int64_t batch, int64_t hidden, int64_t intermediate,
                                const tmc_gemv_config *config, void *stream);

/* Batch-1 decode GEMV / gated MLP with the preceding Add+RMSNorm folded in
 * (emitDecoderResidualRMSNorm, DecoderLLMMetalEmitter.cpp:417-477, then
 * emitDecodeGEMV / emitDecoderGatedMLP): x = h(s * rsqrt(mean(s^2) + eps) *
 * gamma) with s = h(residual + update) written to sum_out, or s = residual
 * when update is NULL (plain RMSNorm; sum_out unused).  Each block computes
 * the row's sum of squares itself (its four waves share the row's 64-chunk
 * groups, then one barrier) in the order of tmc_add_rmsnorm_threads /
 * tmc_rmsnorm_threads with one 16-byte chunk per thread, so x equals those
 * kernels' output bit for bit at any thread count >= in_features / 8 (the
 * 512-thread norm the batch-1 decoder runs at hidden 4096).  batch must be 1;
 * in_features a multiple of 8 up to 8192; all operands 16-byte aligned; fp16
 * operands.  config: NULL / algorithm 0 = the GEMV's default for the shape,
 * else a dot configuration (algorithm 1). */
int tmc_add_rmsnorm_gemv_f16(const void *residual, const void *update, const void *gamma,
                             const void *w, void *sum_out, void *y, int y_dtype, int64_t batch,
                             int64_t in_features, int64_t out_features, float epsilon,
                             const tmc_gemv_config *config, void *stream);
int tmc_add_rmsnorm_gate_up_silu_f16(const void *residual, const void *update, const void *gamma,
                                     const void *w_gate, const void *w_up, void *sum_out,
                                     void *out, int64_t batch, int64_t hidden,
                                     int64_t intermediate, float epsilon,
                                     const tmc_gemv_config *config, void *stream);

/* Batch-1 GEMV with the residual add in its epilogue (emitLinearResidual,
 * DecoderLLMMetalEmitter.cpp:604-622): y = h(h(W x) + residual), the fp16
 * rounding of the projection kept, so y equals tmc_gemv_f16 followed by
 * tmc_add bit for bit.  The batch-1 decoder runs its o and down projections
 * through it and folds the following norms into the next GEMV's prologue.
 * batch must be 1; in_features a multiple of 8; x and W 16-byte aligned.
 * config: NULL / algorithm 0 = tmc_gemv_f16's default for the shape, else a
 * dot configuration (algorithm 1) or the persistent dot (algorithm 5). */
int tmc_gemv_residual_f16(const void *x, const void *w, const void *residual, void *y,
                          int64_t batch, int64_t in_features, int64_t out_features,
                          const tmc_gemv_config *config, void *stream);

/* Activation layouts of the batch > 1 GEMM path.  TMC_LAYOUT_X_PACKED: the
 * GEMM's activations x [batch, in] are in fragment order; TMC_LAYOUT_Y_PACKED:
 * the kernel writes its fp16 output in fragment order (for the next GEMM).
 * Fragment order of A [rows, cols]: 16-row pass r / 16, 32-column chunk
 * c / 32, lane r % 16 + 16 * ((c % 32) / 8), element c % 8 -- the A operand of
 * v_mfma_f32_16x16x32_f16 -- at ((r / 16) * ceil(cols / 32) + c / 32) * 1024
 * bytes; rows past `rows` and columns past `cols` inside the last pass and
 * chunk are never read. */
#define TMC_LAYOUT_X_PACKED 1
#define TMC_LAYOUT_Y_PACKED 2
int64_t tmc_packed_activation_elements(int64_t rows, int64_t cols);
/* Reorder row-major fp16 activations into fragment order (and back with
 * `unpack` != 0). */
int tmc_pack_activations_f16(const void *src, void *dst, int64_t rows, int64_t cols, int unpack,
                             void *stream);

/* tmc_add_rmsnorm (update != NULL) or tmc_rmsnorm (update == NULL; sum_out
 * unused) with a layout: 0 = row-major, TMC_LAYOUT_Y_PACKED = the normalized
 * rows in fragment order (fp16, width % 8 == 0, width <= 8192, 16-byte
 * aligned operands); the sum stays row-major. */
int tmc_add_rmsnorm_ex(const void *residual, const void *update, const void *w, void *sum_out,
                       void *norm_out, int dtype, int64_t rows, int64_t width, float epsilon,
                       int layout, void *stream);

/* Fragment-packed weights for the batch > 1 skinny GEMM.  No reference
 * counterpart (the reference streams row-major weights, DecodeGEMVMetalEmitter
 * .cpp:68-132): a one-time repacking of W [out, in] row-major into tiles of
 * 16 rows x 32 k, each 64 lanes x 8 halves in the B-operand order of
 * v_mfma_f32_16x16x32_f16 (lane = n % 16 + 16 * ((k % 32) / 8), element
 * k % 8), tile (n / 16, k / 32) at ((n / 16) * ceil(in / 32) + k / 32) * 1024
 * bytes, zero-padded.  tmc_packed_weight_elements gives the packed fp16
 * element count (0 for a bad shape). */
int64_t tmc_packed_weight_elements(int64_t out_features, int64_t in_features);
int tmc_pack_weights_f16(const void *w, void *packed, int64_t out_features, int64_t in_features,
                         void *stream);
/* The same with gamma [in_features] folded in: element (n, k) is stored as
 * fp16(W[n, k] * gamma[k]) (gamma NULL: tmc_pack_weights_f16).  The weights
 * of the tmc_*_packed_norm_f16 entry points. */
int tmc_pack_weights_scaled_f16(const void *w, const void *gamma, void *packed,
                                int64_t out_features, int64_t in_features, void *stream);

/* tmc_gemv_f16 / tmc_gate_up_silu_f16 semantics over packed weights, any
 * batch (16 rows per pass); in_features % 8 == 0, x and the packed buffers
 * 16-byte aligned.  config (may be NULL): algorithm 0 = default for the shape,
 * otherwise unroll 1|2|4 K tiles of 128 in flight and k_split 1..16 waves
 * per 16-row output tile. */
int tmc_gemm_packed_f16(const void *x, const void *packed_w, void *y, int y_dtype, int64_t batch,
                        int64_t in_features, int64_t out_features, const tmc_gemv_config *config,
                        void *stream);
int tmc_gate_up_silu_packed_f16(const void *x, const void *packed_gate, const void *packed_up,
                                void *out, int64_t batch, int64_t hidden, int64_t intermediate,
                                const tmc_gemv_config *config, void *stream);
/* The same with activation layouts (TMC_LAYOUT_* bits): x packed, and/or
 * an fp16 output written packed. */
int tmc_gemm_packed_ex_f16(const void *x, const void *packed_w, void *y, int y_dtype,
                           int64_t batch, int64_t in_features, int64_t out_features, int layout,
                           const tmc_gemv_config *config, void *stream);
int tmc_gate_up_silu_packed_ex_f16(const void *x, const void *packed_gate, const void *packed_up,
                                   void *out, int64_t batch, int64_t hidden, int64_t intermediate,
                                   int layout, const tmc_gemv_config *config, void *stream);

/* Batched decode fusion of the q.k.v projection over fragment-packed
 * weights (tmc_gemm_packed_ex_f16, same defaults and configs) with
 * tmc_decode_rope_append: the projection rows are never stored; each output
 * feature pair of request b is rounded to fp16, rotated (q, k) and written
 * to q_out [batch, q_heads*head_dim] or into the pools through block_tables
 * [batch, max_pages] at position valid_lengths[b]-1, with the bits of the
 * two-kernel sequence.  layout: 0 or TMC_LAYOUT_X_PACKED.  Same skip rules
 * as tmc_decode_rope_append. */
int tmc_qkv_rope_append_packed_f16(const void *x, const void *packed_w, const float *cosine,
                                   const float *sine, const int32_t *valid_lengths,
                                   const int32_t *block_tables, const int32_t *active_count,
                                   void *q_out, void *key_pool, void *value_pool, int64_t batch,
                                   int64_t hidden, int64_t q_heads, int64_t kv_heads,
                                   int64_t head_dim, int64_t capacity, int64_t page_size,
                                   int64_t max_pages, int layout, const tmc_gemv_config *config,
                                   void *stream);

/* Batched decode with the RMSNorm folded into the packed projection
 * (emitDecoderRMSNorm, DecoderLLMMetalEmitter.cpp:63-108, applied in the
 * projection as the fusion candidate emitDecoderQKVFusion :538-602 does):
 * x is the un-normalized residual stream s [batch, in]; packed_w holds
 * W . diag(gamma) (tmc_pack_weights_scaled_f16 with the norm's gamma); row r
 * of the product is scaled by 1 / sqrt(sum_k s[r, k]^2 / in + epsilon)
 * before the epilogue (fp16 / fp32 store, SiLU gating, RoPE + append), the
 * squares taken from the activation fragments the MFMA reads.  The fp16
 * rounding falls on W * gamma instead of the normalized value, so the
 * result matches RMSNorm followed by the plain entry point within the fp16
 * path tolerance, not bit for bit.  epsilon > 0; config k_split at most 4
 * (the default is clamped there).  Arguments otherwise as the entry points
 * above. */
int tmc_gemm_packed_norm_f16(const void *x, const void *packed_w, void *y, int y_dtype,
                             int64_t batch, int64_t in_features, int64_t out_features,
                             float epsilon, int layout, const tmc_gemv_config *config,
                             void *stream);
int tmc_gate_up_silu_packed_norm_f16(const void *x, const void *packed_gate,
                                     const void *packed_up, void *out, int64_t batch,
                                     int64_t hidden, int64_t intermediate, float epsilon,
                                     int layout, const tmc_gemv_config *config, void *stream);
int tmc_rmsnorm_qkv_rope_append_packed_f16(const void *x, const void *packed_w,
                                           const float *cosine, const float *sine,
                                           const int32_t *valid_lengths,
                                           const int32_t *block_tables,
                                           const int32_t *active_count, void *q_out,
                                           void *key_pool, void *value_pool, int64_t batch,
                                           int64_t hidden, int64_t q_heads, int64_t kv_heads,
                                           int64_t head_dim, int64_t capacity, int64_t page_size,
                                           int64_t max_pages, float epsilon, int layout,
                                           const tmc_gemv_config *config, void *stream);
/* emitLinearResidual (DecoderLLMMetalEmitter.cpp:604-621) over packed
 * weights, any batch: y = fp16(fp16(x W^T) + residual), residual [batch, out]
 * in y's layout (TMC_LAYOUT_Y_PACKED: the packed activation order). */
int tmc_gemm_packed_residual_f16(const void *x, const void *packed_w, const void *residual,
                                 void *y, int64_t batch, int64_t in_features,
                                 int64_t out_features, int layout, const tmc_gemv_config *config,
                                 void *stream);

/* emitDecoderRMSNorm (DecoderLLMMetalEmitter.cpp:63-108) / emitRMSNorm
 * (MetalEmitter.cpp:12-76): y = x * rsqrt(mean(x^2) + eps) * w, fp32
 * reduction, dtype TMC_F16 or TMC_F32 for x, w, y. */
int tmc_rmsnorm(const void *x, const void *w, void *y, int dtype, int64_t rows, int64_t width,
                float epsilon, void *stream);

/* emitDecoderResidualRMSNorm (DecoderLLMMetalEmitter.cpp:417-477):
 * s = h(r + u) written to sum_out, n = h(s * rsqrt(mean(s^2)+eps) * w). */
int tmc_add_rmsnorm(const void *residual, const void *update, const void *w, void *sum_out,
                    void *norm_out, int dtype, int64_t rows, int64_t width, float epsilon,
                    void *stream);

/* RMSNorm / Add+RMSNorm at a chosen workgroup size: the RMSNorm tuner's
 * candidates (emitRMSNorm(op, threads), MetalEmitter.cpp:12-76, and its
 * baseline emitRMSNormBaseline, RMSNormBaseline.cpp:13-72, retargeted to
 * gfx950).  threads is 64, 128, 256, 512 or 1024 (0 = 256).  variant 0 keeps
 * the row in registers when width % 8 == 0 and width <= 32 * threads (one
 * read pass), else reads it twice; variant 1 always runs the two-pass kernel
 * (at 256 threads, the tuner's fixed baseline).  Same results as
 * tmc_rmsnorm / tmc_add_rmsnorm up to fp32 summation order. */
int tmc_rmsnorm_threads(const void *x, const void *w, void *y, int dtype, int64_t rows,
                        int64_t width, float epsilon, int threads, int variant, void *stream);
int tmc_add_rmsnorm_threads(const void *residual, const void *update, const void *w,
                            void *sum_out, void *norm_out, int dtype, int64_t rows, int64_t width,
                            float epsilon, int threads, int variant, void *stream);

/* emitDecoderSiLUMul (DecoderLLMMetalEmitter.cpp:395-415):
 * out = h(h(g / (1 + exp(-g))) * u). */
int tmc_silu_mul(const void *gate, const void *up, void *out, int dtype, int64_t count,
                 void *stream);

/* emitDecoderAdd (DecoderLLMMetalEmitter.cpp:375-393): out = h(a + b). */
int tmc_add(const void *a, const void *b, void *out, int dtype, int64_t count, void *stream);

/* Element-wise kernels of the graph path with a chosen workgroup size (64,
 * 128 or 256): op 0 Add h(a + b), 1 Mul h(a * b), 2 SiLU h(a / (1 + exp(-a)))
 * (b unused, may be NULL), 3 the fused SiLU + Mul region
 * (FusionMetalEmitter.cpp:103-210), equal to op 2 followed by op 1.  The
 * graph executor's baseline and fused-region kernels. */
int tmc_elementwise(int op, const void *a, const void *b, void *out, int dtype, int64_t count,
                    int threads, void *stream);

/* emitDecoderEmbedding (DecoderLLMMetalEmitter.cpp:35-61): out[r] =
 * table[token[r]]; an out-of-range token leaves its row untouched. */
int tmc_embedding(const int32_t *tokens, const void *table, void *out, int dtype, int64_t rows,
                  int64_t hidden, int64_t vocabulary, void *stream);

/* emitDecoderRoPE (DecoderLLMMetalEmitter.cpp:110-158): x token-major
 * [batch, seq, heads*D], fp32 tables [capacity, D/2], position
 * valid - seq + t with valid read from valid_length[0]; out head-major
 * [batch, heads, seq, D].  valid < seq or valid > capacity: no-op. */
int tmc_rope(const void *x, const float *cosine, const float *sine,
             const int32_t *valid_length, void *out, int dtype, int64_t batch, int64_t seq,
             int64_t heads, int64_t head_dim, int64_t capacity, void *stream);

/* emitServingRoPE (DecoderLLMMetalEmitter.cpp:260-312): one token per
 * request, position valid_lengths[r] - 1, requests >= active_count[0] and
 * invalid lengths skipped; out [max_batch, heads, D]. */
int tmc_serving_rope(const void *x, const float *cosine, const float *sine,
                     const int32_t *valid_lengths, const int32_t *active_count, void *out,
                     int dtype, int64_t max_batch, int64_t heads, int64_t head_dim,
                     int64_t capacity, void *stream);

/* emitDecoderCacheAppend (DecoderLLMMetalEmitter.cpp:160-203): bit copy of
 * seq tokens into a contiguous cache [batch, heads, capacity, D] at
 * positions valid-seq..valid-1. `head_major` selects the input layout. */
int tmc_kv_append(const void *input, const int32_t *valid_length, void *cache, int dtype,
                  int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, int64_t capacity,
                  int head_major, void *stream);

/* emitDecoderPagedCacheAppend (DecoderLLMMetalEmitter.cpp:205-258): cache
 * pages [page][batch][heads][page_size][D] through block_table[pos/page]. */
int tmc_paged_kv_append(const void *input, const int32_t *valid_length,
                        const int32_t *block_table, void *cache, int dtype, int64_t batch,
                        int64_t seq, int64_t heads, int64_t head_dim, int64_t capacity,
                        int64_t page_size, int head_major, void *stream);

/* emitServingPagedCacheAppend (DecoderLLMMetalEmitter.cpp:314-373): one
 * token per request into pool pages [page][heads][page_size][D] through
 * block_tables[r*max_pages + pos/page]. */
int tmc_serving_kv_append(const void *input, const int32_t *valid_lengths,
                          const int32_t *block_tables, const int32_t *active_count, void *cache,
                          int dtype, int64_t max_batch, int64_t heads, int64_t head_dim,
                          int64_t capacity, int64_t page_size, int head_major, void *stream);

/* Bytes of device workspace the split-KV attention needs for these limits
 * (0 when none is needed).  Layout, the same for every head size: int32
 * arrival counters, one per (request, kv head), in a fixed 64 KiB area at
 * the start (batch * kv_heads * 4 bytes rounded up to 256 when that is
 * larger), then one (weighted[D], max, sum) fp32 partial per request, query
 * head and split.  For head_dim 128 the last split block of a row merges the
 * row's partials in the same launch and resets its counter.  The workspace
 * must be zero before its first use; every launch leaves the counters at
 * zero and no launch's partials overlap the counter area, so one workspace
 * serves launches of different shapes in any order when it is large enough
 * for each and batch * kv_heads <= 16384 for all of them (a larger shape
 * needs a workspace of its own).  Launches that share one workspace must not
 * overlap. */
size_t tmc_attention_workspace_bytes(int64_t batch, int64_t q_heads, int64_t kv_heads,
                                     int64_t head_dim, int64_t capacity);

/* Decode attention over a contiguous cache (emitKVAttention,
 * KVCacheMetalEmitter.cpp:119-208, queryLength 1): caches
 * [batch, kv_heads, capacity, D], q [batch, q_heads, D], out
 * [batch, q_heads*D]; attends [0, valid_length[0]); query head h reads kv
 * head h / (q_heads/kv_heads).  valid < 1 or > capacity: no-op. */
int tmc_decode_attention(const void *q, const void *key_cache, const void *value_cache,
                         const int32_t *valid_length, void *out, int dtype, int64_t batch,
                         int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t capacity,
                         void *workspace, size_t workspace_bytes, void *stream);

/* Paged decode attention (emitServingPagedKVAttention,
 * KVCacheMetalEmitter.cpp:312-406, generalised to GQA): element
 * (page, kvh, offset, d) at page*page_stride + kvh*head_stride +
 * offset*D + d; request r attends [0, valid_lengths[r]) through
 * block_tables[r*max_pages + pos/page_size].  pool_pages is the number of
 * pages each pool holds (0 = unknown); a page id at or past it counts as
 * missing.  Requests >= active_count[0] (active_count may be NULL = all),
 * invalid lengths, or a missing (negative) page in range leave their output
 * untouched.  No counterpart of pool_pages in the reference: it bounds every
 * pool access the kernel makes. */
int tmc_paged_decode_attention(const void *q, const void *key_pool, const void *value_pool,
                               const int32_t *valid_lengths, const int32_t *block_tables,
                               const int32_t *active_count, void *out, int dtype,
                               int64_t max_batch, int64_t q_heads, int64_t kv_heads,
                               int64_t head_dim, int64_t page_size, int64_t max_pages,
                               int64_t pool_pages, int64_t page_stride, int64_t head_stride,
                               void *workspace, size_t workspace_bytes, void *stream);

/* The same with an output layout: 0 = out [max_batch, q_heads*D] row-major,
 * TMC_LAYOUT_Y_PACKED = out in the packed activation order
 * (tmc_packed_activation_elements(max_batch, q_heads*D) fp16 elements,
 * 16-byte aligned), so that the o projection reads it as packed activations
 * (tmc_gemm_packed_residual_f16 with TMC_LAYOUT_X_PACKED).  No counterpart in the
 * reference, whose attention output feeds a GEMV in row-major order. */
int tmc_paged_decode_attention_ex(const void *q, const void *key_pool, const void *value_pool,
                                  const int32_t *valid_lengths, const int32_t *block_tables,
                                  const int32_t *active_count, void *out, int dtype,
                                  int64_t max_batch, int64_t q_heads, int64_t kv_heads,
                                  int64_t head_dim, int64_t page_size, int64_t max_pages,
                                  int64_t pool_pages, int64_t page_stride, int64_t head_stride,
                                  void *workspace, size_t workspace_bytes, int layout,
                                  void *stream);

/* tmc_paged_decode_attention without a workspace argument and without any
 * allocation.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The split partials live in a
 * static device array of tmc_attention_scratch_bytes() (16 MiB) per GPU,
 * held until the process ends; limits whose tmc_attention_workspace_bytes()
 * exceed it are rejected with an error before any launch.  All calls on one
 * GPU share that array: calls that overlap on one GPU (different streams,
 * different host threads) race and must be serialised by the caller.  Each
 * call writes every partial it reads, and the merge counters (zero when the
 * library loads) are left at zero after every call, so nothing needs
 * clearing between calls.  Same arguments, results and errors as
 * tmc_paged_decode_attention otherwise. */
int tmc_paged_decode_attention_noalloc(const void *q, const void *key_pool,
                                       const void *value_pool, const int32_t *valid_lengths,
                                       const int32_t *block_tables, const int32_t *active_count,
                                       void *out, int dtype, int64_t max_batch, int64_t q_heads,
                                       int64_t kv_heads, int64_t head_dim, int64_t page_size,
                                       int64_t max_pages, int64_t pool_pages, int64_t page_stride,
                                       int64_t head_stride, void *stream);
/* Bytes of the static scratch behind tmc_paged_decode_attention_noalloc. */
size_t tmc_attention_scratch_bytes(void);

/* Paged attention + output projection for one decode token (batch 1), the
 * fusion candidate emitPagedAttentionOutputProjection
 * (DecoderLLMMetalEmitter.cpp:623-698, queryLength 1) with the residual add
 * of emitLinearResidual (:604-621):
 *   context = paged attention of request 0 (as tmc_paged_decode_attention,
 *             rounded to fp16 as that kernel stores it),
 *   y[n]    = fp16(fp16(sum_k weight[n, k] * context[k]) + residual[n]),
 * or y[n] = fp16(sum) when residual is NULL.  weight is
 * [out_features, q_heads*128] row-major fp16.  Limits: head_dim 128,
 * q_heads / kv_heads 1 or 2, pages of a multiple of 16 positions,
 * page_size * max_pages <= 1024, pool_pages > 0 with each pool below 4 GiB,
 * out_features a multiple of 128 (64 when q_heads = 2 * kv_heads).  An
 * inactive request (active_count[0] < 1), an invalid length or a missing page
 * leaves y untouched.  The sum over k is taken per kv head and the kv heads'
 * sums are added in head order: the result is deterministic.
 * workspace: tmc_attention_output_workspace_bytes() bytes, zeroed once
 * before the first call; it starts with per-slice arrival counters, which
 * every call leaves at zero again.  Calls that share a workspace must not
 * overlap.  Measured slower than tmc_paged_decode_attention followed by
 * tmc_gemv_residual_f16 on MI355X (14.6 against 13.1 us at Llama-7B widths,
 * 132 positions), so the decoder keeps the two launches by default. */
size_t tmc_attention_output_workspace_bytes(int64_t q_heads, int64_t kv_heads,
                                            int64_t out_features);
int tmc_paged_attention_output_f16(const void *q, const void *key_pool, const void *value_pool,
                                   const int32_t *valid_lengths, const int32_t *block_tables,
                                   const int32_t *active_count, const void *weight,
                                   const void *residual, void *y, int64_t q_heads,
                                   int64_t kv_heads, int64_t head_dim, int64_t page_size,
                                   int64_t max_pages, int64_t pool_pages, int64_t page_stride,
                                   int64_t head_stride, int64_t out_features, void *workspace,
                                   size_t workspace_bytes, void *stream);

/* Decode-step fusion of emitServingRoPE (DecoderLLMMetalEmitter.cpp:260-312)
 * for q and k with emitServingPagedCacheAppend (:314-373) for the rotated k
 * and v, reading one fused projection row per request laid out
 * [q_heads | kv_heads (key) | kv_heads (value)] x head_dim.  The token of
 * request b sits at position valid_lengths[b]-1: the rotated query goes to
 * q_out [max_batch, q_heads*head_dim]; the rotated key and the value (bit
 * copy) go to the pools [page][kv_heads][page_size][head_dim] through
 * block_tables [max_batch, max_pages], max_pages = ceil(capacity/page_size).
 * Rows >= active_count[0], lengths outside [1, capacity] and negative page
 * entries are skipped.  The rotation is bit-identical to tmc_serving_rope. */
int tmc_decode_rope_append(const void *qkv, const float *cosine, const float *sine,
                           const int32_t *valid_lengths, const int32_t *block_tables,
                           const int32_t *active_count, void *q_out, void *key_pool,
                           void *value_pool, int dtype, int64_t max_batch, int64_t q_heads,
                           int64_t kv_heads, int64_t head_dim, int64_t capacity,
                           int64_t page_size, int64_t max_pages, void *stream);

/* Batch-1 decode fusion of the q.k.v projection (emitDecodeGEMV,
 * DecodeGEMVMetalEmitter.cpp:68-132, over the fused [q | k | v] weight
 * [(q_heads + 2*kv_heads)*head_dim, hidden]) with tmc_decode_rope_append for
 * its one request: the projection row is never stored; each pair of output
 * features is rounded to fp16, rotated (q, k) and written to q_out, or into
 * the pools through block_table [max_pages] at position valid_lengths[0]-1,
 * with the bits tmc_gemv_f16 followed by tmc_decode_rope_append produce.
 * config: NULL or algorithm 0 for the default, else the dot algorithm with
 * rows_per_wave 2 (a wave owns one pair).  Same skip rules as
 * tmc_decode_rope_append (active_count[0] < 1, length outside [1, capacity],
 * negative page). */
int tmc_qkv_rope_append_f16(const void *x, const void *w, const float *cosine, const float *sine,
                            const int32_t *valid_lengths, const int32_t *block_table,
                            const int32_t *active_count, void *q_out, void *key_pool,
                            void *value_pool, int64_t hidden, int64_t q_heads, int64_t kv_heads,
                            int64_t head_dim, int64_t capacity, int64_t page_size,
                            const tmc_gemv_config *config, void *stream);

/* tmc_qkv_rope_append_f16 of x = RMSNorm(residual + update) * gamma (update
 * NULL: RMSNorm(residual) * gamma), the norm computed in each block as
 * tmc_add_rmsnorm_gemv_f16 computes it (bit-identical to tmc_add_rmsnorm /
 * tmc_rmsnorm with one 16-byte chunk per thread; emitDecoderResidualRMSNorm,
 * DecoderLLMMetalEmitter.cpp:417-477); with an update, sum_out receives
 * h(residual + update).  hidden at most 8192.  The batch-1 decoder runs it
 * (update NULL) on the residual stream that tmc_gemv_residual_f16 wrote. */
int tmc_add_rmsnorm_qkv_rope_append_f16(const void *residual, const void *update,
                                        const void *gamma, const void *w, void *sum_out,
                                        const float *cosine, const float *sine,
                                        const int32_t *valid_lengths, const int32_t *block_table,
                                        const int32_t *active_count, void *q_out, void *key_pool,
                                        void *value_pool, int64_t hidden, int64_t q_heads,
                                        int64_t kv_heads, int64_t head_dim, int64_t capacity,
                                        int64_t page_size, float epsilon,
                                        const tmc_gemv_config *config, void *stream);

/* The chunk-prefill form of tmc_decode_rope_append: every row is a token of
 * one request, so the rows share one block table [max_pages]; row r's token
 * sits at position valid_lengths[r]-1 (causal chunk: start + r + 1).  Stage
 * building of prefillChunked (DecoderLLMExecutor.cpp:982-1034) with the
 * RoPE and cache append of emitServingRoPE / emitServingPagedCacheAppend. */
int tmc_prefill_rope_append(const void *qkv, const float *cosine, const float *sine,
                            const int32_t *valid_lengths, const int32_t *block_table,
                            const int32_t *active_count, void *q_out, void *key_pool,
                            void *value_pool, int dtype, int64_t rows, int64_t q_heads,
                            int64_t kv_heads, int64_t head_dim, int64_t capacity,
                            int64_t page_size, int64_t max_pages, void *stream);

/* Several requests in one prefill chunk: row r uses table row row_table[r]
 * of block_tables [table_rows, max_pages]; rows whose entry is outside
 * [0, table_rows) are skipped.  Otherwise as tmc_prefill_rope_append. */
int tmc_prefill_rope_append_rows(const void *qkv, const float *cosine, const float *sine,
                                 const int32_t *valid_lengths, const int32_t *block_tables,
                                 const int32_t *row_table, int64_t table_rows,
                                 const int32_t *active_count, void *q_out, void *key_pool,
                                 void *value_pool, int dtype, int64_t rows, int64_t q_heads,
                                 int64_t kv_heads, int64_t head_dim, int64_t capacity,
                                 int64_t page_size, int64_t max_pages, void *stream);

/* emitTiledGEMM (DecodeGEMVMetalEmitter.cpp:134-169), the prefill linear
 * layer: y[m, n] = x[m, k] weight[n, k]^T, fp16 inputs, fp32 accumulation,
 * y fp16 or fp32 (out_dtype), all row-major, on the hand-written gfx950 MFMA
 * GEMM (v_mfma_f32_16x16x32_f16, 128 x 128 output tiles per 256-thread
 * workgroup; k a multiple of 8, x and weight 16-byte aligned and each below
 * 4 GiB).  When the output tiles alone would leave CUs idle and the
 * workspace holds the fp32 partials, K is split over several workgroups and
 * a second launch adds the partials in split order.  workspace may be NULL
 * with workspace_bytes 0 (no split); tmc_gemm_rows_workspace_bytes() is the
 * size the decoder binds (32 MiB).  Calls that share a workspace must be
 * ordered on one stream.  Nothing is timed or allocated; calls may be
 * captured in a graph. */
size_t tmc_gemm_rows_workspace_bytes(void);
/* tmc_gemm_rows_f16 without a workspace (never splits K). */
int tmc_gemm_mfma_f16(const void *x, const void *weight, void *y, int out_dtype, int64_t m,
                      int64_t k, int64_t n, void *stream);
int tmc_gemm_rows_f16(const void *x, const void *weight, void *y, int out_dtype, int64_t m,
                      int64_t k, int64_t n, void *workspace, size_t workspace_bytes,
                      void *stream);

/* emitPagedKVAttention with causalPrefill (KVCacheMetalEmitter.cpp:210-310,
 * attended = valid - S + q + 1): query token r of a chunk (q [rows, q_heads,
 * D], RoPE applied) attends positions [0, valid_lengths[r]) of one request's
 * pages (block_table [max_pages]; pools [pages][kv_heads][page_size][D] with
 * the given strides in elements); out [rows, q_heads, D].  Rows >=
 * active_count[0] and lengths outside [1, page_size * max_pages] are left
 * untouched, as is a row whose range reaches a page entry outside
 * [0, pool_pages).  D is 64 or 128; q_heads / kv_heads must divide 64. */
int tmc_prefill_attention_f16(const void *q, const void *key_pool, const void *value_pool,
                              const int32_t *valid_lengths, const int32_t *block_table,
                              const int32_t *active_count, void *out, int64_t rows,
                              int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                              int64_t page_size, int64_t max_pages, int64_t pool_pages,
                              int64_t page_stride, int64_t head_stride, void *stream);

/* Several requests in one prefill chunk: the rows are cut into tiles of
 * 64 / (q_heads / kv_heads) tokens and a tile uses table row
 * row_table[first row of the tile] of block_tables [table_rows, max_pages];
 * a caller packing several requests starts each request at a tile boundary
 * (a row of another table row inside a tile is left untouched).  With
 * row_table NULL, table_rows must be 1 (tmc_prefill_attention_f16). */
int tmc_prefill_attention_rows_f16(const void *q, const void *key_pool, const void *value_pool,
                                   const int32_t *valid_lengths, const int32_t *block_tables,
                                   const int32_t *row_table, int64_t table_rows,
                                   const int32_t *active_count, void *out, int64_t rows,
                                   int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                   int64_t page_size, int64_t max_pages, int64_t pool_pages,
                                   int64_t page_stride, int64_t head_stride, void *stream);

/* emitTokenArgmax (TransformerDecodeMetalEmitter.cpp:198-256): greedy token
 * per row over fp32 logits, ties to the lowest index. */
int tmc_argmax_f32(const float *logits, int32_t *tokens, int64_t rows, int64_t vocabulary,
                   void *stream);

/* Chained greedy decode, queued between two step graphs: for r < rows,
 * tokens[r] = history[r] = next_tokens[r] and lengths[r] += 1 (history and
 * lengths may be null).  No counterpart in the reference, whose steps return
 * to the host: it replaces three queued copies per step (tokens, history,
 * lengths) with one launch. */
int tmc_decode_chain(const int32_t *next_tokens, int32_t *tokens, int32_t *lengths,
                     int32_t *history, int64_t rows, void *stream);

/* Token-only LM head (the decode step's tail when no logits are read,
 * DecoderLLMExecutor.cpp:837-845,929-930): a partial pass computes the LM
 * head's logits and keeps, per block, the greatest (value, index) in the
 * greedy-token order (ties to the lowest index, NaN never selected) in a
 * workspace of partial slots; the final pass folds each row's slots into its
 * token.  The tokens equal tmc_argmax_f32 over the logits the same LM head
 * writes.  Workspace layout: int32 slot count at byte 0, fp32 values
 * [rows][vocabulary] from byte 256, then int32 indices [rows][vocabulary]. */
size_t tmc_lm_head_argmax_workspace_bytes(int64_t rows, int64_t vocabulary);

/* emitLMHeadPartialArgmax (DecoderLLMMetalEmitter.cpp:700-728) for batch 1
 * with the final RMSNorm folded in, as tmc_add_rmsnorm_gemv_f16 without an
 * update: logits of W [vocabulary, in_features] times the normalized
 * residual, reduced to partial slots. */
int tmc_rmsnorm_lm_head_partial_argmax_f16(const void *residual, const void *gamma,
                                           const void *w, void *workspace, size_t workspace_bytes,
                                           int64_t in_features, int64_t vocabulary, float epsilon,
                                           const tmc_gemv_config *config, void *stream);

/* emitLMHeadPartialArgmax for batch > 1 on fragment-packed weights with the
 * final norm folded in (as tmc_gemm_packed_norm_f16 with an fp32 output;
 * layout 0 or TMC_LAYOUT_X_PACKED): one slot per 16-row tile of W per
 * batch row. */
int tmc_lm_head_partial_argmax_packed_norm_f16(const void *x, const void *packed_w,
                                               void *workspace, size_t workspace_bytes,
                                               int64_t batch, int64_t in_features,
                                               int64_t vocabulary, float epsilon, int layout,
                                               const tmc_gemv_config *config, void *stream);

/* emitLMHeadFinalArgmax (DecoderLLMMetalEmitter.cpp:730-753): tokens[row]
 * from the row's partial slots. */
int tmc_lm_head_final_argmax(void *workspace, size_t workspace_bytes, int32_t *tokens,
                             int64_t rows, int64_t vocabulary, void *stream);

/* Pinned host memory (hipHostMalloc), readable and writable by kernels:
 * the spill space of preempted requests' KV pages.  No reference counterpart
 * (the reference snapshots float vectors, ServingRuntime.cpp:426-930). */
int tmc_host_alloc(size_t bytes, void **out);
void tmc_host_free(void *ptr);

/* Page-granular copies between a KV pool and a contiguous buffer (device or
 * pinned host): scatter == 0 gathers dst[i] = src page pages[i]; scatter != 0
 * writes dst page pages[i] = src[i]; i < count, each page page_bytes bytes
 * (a multiple of 16).  `pages` must be readable by the device (device or
 * pinned host memory) and hold ids below the pool's page count; bits are
 * copied unchanged. */
int tmc_copy_pages(const void *src, void *dst, const int32_t *pages, int64_t count,
                   int64_t page_bytes, int scatter, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TMC_HIP_H */
