/* Measurement helpers exported by libtmc_hip.so beside the decode backend.
 *
 * Not part of the drop-in boundary (include/tmc_hip.h): no reference
 * interface maps to them and no executor calls them.  bench.py, the tests and
 * the counter passes use them to make synthetic weights on the device and to
 * measure the ceilings the kernels are judged against.  Same conventions as
 * tmc_hip.h: 0 = success, tmc_last_error() holds the message otherwise. */
#ifndef TMC_BENCH_H
#define TMC_BENCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Synthetic data: fill `count` elements of dtype (TMC_F16 / TMC_F32 /
 * TMC_BF16) with N(mean, std) values from a counter-based generator
 * (splitmix64 + Box-Muller) keyed by `seed`. */
int tmc_fill_normal(void *ptr, int dtype, int64_t count, uint64_t seed, float mean, float std,
                    void *stream);

/* Plain device copy kernel: the streaming probe whose counter readings
 * calibrate FETCH_SIZE / WRITE_SIZE, and the practical HBM copy rate. */
int tmc_copy_bytes(const void *src, void *dst, size_t bytes, void *stream);

/* Read-only streaming probe: reads `bytes` of src once (4096 blocks, four
 * 16-byte non-temporal loads per lane in flight) and writes nothing but, when
 * a block's sum hits a fixed constant, the 4-byte `sink`.  Its duration is the
 * floor of any kernel that must read those bytes once in one launch (the
 * GEMVs read their weights exactly so). */
int tmc_read_probe(const void *src, size_t bytes, void *sink, void *stream);

/* Bandwidth probe of the paged attention access pattern (head_dim 128, pages
 * of a multiple of 16 positions): reads the K and V bytes
 * tmc_paged_decode_attention would read for these lengths and block tables,
 * and nothing else; `sink` (4 bytes of device memory) is written only when
 * the xor of the loaded words hits a fixed constant.  It measures the ceiling
 * of the gather itself, as tmc_copy_bytes does for streaming. */
int tmc_paged_gather_probe(const void *key_pool, const void *value_pool,
                           const int32_t *valid_lengths, const int32_t *block_tables,
                           int64_t batch, int64_t kv_heads, int64_t head_dim, int64_t page_size,
                           int64_t max_pages, int64_t pool_pages, int64_t page_stride,
                           int64_t head_stride, void *sink, void *stream);

/* Per-wave timestamps of the last launches of the 4-wave split-attention
 * kernel and the 8-wave one-split kernel (contiguous caches and 16-position
 * pages), for a library built with
 * TMC_ATTN_TIMELINE=1 (libtmc_hip_timeline.so): copies `waves` x 48 slots
 * (layout beside the switch in attention.hip) to the host array `events`,
 * after a device synchronize.  Other builds return an error.  No counterpart
 * in the reference: a diagnostic of this backend's decode attention. */
int tmc_attention_timeline(uint64_t *events, int64_t waves);

#ifdef __cplusplus
}
#endif

#endif /* TMC_BENCH_H */
