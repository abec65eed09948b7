// Chunked prefill for gfx950: the prompt GEMMs and causal paged attention
// over a chunk of one request's tokens.
//
// Reference: prefillChunked (DecoderLLMExecutor.cpp:982-1034) runs a stage
// whose linear layers are emitTiledGEMM (DecodeGEMVMetalEmitter.cpp:134-169,
// Y[m, n] = X[m, k] W[n, k]^T with fp32 accumulation) and whose attention is
// emitPagedKVAttention with causalPrefill (KVCacheMetalEmitter.cpp:210-310):
// query token q of a chunk of S tokens attends positions [0, valid - S + q + 1).
//
//  * the prompt projections are GEMMs with M = chunk tokens (gemm.hip).
//  * prefill_attention_kernel: one 256-thread workgroup per (kv head, tile of
//    64 query vectors = 64/G tokens x the G query heads of that kv head).
//    K/V blocks of 64 positions are staged through LDS (K row-major, V
//    transposed) and both products run on v_mfma_f32_16x16x32_f16: scores
//    transposed (S^T = K Q^T), so each lane owns one query column and the
//    softmax max is two cross-lane steps, and O^T = V^T P^T takes P^T
//    straight from the score registers (the k-slot order of both operands is
//    the same permutation of the 32 positions of a step).
#include "tmc_abi.hpp"
#include "tmc_device.hpp"

#include <cmath>
#include <mutex>
#include <vector>

namespace tmc {
namespace {

// ------------------------------------------------------------ prefill attention
constexpr int kPaThreads = 256;
constexpr int kPaWaves = kPaThreads / kWave;
constexpr int kPaVectors = 16 * kPaWaves;  // query vectors per workgroup
constexpr int kPaBlock = 64;               // positions per K/V block
constexpr int kKPad = 8;                   // halves of padding per K row in LDS
// V^T rows of 64 + 4 halves (34 dwords): the 16 lanes of one 8-byte LDS
// access phase (rows j = 0..15, 32 banks) land on distinct bank pairs; a
// 36-dword row stride puts rows j and j + 8 on the same banks.
constexpr int kVPad = 4;                   // halves of padding per V^T row in LDS
constexpr size_t kPaMaxLds = 64 * 1024;    // LDS per workgroup the launch stays within

struct PrefillParams {
  const half_t* q;       // [rows, q_heads, D]
  const half_t* k;       // pool [pages][kv_heads][page_size][D]
  const half_t* v;
  half_t* out;           // [rows, q_heads, D]
  const int32_t* valid;  // [rows] valid length of each query token
  const int32_t* table;  // [table_rows][max_pages] pages of the chunk's requests
  const int32_t* row_table;  // [rows] table row of each token, or null: row 0 for all
  int table_rows;
  const int32_t* active; // [1] query tokens present
  long page_stride, head_stride, pool_pages;
  unsigned pool_bytes;   // bytes of each pool when below 4 GiB (buffer loads), else 0
  int rows, q_heads, kv_heads, group, tokens_per_tile, tiles;
  int page_size, max_pages;
  int page_shift;        // log2(page_size) when it is a power of two, else -1
  float scale_log2;
};

// Per-thread share of one block: K as 16-byte chunks (item = position x
// chunk), V as items of 4 positions x 8 dims (item = quad + 16 * octet).
template <int D>
struct PaBlockRegs {
  static constexpr int kItems = kPaBlock * D / 8;
  static constexpr int vItems = (kPaBlock / 4) * (D / 8);
  static constexpr int kPer = (kItems + kPaThreads - 1) / kPaThreads;
  static constexpr int vPer = (vItems + kPaThreads - 1) / kPaThreads;
  h8 k[kPer];
  h8 v[4][vPer];
};

// Global loads of one 64-position block into registers (zero where the
// position is at or past `end` or its page is absent).  BUF (pools below
// 4 GiB): raw buffer loads with the out-of-range offset for absent data, so
// every load issues unconditionally; otherwise predicated global loads.
template <int D, bool BUF, bool OFFS>
__device__ __forceinline__ void pa_load(const PrefillParams& p, const int* table, int kvh, int base,
                                        int end, PaBlockRegs<D>& r) {
  using R = PaBlockRegs<D>;
  constexpr int CH = D / 8;  // 16-byte chunks per position
  const int tid = (int)threadIdx.x;
  __builtin_assume(tid < kPaThreads);
  const h8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  const __amdgpu_buffer_rsrc_t rk = buffer_resource(p.k, p.pool_bytes);
  const __amdgpu_buffer_rsrc_t rv = buffer_resource(p.v, p.pool_bytes);
  if constexpr (OFFS) {
    // `table` holds each page's byte offset for this kv head (kBufferAbsent
    // for an absent page) and the page size is a power of two of at least 4:
    // a 4-position V group lies in one page, so it costs one lookup.
    const int shift = p.page_shift, mask = p.page_size - 1;
    auto page_off = [&](int pos) -> unsigned {
      return (unsigned)table[pos < end ? pos >> shift : 0];
    };
#pragma unroll
    for (int i = 0; i < R::kPer; ++i) {
      const int item = tid + i * kPaThreads;
      const int pos = base + item / CH;
      const unsigned off = page_off(pos);
      const bool ok = pos < end && off != kBufferAbsent &&
                      (R::kItems % kPaThreads == 0 || item < R::kItems);
      r.k[i] = buffer_load_h8(
          rk, ok ? off + (unsigned)(((pos & mask) * D + 8 * (item % CH)) * 2) : kBufferAbsent);
    }
#pragma unroll
    for (int i = 0; i < R::vPer; ++i) {
      const int item = tid + i * kPaThreads;
      const int quad = item % (kPaBlock / 4), octet = item / (kPaBlock / 4);
      const int pos0 = base + 4 * quad;
      const unsigned off = page_off(pos0);
      const unsigned row0 = off + (unsigned)(((pos0 & mask) * D + 8 * octet) * 2);
      const bool group_ok = off != kBufferAbsent && (R::vItems % kPaThreads == 0 || item < R::vItems);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        r.v[q][i] = buffer_load_h8(
            rv, group_ok && pos0 + q < end ? row0 + (unsigned)(q * D * 2) : kBufferAbsent);
    }
    return;
  }
  const bool pow2 = p.page_shift >= 0;
  // Element offset of (pos, 8-element column), or -1 when absent; computed
  // with selects only (table[0] exists whenever end > 0).
  auto at = [&](int pos, int column) -> long {
    const bool in_range = pos < end;
    const int slot = pow2 ? pos >> p.page_shift : pos / p.page_size;
    const int row = pow2 ? pos & (p.page_size - 1) : pos - slot * p.page_size;
    const int page = table[in_range ? slot : 0];
    const bool ok = in_range && page >= 0 && page < p.pool_pages;
    if constexpr (BUF) {  // below 4 GiB: 32-bit element offsets
      const unsigned e = (unsigned)page * (unsigned)p.page_stride +
                         (unsigned)kvh * (unsigned)p.head_stride + (unsigned)(row * D + column);
      return ok ? (long)e : -1;
    } else {
      const long e = (long)page * p.page_stride + (long)kvh * p.head_stride + (long)row * D + column;
      return ok ? e : -1;
    }
  };
#pragma unroll
  for (int i = 0; i < R::kPer; ++i) {
    const int item = tid + i * kPaThreads;
    long e = at(base + item / CH, 8 * (item % CH));
    if constexpr (R::kItems % kPaThreads != 0) e = item < R::kItems ? e : -1;
    if constexpr (BUF) {
      r.k[i] = buffer_load_h8(rk, e < 0 ? kBufferAbsent : (unsigned)e * 2u);
    } else {
      r.k[i] = e < 0 ? zero : load_h8(p.k + e);
    }
  }
#pragma unroll
  for (int i = 0; i < R::vPer; ++i) {
    const int item = tid + i * kPaThreads;
    const int quad = item % (kPaBlock / 4), octet = item / (kPaBlock / 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      long e = at(base + 4 * quad + q, 8 * octet);
      if constexpr (R::vItems % kPaThreads != 0) e = item < R::vItems ? e : -1;
      if constexpr (BUF) {
        r.v[q][i] = buffer_load_h8(rv, e < 0 ? kBufferAbsent : (unsigned)e * 2u);
      } else {
        r.v[q][i] = e < 0 ? zero : load_h8(p.v + e);
      }
    }
  }
}

// Registers -> LDS: K row-major [64][D + kKPad], V transposed [D][64 + kVPad].
template <int D>
__device__ __forceinline__ void pa_store(PaBlockRegs<D>& r, half_t* sk, half_t* svt) {
  constexpr int CH = D / 8;
  // Pin the loaded registers here (after the barrier that precedes this
  // call): without it the compiler moves the V transposition up to the
  // loads and waits for each load as soon as it is issued.
#pragma unroll
  for (int i = 0; i < PaBlockRegs<D>::kPer; ++i) asm volatile("" : "+v"(r.k[i]));
#pragma unroll
  for (int i = 0; i < PaBlockRegs<D>::vPer; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) asm volatile("" : "+v"(r.v[q][i]));
#pragma unroll
  for (int i = 0; i < PaBlockRegs<D>::kPer; ++i) {
    const int item = threadIdx.x + i * kPaThreads;
    if (item >= PaBlockRegs<D>::kItems) break;
    *reinterpret_cast<h8*>(sk + (item / CH) * (D + kKPad) + 8 * (item % CH)) = r.k[i];
  }
#pragma unroll
  for (int i = 0; i < PaBlockRegs<D>::vPer; ++i) {
    const int item = threadIdx.x + i * kPaThreads;
    if (item >= PaBlockRegs<D>::vItems) break;
    const int quad = item % (kPaBlock / 4), octet = item / (kPaBlock / 4);
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const h4 col = {r.v[0][i][d], r.v[1][i][d], r.v[2][i][d], r.v[3][i][d]};
      *reinterpret_cast<h4*>(svt + (8 * octet + d) * (kPaBlock + kVPad) + 4 * quad) = col;
    }
  }
}

// One staged 64-position block for this lane's query column: scores on
// MFMA, online softmax in the log2 domain, then O^T += V^T P^T on MFMA.
template <int D>
__device__ __forceinline__ void pa_compute(const PrefillParams& p, const half_t* s_k,
                                           const half_t* s_vt, const h8 (&qb)[D / 32], int base,
                                           int len, bool full, int j, int g, float& m,
                                           float& lsum, f4 (&o)[D / 16]) {
  constexpr int KS = D / 32;
  constexpr int DT = D / 16;
  // Scores S^T[pos][query] for 4 tiles of 16 positions.
  float sc[4][4];
  float bmax = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const half_t* krow = s_k + (16 * kt + j) * (D + kKPad) + 8 * g;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const h8*>(krow + 32 * s),
                                                   qb[s], acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int pos = base + 16 * kt + 4 * g + r;
      // full: the whole block lies below every query's length in this wave
      sc[kt][r] = full || pos < len ? acc[r] * p.scale_log2 : -INFINITY;
      bmax = fmaxf(bmax, sc[kt][r]);
    }
  }
  bmax = fmaxf(bmax, __shfl_xor(bmax, 16, kWave));
  bmax = fmaxf(bmax, __shfl_xor(bmax, 32, kWave));
  const float next = fmaxf(m, bmax);
  const float alpha = next == -INFINITY ? 1.0f : fast_exp2(m - next);
  m = next;
  h8 pb[2];
  float psum = 0.0f;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pr = !full && sc[kt][r] == -INFINITY ? 0.0f : fast_exp2(sc[kt][r] - next);
      const half_t ph = (half_t)pr;
      psum += (float)ph;  // the denominator sums the weights the product uses
      pb[kt >> 1][4 * (kt & 1) + r] = ph;
    }
  lsum = lsum * alpha + psum;
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] *= alpha;
  // O^T[d][query] += V^T[d][pos] P^T[pos][query]; slot 8g+e of step c is
  // position 32c + 4g + e (e < 4) or 32c + 16 + 4g + (e - 4).
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    const half_t* vrow = s_vt + (16 * t + j) * (kPaBlock + kVPad) + 4 * g;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const h4 lo = *reinterpret_cast<const h4*>(vrow + 32 * c);
      const h4 hi = *reinterpret_cast<const h4*>(vrow + 32 * c + 16);
      const h8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb[c], o[t], 0, 0, 0);
    }
  }
}

// TLDS: the request's block table is staged in LDS (dynamic, max_pages
// entries) so a block's K/V addresses need no global round trip first.
// BUF: see pa_load.  With TLDS, BUF and a power-of-two page size of at
// least 4 the LDS table holds byte offsets (pa_load's OFFS form).
template <int D, bool TLDS, bool BUF>
__global__ __launch_bounds__(kPaThreads) void prefill_attention_kernel(PrefillParams p) {
  constexpr int KS = D / 32;  // k-steps of the score product
  constexpr int DT = D / 16;  // 16-dim output tiles
  __shared__ __attribute__((aligned(16))) half_t s_k[kPaBlock * (D + kKPad)];
  __shared__ __attribute__((aligned(16))) half_t s_vt[D * (kPaBlock + kVPad)];
  __shared__ int s_bounds[2];
  extern __shared__ int s_table[];

  // Workgroup -> (kv head, tile).  With kv_heads a multiple of 8, the tiles
  // of one kv head stay on one XCD (workgroups are dealt to the 8 XCDs
  // round-robin), so its K/V blocks are shared through that XCD's L2; the
  // longest (last) tiles of each head start first.
  const int id = blockIdx.x;
  int kvh, tile;
  if (p.kv_heads % 8 == 0) {
    const int xcd = id % 8, j = id / 8;
    kvh = xcd + 8 * (j / p.tiles);
    tile = p.tiles - 1 - j % p.tiles;
  } else {
    kvh = id / p.tiles;
    tile = p.tiles - 1 - id % p.tiles;
  }
  const int active = min(p.active[0], p.rows);
  const int t0 = tile * p.tokens_per_tile;
  if (t0 >= active) return;
  // The tile's request: the table row of its first token (a caller packing
  // several requests starts each at a tile boundary; a token of another
  // table row in the tile gets no output).
  const int tile_table = p.row_table ? p.row_table[t0] : 0;
  if (tile_table < 0 || tile_table >= p.table_rows) return;
  const int32_t* request_table = p.table + (size_t)tile_table * p.max_pages;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int j = lane & 15, g = lane >> 4;
  // This lane's query column: vector wave*16 + j = token offset * G + head offset.
  const int vec = wave * 16 + j;
  const int token = t0 + vec / p.group;
  const int head = kvh * p.group + vec % p.group;
  const int capacity = p.page_size * p.max_pages;
  int len = 0;
  if (vec < p.tokens_per_tile * p.group && token < active) {
    len = p.valid[token];
    if (len < 1 || len > capacity) len = -1;  // no output for this query
    if (p.row_table && p.row_table[token] != tile_table) len = -1;
  }

  const bool offs = TLDS && BUF && p.page_shift >= 2;  // workgroup-uniform
  // Attended extent of the tile and the first absent page below it.
  if (threadIdx.x == 0) {
    s_bounds[0] = 0;
    s_bounds[1] = 0x7fffffff;
  }
  __syncthreads();
  if (g == 0 && len > 0) atomicMax(&s_bounds[0], len);
  __syncthreads();
  const int end = s_bounds[0];
  if (end == 0) return;
  {
    const int pages = (end + p.page_size - 1) / p.page_size;
    int first_bad = 0x7fffffff;
    for (int i = threadIdx.x; i < pages; i += kPaThreads) {
      const int page = request_table[i];
      const bool ok = page >= 0 && page < p.pool_pages;
      if (TLDS) {
        if (offs)
          s_table[i] = (int)(ok ? (unsigned)(((long)page * p.page_stride +
                                              (long)kvh * p.head_stride) * 2)
                                : kBufferAbsent);
        else
          s_table[i] = page;
      }
      if (!ok) first_bad = min(first_bad, i);
    }
    if (first_bad != 0x7fffffff) atomicMin(&s_bounds[1], first_bad);
  }
  __syncthreads();
  const long bad_from = (long)s_bounds[1] * p.page_size;  // positions at/after: absent page

  const h8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  h8 qb[KS];
  {
    const half_t* qrow = p.q + ((size_t)token * p.q_heads + head) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) qb[s] = len > 0 ? load_h8(qrow + 32 * s + 8 * g) : zero;
  }
  f4 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float m = -INFINITY, lsum = 0.0f;

  const int* table = TLDS ? s_table : request_table;
  // Shortest length among the wave's live queries: blocks below it need no mask.
  int wave_min = len > 0 ? len : 0x7fffffff;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) wave_min = min(wave_min, __shfl_xor(wave_min, off, kWave));
  // The next block's loads are issued as soon as the current one is in LDS
  // and land during its compute.  (Two or three blocks in flight measured
  // no faster.)
  PaBlockRegs<D> regs;
  auto load = [&](int at) {
    if (offs) pa_load<D, BUF, TLDS && BUF>(p, table, kvh, at, end, regs);
    else pa_load<D, BUF, false>(p, table, kvh, at, end, regs);
  };
  load(0);
  for (int base = 0; base < end; base += kPaBlock) {
    __syncthreads();  // the previous block's LDS reads are done
    pa_store<D>(regs, s_k, s_vt);
    __syncthreads();
    if (base + kPaBlock < end) load(base + kPaBlock);
    const bool full = base + kPaBlock <= wave_min;  // wave-uniform
    pa_compute<D>(p, s_k, s_vt, qb, base, len, full, j, g, m, lsum, o);
  }

  lsum += __shfl_xor(lsum, 16, kWave);
  lsum += __shfl_xor(lsum, 32, kWave);
  if (len <= 0 || len > bad_from) return;
  const float inv = 1.0f / lsum;
  half_t* orow = p.out + ((size_t)token * p.q_heads + head) * D;
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    const h4 val = {(half_t)(o[t][0] * inv), (half_t)(o[t][1] * inv), (half_t)(o[t][2] * inv),
                    (half_t)(o[t][3] * inv)};
    *reinterpret_cast<h4*>(orow + 16 * t + 4 * g) = val;
  }
}

}  // namespace
}  // namespace tmc

using namespace tmc;


extern "C" int tmc_prefill_attention_rows_f16(const void* q, const void* key_pool,
                                              const void* value_pool, const int32_t* valid_lengths,
                                              const int32_t* block_tables, const int32_t* row_table,
                                              int64_t table_rows, const int32_t* active_count,
                                              void* out, int64_t rows, int64_t q_heads,
                                              int64_t kv_heads, int64_t head_dim, int64_t page_size,
                                              int64_t max_pages, int64_t pool_pages,
                                              int64_t page_stride, int64_t head_stride,
                                              void* stream) {
  TMC_REQUIRE(q && key_pool && value_pool && valid_lengths && block_tables && active_count && out,
              "Prefill attention: null device pointer.");
  TMC_REQUIRE(table_rows >= 1 && (row_table || table_rows == 1) && table_rows < (1LL << 24),
              "Prefill attention: table_rows must be 1 without a row table, else at least 1.");
  TMC_REQUIRE(head_dim == 64 || head_dim == 128, "Prefill attention: head_dim must be 64 or 128.");
  TMC_REQUIRE(rows > 0 && rows < (1LL << 24) && q_heads > 0 && kv_heads > 0 &&
                  q_heads % kv_heads == 0,
              "Prefill attention: invalid rows or heads.");
  const int64_t group = q_heads / kv_heads;
  TMC_REQUIRE(group <= kPaVectors && kPaVectors % group == 0,
              "Prefill attention: q_heads / kv_heads must divide 64.");
  TMC_REQUIRE(page_size > 0 && max_pages > 0 && page_size * max_pages < (1LL << 30) &&
                  pool_pages > 0 && pool_pages < (1LL << 31),
              "Prefill attention: invalid page geometry.");
  TMC_REQUIRE(head_stride >= page_size * head_dim &&
                  page_stride >= (kv_heads - 1) * head_stride + page_size * head_dim,
              "Prefill attention: the head stride must hold a head's page rows and the page "
              "stride every kv head.");
  PrefillParams p{};
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(key_pool);
  p.v = static_cast<const half_t*>(value_pool);
  p.out = static_cast<half_t*>(out);
  p.valid = valid_lengths;
  p.table = block_tables;
  p.row_table = row_table;
  p.table_rows = (int)table_rows;
  p.active = active_count;
  p.page_stride = page_stride;
  p.head_stride = head_stride;
  p.pool_pages = pool_pages;
  p.rows = (int)rows;
  p.q_heads = (int)q_heads;
  p.kv_heads = (int)kv_heads;
  p.group = (int)group;
  p.tokens_per_tile = (int)(kPaVectors / group);
  p.tiles = (int)((rows + p.tokens_per_tile - 1) / p.tokens_per_tile);
  p.page_size = (int)page_size;
  p.max_pages = (int)max_pages;
  p.page_shift = -1;
  for (int b = 0; b < 31; ++b)
    if (page_size == (int64_t)1 << b) p.page_shift = b;
  p.scale_log2 = (float)(1.0 / std::sqrt((double)head_dim)) * 1.4426950408889634f;
  const dim3 grid((unsigned)((int64_t)p.tiles * kv_heads));
  // The table goes to LDS when it fits beside the K/V blocks in 64 KiB.
  const size_t static_lds = (size_t)kPaBlock * (head_dim + kKPad) * 2 +
                            (size_t)head_dim * (kPaBlock + kVPad) * 2 + 16;
  const size_t table_lds = (size_t)max_pages * 4;
  const bool tlds = static_lds + table_lds <= kPaMaxLds;
  const size_t dyn = tlds ? table_lds : 0;
  const hipStream_t s = as_stream(stream);
  const uint64_t pool_bytes = (uint64_t)pool_pages * (uint64_t)page_stride * 2;
  const bool buf = pool_bytes < kBufferAbsent;
  p.pool_bytes = buf ? (unsigned)pool_bytes : 0u;
#define TMC_PA_LAUNCH(DIM, T, B)                                                                  \
  hipLaunchKernelGGL((prefill_attention_kernel<DIM, T, B>), grid, dim3(kPaThreads), dyn, s, p)
  if (head_dim == 128) {
    if (tlds) {
      if (buf) TMC_PA_LAUNCH(128, true, true); else TMC_PA_LAUNCH(128, true, false);
    } else {
      if (buf) TMC_PA_LAUNCH(128, false, true); else TMC_PA_LAUNCH(128, false, false);
    }
  } else {
    if (tlds) {
      if (buf) TMC_PA_LAUNCH(64, true, true); else TMC_PA_LAUNCH(64, true, false);
    } else {
      if (buf) TMC_PA_LAUNCH(64, false, true); else TMC_PA_LAUNCH(64, false, false);
    }
  }
#undef TMC_PA_LAUNCH
  return check_launch("prefill_attention_kernel");
}

extern "C" int tmc_prefill_attention_f16(const void* q, const void* key_pool, const void* value_pool,
                                         const int32_t* valid_lengths, const int32_t* block_table,
                                         const int32_t* active_count, void* out, int64_t rows,
                                         int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                         int64_t page_size, int64_t max_pages, int64_t pool_pages,
                                         int64_t page_stride, int64_t head_stride, void* stream) {
  return tmc_prefill_attention_rows_f16(q, key_pool, value_pool, valid_lengths, block_table,
                                        nullptr, 1, active_count, out, rows, q_heads, kv_heads,
                                        head_dim, page_size, max_pages, pool_pages, page_stride,
                                        head_stride, stream);
}
