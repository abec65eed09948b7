// Split-KV decode attention for gfx950 (fp16 K/V, fp32 softmax).
//
// Reference semantics: emitKVAttention / emitPagedKVAttention /
// emitServingPagedKVAttention (KVCacheMetalEmitter.cpp:119-406): for each
// (request, head) attend positions [0, valid), online softmax, output
// T(weighted / denominator).  The reference runs one threadgroup per head and
// walks positions serially with a tree reduction per position; here the
// positions of one (request, kv head) are cut into CHUNK-position splits,
// one 256-thread block per split, and the GROUP query heads that share a kv
// head (GQA) are served from the same K/V loads.
//
// A multi-split (request, kv head) stores one (max, sum, weighted) partial
// per split in the workspace and the partials are merged in split order:
// at D = 128 with a GQA group of at most 4 by the row's last-arriving split
// block (merge_if_last: agent-scope stores and loads and an arrival counter,
// no fences), otherwise by attn_combine_kernel, one block per (request,
// query head).  (An earlier in-kernel merge with device-scope fences, each
// of which writes back and invalidates the XCD's L2, measured several times
// slower.)
//
// D = 128 runs attn_mfma_kernel (scores from v_mfma_f32_16x16x32_f16, see the
// comment above it); smaller heads run attn_partial_kernel: RL = D/8 lanes
// hold one position's 16-byte slices, so one 16-byte load covers NR = 64/RL
// consecutive positions, a wave tile is J = 4 such loads, and rows are
// folded together once per split (cross-row shuffles).
#include "tmc_abi.hpp"
#include "tmc_device.hpp"

#include <algorithm>
#include <climits>
#include <mutex>

// Split partials of tmc_paged_decode_attention_noalloc: a file-scope device
// array, so that entry point needs no allocation.  Each GPU the library runs
// on holds its own copy until the process ends; host code reaches it only
// through the address hipGetSymbolAddress returns for the current device.
constexpr size_t kScratchBytes = 16u << 20;
constexpr size_t kScratchCounterBytes = 64u << 10;  // merge counters at the scratch's start
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

// Build switch: 1 records per-wave timestamps of the 4-wave split kernel and
// the 8-wave one-split kernel for contiguous caches and 16-position pages
// (bench.py's C3 and C4, the batch-16 7B decode step's attention) into
// `timeline`, read back by tmc_attention_timeline.  Per wave
// (block-linear index * waves per block + wave), kTimelineEvents slots: 0 / 1 the 100 MHz
// real-time clock at entry and exit, 2 HW_ID | XCC_ID << 32, 3 the shader
// clock (s_memtime) at entry, 9 once the block knows its unit (dealt
// blocks; else the entry clock), 4 before the first step, 5 before the
// cross-wave merge and partial write, 6 after it, 7 at exit, 8 the wave's
// step count (99: the block had no work), and for steps s < 12: 10 + 3s
// before the step's loads, 11 + 3s once they have all arrived, 12 + 3s
// after the step's arithmetic.  Waiting for every load of a step before
// its timestamp costs the kernel about 10% (C4 37.9 -> 41.9 us on MI355X).
#ifndef TMC_ATTN_TIMELINE
#define TMC_ATTN_TIMELINE 0
#endif
#if TMC_ATTN_TIMELINE
constexpr int kTimelineWaves = 8192;
constexpr int kTimelineEvents = 48;
static __device__ unsigned long long timeline[kTimelineWaves * kTimelineEvents];
#endif

namespace tmc {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kTilesPerWave = 2;  // VALU kernel (D < 128)
// D == 128 kernel: a wave step is kMfmaTiles 16-position MFMA tiles whose
// K/V loads are all issued before the first MFMA.  (Keeping a second step's
// loads in flight was measured slower: the extra registers halve occupancy.)
// Positions per split are chosen per launch from 128 ... 1024 (chunk_for).
constexpr int kMfmaTiles = 2;
constexpr int kMfmaStep = 16 * kMfmaTiles;
constexpr int kMfmaMinChunk = 128;  // four waves x one 32-position step
constexpr int kMfmaMaxChunk = 1024;
// One-split blocks of 16 waves (D = 128, see split_plan): a wave walks at
// most two 32-position steps of a 1024-position row.  GQA groups up to 2:
// at 1024 threads a lane has 128 registers, and a group of 4 spills.
constexpr int kWideWaves = 16;
constexpr int kWideMaxGroup = 2;
// One-split rows too many for the 16-wave blocks (batch 16 MHA): 8-wave
// blocks (MHA only).  Measured on the 7B decode step at batch 16: 4858 ->
// 4919 tokens/s against 4-wave blocks.
constexpr int kMidWaves = 8;
// Build switch: 1 merges every multi-split row in a launch of its own
// (attn_combine_kernel) instead of in the attention kernel, so that no
// block reads another block's partials (no cross-block arrival counters).
#ifndef TMC_ATTN_MERGE_LAUNCH
#define TMC_ATTN_MERGE_LAUNCH 0
#endif
struct AttnParams {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  half_t* out;
  float* ws;
  const int32_t* valid;   // contiguous: valid[0]; paged: valid[request]
  const int32_t* tables;  // paged: [request][max_pages]
  const int32_t* active;  // paged: active request count, may be null
  long page_stride;       // paged: elements between pages
  long head_stride;       // paged: elements between kv heads inside a page
  int q_heads, kv_heads, capacity, page_size, max_pages, max_splits;
  int page_shift;         // log2(page_size) when it is a power of two, else -1
  long pool_pages;        // paged: pages in each pool (0 = unknown, no bound check)
  int chunk;              // positions per split
  int waves;              // waves per block (D = 128: kWaves, or kWideWaves for one split)
  unsigned kv_bytes;      // bytes of the K (and of the V) buffer when < 4 GiB, else 0
  float scale_log2;       // (1/sqrt(D)) * log2(e)
  int* arrivals;          // D = 128 multi-split: [batch][kv_heads] split counters (workspace start)
  long out_pass;          // > 0: out in the packed activation order, elements per 16-row pass
};

// Element of out for request b, column col (query head * D + d): row-major,
// or with out_pass > 0 the packed GEMM's activation fragment order (16-row
// pass b / 16, 32-column chunk, lane (b % 16) + 16 * (col % 32 / 8)), which
// the o projection then reads as packed activations.
__device__ __forceinline__ size_t out_index(const AttnParams& p, int b, int col, int width) {
  if (p.out_pass <= 0) return (size_t)b * width + col;
  return (size_t)(b >> 4) * p.out_pass +
         ((size_t)(col >> 5) * 64 + (b & 15) + 16 * ((col & 31) >> 3)) * 8 + (col & 7);
}

// Timeline slot e of this wave (TMC_ATTN_TIMELINE builds; lane 0 writes).
template <bool ON>
__device__ __forceinline__ void timeline_put(int e, unsigned long long v) {
#if TMC_ATTN_TIMELINE
  if constexpr (ON) {
    const unsigned w = (blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)) *
                           (blockDim.x / kWave) + threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0 && w < (unsigned)kTimelineWaves)
      timeline[(size_t)w * kTimelineEvents + e] = v;
  }
#endif
}
__device__ __forceinline__ unsigned long long shader_clock() { return __builtin_amdgcn_s_memtime(); }

// Positions per split of the VALU kernel (D < 128): 4 waves x 2 tiles of
// 4*64/(D/8) positions.
template <int D> constexpr int chunk_positions() {
  return kWaves * kTilesPerWave * 4 * (kWave / (D / 8));
}

__device__ __forceinline__ int page_of(const AttnParams& p, int pos) {
  return p.page_shift >= 0 ? pos >> p.page_shift : pos / p.page_size;
}

__device__ __forceinline__ int slot_in_page(const AttnParams& p, int pos) {
  return p.page_shift >= 0 ? pos & (p.page_size - 1) : pos % p.page_size;
}

template <bool PAGED>
__device__ __forceinline__ int valid_length(const AttnParams& p, int b) {
  return PAGED ? p.valid[b] : p.valid[0];
}

// (request, split) unit of a paged block of the 4-wave split kernel or the
// 8-wave one-split kernel.  A launch runs `rows` x `splits` units per kv head
// (slot v = split + splits * request, the grid's order); blocks whose slots
// are `per_round` apart (per_round = 256 / kv_heads, the slots of one round
// over MI355X's 256 CUs) land on one CU, so a CU's time follows the sum of
// two units' positions.  Slots [0, per_round) take the units in order of
// decreasing positions (a unit holds min(chunk, length - split * chunk) of
// its request's positions, 0 past the request's end) and the rest in
// increasing order, pairing heavy units with light or empty ones.  Every
// block derives the same permutation from all rows' lengths (ties by slot;
// rows at or past the active count hold no positions), so each unit still
// runs once.  The first wave sorts the units (one per lane) with a bitonic
// network of lane exchanges, 21 dependent steps instead of a pass over every
// other unit per lane; one barrier; every thread of the block calls it.
constexpr int kDealMax = kWave;
__device__ int dealt_unit(const AttnParams& p, int slot, int rows, int splits, int chunk,
                          int per_round) {
  __shared__ int s_order[kDealMax];
  const int units = rows * splits;
  if (units > kDealMax || per_round < 1 || units <= per_round) return slot;
  const int t = threadIdx.x;
  if (t < kWave) {
    const int active = p.active ? p.active[0] : rows;
    // key: positions, then the lower unit first; lanes past the units last
    int key = -1;
    if (t < units) {
      // the length and the active count are read together (both in bounds)
      const int row = t / splits;
      const int length = p.valid[row];
      const int ok = row < active && length >= 1 && length <= p.capacity;
      const int work = ok ? max(0, min(chunk, length - (t % splits) * chunk)) : 0;
      key = work * kWave + (kWave - 1 - t);
    }
    // descending bitonic sort over the wave's 64 lanes
#pragma unroll
    for (int k = 2; k <= kWave; k <<= 1)
#pragma unroll
      for (int j = k >> 1; j > 0; j >>= 1) {
        const int other = __shfl_xor(key, j, kWave);
        const bool take_max = ((t & k) == 0) == ((t & j) == 0);
        key = take_max ? max(key, other) : min(key, other);
      }
    if (t < units) s_order[t] = kWave - 1 - (key & (kWave - 1));
  }
  __syncthreads();
  return s_order[slot < per_round ? slot : units - 1 - (slot - per_round)];
}

// Positions per split of the D = 128 kernel for a row of `valid` positions.
// A contiguous cache (every row has the launch's one length) cuts the row
// into max_splits splits of its own length, rounded up to 32-position
// steps, instead of splits of the capacity's chunk, which leave blocks idle
// when the length is far below the capacity (C3 at L 1025 of 4096: 11.0 ->
// 8.7 us on MI355X; at L 4095 the splits are the same).  Paged rows, whose
// lengths differ, keep the capacity's chunk.
template <bool PAGED>
__device__ __forceinline__ int mfma_chunk(const AttnParams& p, int valid) {
  if (PAGED || p.max_splits <= 1) return p.chunk;
  const int steps = (valid + kMfmaStep - 1) / kMfmaStep;
  return (steps + p.max_splits - 1) / p.max_splits * kMfmaStep;
}

// Positions [p0, p0 + TILE) of one wave: K/V slices for lane (row r, column
// chunk c) at positions p0 + r + NR*j, j < 4.
template <int D, bool PAGED>
struct TileLoad {
  static constexpr int RL = D / 8;
  static constexpr int NR = kWave / RL;
  h8 k[4], v[4];
  bool ok[4];

  __device__ __forceinline__ void load(const AttnParams& p, const int* s_pages, int page0,
                                       size_t contiguous_base, int kvh, int p0, int end, int r,
                                       int c) {
    const h8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pos = p0 + r + NR * j;
      ok[j] = pos < end;
      size_t off = 0;
      if constexpr (PAGED) {
        const int page = ok[j] ? s_pages[page_of(p, pos) - page0] : -1;
        ok[j] = ok[j] && page >= 0 && (p.pool_pages == 0 || page < p.pool_pages);
        off = (size_t)page * p.page_stride + (size_t)kvh * p.head_stride +
              (size_t)slot_in_page(p, pos) * D + 8 * c;
      } else {
        off = contiguous_base + (size_t)pos * D + 8 * c;
      }
      k[j] = ok[j] ? load_h8(p.k + off) : zero;
      v[j] = ok[j] ? load_h8(p.v + off) : zero;
    }
  }
};

// Online-softmax update of the GROUP heads with one loaded tile.
template <int D, int GROUP>
__device__ __forceinline__ void attend_tile(const h8 (&qv)[GROUP], const h8 (&kt)[4],
                                            const h8 (&vt)[4], const bool (&ok)[4],
                                            float scale_log2, float (&m)[GROUP],
                                            float (&l)[GROUP], float (&o)[GROUP][8]) {
  constexpr int RL = D / 8;
#pragma unroll
  for (int g = 0; g < GROUP; ++g) {
    float s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float dot = group_sum<RL>(dot8(qv[g], kt[j], 0.0f));
      s[j] = ok[j] ? dot * scale_log2 : -INFINITY;
    }
    float tile_max = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    tile_max = cross_max<RL>(tile_max);
    const float next = fmaxf(m[g], tile_max);
    const float alpha = next == -INFINITY ? 1.0f : fast_exp2(m[g] - next);
    float psum = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) o[g][t] *= alpha;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float pj = ok[j] ? fast_exp2(s[j] - next) : 0.0f;
      psum += pj;
#pragma unroll
      for (int t = 0; t < 8; ++t) o[g][t] += pj * (float)vt[j][t];
    }
    l[g] = l[g] * alpha + psum;
    m[g] = next;
  }
}

// End of a split block: merge the block's 4 wave partials (in LDS), then
// write the output (one split) or the split's partial slot.  Rows whose
// attended range needs a negative page keep their output untouched (the
// reference kernel returns before writing); attn_combine_kernel applies the
// same rule for multi-split rows.
// With p.arrivals set the slots are written with agent-scope stores
// (written through to memory) for the merge by the row's last split block.
template <int D, int GROUP, bool PAGED, int WAVES = kWaves>
__device__ void finish_split(const AttnParams& p, int b, int kvh, int split, int nsplit,
                             bool bad, const float (*s_m)[GROUP], const float (*s_l)[GROUP],
                             const float (*s_o)[GROUP][D]) {
  // `bad`: a page of this split's range is negative or past the pool.  One
  // split covers the whole attended range, so its output stays untouched; a
  // split of several marks its slot (denominator -1) and the merge leaves the
  // output untouched when any slot is marked.
  const bool single = nsplit == 1;
  if (single && bad) return;
  for (int idx = threadIdx.x; idx < GROUP * D; idx += WAVES * kWave) {
    const int g = idx / D, d = idx % D;
    float mx = s_m[0][g];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) mx = fmaxf(mx, s_m[w][g]);
    float lsum = 0.0f, osum = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float scale = s_m[w][g] == -INFINITY ? 0.0f : fast_exp2(s_m[w][g] - mx);
      lsum += scale * s_l[w][g];
      osum += scale * s_o[w][g][d];
    }
    const int qh = kvh * GROUP + g;
    if (single) {
      p.out[out_index(p, b, qh * D + d, p.q_heads * D)] = (half_t)(osum / lsum);
    } else {
      float* slot = p.ws + (((size_t)b * p.q_heads + qh) * p.max_splits + split) * (D + 2);
      if (p.arrivals) {
        __hip_atomic_store(slot + d, osum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == 0) {
          __hip_atomic_store(slot + D, mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(slot + D + 1, bad ? -1.0f : lsum, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
      } else {
        slot[d] = osum;
        if (d == 0) {
          slot[D] = mx;
          slot[D + 1] = bad ? -1.0f : lsum;
        }
      }
    }
  }
}

// Merge the split partials of one (request, query head): thread d owns
// output column d.  The first 8 slots are loaded together with the valid
// length (one memory round trip; slots past the request's splits are read
// but ignored), later ones 8 at a time, folded with a running maximum.  A
// slot whose denominator is negative marks a bad page: the output stays
// untouched.
template <int D, bool PAGED>
__global__ __launch_bounds__(D) void attn_combine_kernel(AttnParams p) {
  const int qh = blockIdx.x, b = blockIdx.y;
  if (PAGED && p.active && b >= p.active[0]) return;
  const int d = threadIdx.x;
  const float* base = p.ws + ((size_t)b * p.q_heads + qh) * p.max_splits * (D + 2);
  float ms[8], ls[8], os[8];
  auto fetch = [&](int s0) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float* slot = base + (size_t)(s0 + k) * (D + 2);
      const bool in = s0 + k < p.max_splits;  // stays inside this row's workspace
      ms[k] = in ? slot[D] : -INFINITY;
      ls[k] = in ? slot[D + 1] : 0.0f;
      os[k] = in ? slot[d] : 0.0f;
    }
  };
  fetch(0);
  const int valid = valid_length<PAGED>(p, b);
  if (valid < 1 || valid > p.capacity) return;
  const int chunk = D == 128 ? mfma_chunk<PAGED>(p, valid) : p.chunk;
  const int nsplit = (valid + chunk - 1) / chunk;
  if (nsplit <= 1) return;
  float mx = -INFINITY, lsum = 0.0f, osum = 0.0f;
  bool bad = false;
  for (int s0 = 0; s0 < nsplit; s0 += 8) {
    if (s0 > 0) fetch(s0);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (s0 + k >= nsplit) {
        ms[k] = -INFINITY;
        ls[k] = 0.0f;
        os[k] = 0.0f;
      } else {
        bad |= ls[k] < 0.0f;
      }
    float next = mx;
#pragma unroll
    for (int k = 0; k < 8; ++k) next = fmaxf(next, ms[k]);
    const float alpha = mx == -INFINITY ? 0.0f : fast_exp2(mx - next);
    lsum *= alpha;
    osum *= alpha;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float scale = ms[k] == -INFINITY ? 0.0f : fast_exp2(ms[k] - next);
      lsum += scale * ls[k];
      osum += scale * os[k];
    }
    mx = next;
  }
  if (PAGED && bad) return;
  p.out[out_index(p, b, qh * D + d, p.q_heads * D)] = (half_t)(osum / lsum);
}

template <int D, int GROUP, bool PAGED>
__global__ __launch_bounds__(kThreads) void attn_partial_kernel(AttnParams p) {
  constexpr int RL = D / 8;
  constexpr int NR = kWave / RL;
  constexpr int TILE = NR * 4;
  constexpr int CHUNK = chunk_positions<D>();
  __shared__ float s_m[kWaves][GROUP];
  __shared__ float s_l[kWaves][GROUP];
  __shared__ float s_o[kWaves][GROUP][D];
  __shared__ int s_pages[PAGED ? CHUNK + 1 : 1];

  const int b = blockIdx.z, kvh = blockIdx.x, split = blockIdx.y;
  if (PAGED && p.active && b >= p.active[0]) return;
  const int valid = valid_length<PAGED>(p, b);
  if (valid < 1 || valid > p.capacity) return;
  const int nsplit = (valid + CHUNK - 1) / CHUNK;
  if (split >= nsplit) return;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int c = lane % RL;
  const int r = lane / RL;
  const int begin = split * CHUNK;
  const int end = min(valid, begin + CHUNK);

  // Block-table entries of this split, fetched once (one latency period
  // instead of one per tile before each K/V load).
  int page0 = 0;
  bool bad = false;
  if constexpr (PAGED) {
    page0 = page_of(p, begin);
    const int entries = page_of(p, end - 1) - page0 + 1;
    int bad_page = 0;
    for (int i = threadIdx.x; i < entries; i += kThreads) {
      const int page = p.tables[(size_t)b * p.max_pages + page0 + i];
      s_pages[i] = page;
      bad_page |= page < 0 || (p.pool_pages > 0 && page >= p.pool_pages);
    }
    bad = __syncthreads_or(bad_page) != 0;
  }

  h8 qv[GROUP];
#pragma unroll
  for (int g = 0; g < GROUP; ++g)
    qv[g] = load_h8(p.q + ((size_t)b * p.q_heads + kvh * GROUP + g) * D + 8 * c);

  float m[GROUP], l[GROUP], o[GROUP][8];
#pragma unroll
  for (int g = 0; g < GROUP; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) o[g][t] = 0.0f;
  }
  const size_t contiguous_base = ((size_t)b * p.kv_heads + kvh) * (size_t)p.capacity * D;

  // Two tiles in flight per wave: this wave's tiles t and t + 4.
  for (int tile = wave;; tile += 2 * kWaves) {
    const int p0a = begin + tile * TILE;
    if (p0a >= end) break;  // wave-uniform
    const int p0b = p0a + kWaves * TILE;
    TileLoad<D, PAGED> a, bt;
    a.load(p, s_pages, page0, contiguous_base, kvh, p0a, end, r, c);
    bt.load(p, s_pages, page0, contiguous_base, kvh, p0b, end, r, c);
    attend_tile<D, GROUP>(qv, a.k, a.v, a.ok, p.scale_log2, m, l, o);
    if (p0b < end) attend_tile<D, GROUP>(qv, bt.k, bt.v, bt.ok, p.scale_log2, m, l, o);
  }

  // Fold the NR position rows of the wave (each row held other positions).
#pragma unroll
  for (int g = 0; g < GROUP; ++g) {
    l[g] = cross_sum<RL>(l[g]);
#pragma unroll
    for (int t = 0; t < 8; ++t) o[g][t] = cross_sum<RL>(o[g][t]);
  }
  if (r == 0) {
#pragma unroll
    for (int g = 0; g < GROUP; ++g) {
#pragma unroll
      for (int t = 0; t < 8; ++t) s_o[wave][g][8 * c + t] = o[g][t];
      if (c == 0) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();
  finish_split<D, GROUP, PAGED>(p, b, kvh, split, nsplit, bad, s_m, s_l, s_o);
}

// ---------------------------------------------------------------- D = 128
// Split partial for D = 128: grid (split, kv head, request).  Wave w takes
// the steps w, w + 4, ... of its split; a step is kMfmaTiles tiles of 16
// positions.
//
// Scores come from v_mfma_f32_16x16x32_f16: A = the tile's 16 K rows, B = the
// GROUP query heads of the kv head as columns (zero columns beyond GROUP).
// Lane l: MFMA row/column j = l % 16, k-group g = l / 16 (MFMA s takes d chunk
// 4s+g); acc[r] = score(position p0 + 4g + r, head j).  PV on VALU
// (consume_step): lane (row g, column chunk j) accumulates positions
// p0 + 4i + g, i < 4, with the probabilities read back from the wave's LDS
// slice; PV on the MFMA for GQA groups of 4 and more (consume_step_pvm).
//
// MODE 0: contiguous cache [request][kv head][capacity][128].  MODE 1: pages
// whose size is a multiple of 16 (a 16-aligned tile lies in one page: one
// block-table lookup per tile).  Both read K/V with raw buffer loads: a
// position that is absent (past the range, or in a missing page) gets an
// offset past the buffer, which the hardware answers with zeros, so no load
// is predicated.  MODE 2: any other page size, or buffers of 4 GiB or more:
// one lookup per position and ordinary predicated loads.
constexpr unsigned kAbsent = 0xFFFFFFF0u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// NT: non-temporal hint (cache policy bit nt) for K/V read once per launch.
// Measured on MI355X: the contiguous cache (MODE 0, L = 4095) reads 3.75 ->
// 4.03 TB/s with it; the paged GQA cache (16-position pages) 3.64 -> 3.40,
// so pages keep the default policy.
template <bool NT>
__device__ __forceinline__ h8 buffer_h8(__amdgpu_buffer_rsrc_t r, unsigned byte_offset) {
  return __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_offset, 0,
                                                                      NT ? 2 : 0));
}

template <int MODE>
struct KvStep {
  h8 k[kMfmaTiles][4], v[kMfmaTiles][4];
  long tile[kMfmaTiles];  // element offset of each tile's first position, -1 = absent
};

template <int MODE>
__device__ __forceinline__ bool page_ok(const AttnParams& p, int page) {
  return page >= 0 && (p.pool_pages == 0 || page < p.pool_pages);
}

// Element offset of position `pos` (MODE 2 lookup), -1 when absent.
__device__ __forceinline__ long paged_offset(const AttnParams& p, const int* s_pages, int page0,
                                             int kvh, int pos, int end) {
  if (pos >= end) return -1;
  const int page = s_pages[page_of(p, pos) - page0];
  if (!page_ok<2>(p, page)) return -1;
  return (long)page * p.page_stride + (long)kvh * p.head_stride +
         (long)slot_in_page(p, pos) * 128;
}

template <int MODE, bool VIA = false>
__device__ __forceinline__ void issue_step(const AttnParams& p, const int* s_pages, int page0,
                                           size_t cbase, int kvh, int p0, int end, int j, int g,
                                           __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                           KvStep<MODE>& st) {
  const h8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int t = 0; t < kMfmaTiles; ++t) {
    const int tp = p0 + 16 * t;
    if constexpr (MODE < 2) {
      long tile = -1;
      if (tp < end) {
        if constexpr (MODE == 0) {
          tile = (long)(cbase + (size_t)tp * 128);
        } else {
          // The tile's page id is the same for every lane: in a scalar
          // register the branch on it stays scalar, so the loads below are
          // issued back to back (a per-lane value turned this into exec-mask
          // control flow and a wait on every load already in flight).
          const int page = __builtin_amdgcn_readfirstlane(s_pages[page_of(p, tp) - page0]);
          if (page_ok<1>(p, page))
            tile = (long)page * p.page_stride + (long)kvh * p.head_stride +
                   (long)slot_in_page(p, tp) * 128;
        }
      }
      st.tile[t] = tile;
      // Absent positions OR kAbsent into an in-range offset: the result
      // lies past the buffer (the hardware returns zeros) and is computed
      // without a select or branch per load.
      const unsigned tb = tile < 0 ? 0u : (unsigned)(tile * 2);
      const unsigned tmask = tile < 0 ? kAbsent : 0u;
      if constexpr (VIA) {
        // whole rows: load q reads positions 4q .. 4q + 3 of the tile, lane
        // (j, g) the 16-byte chunk j of position 4q + g (8 full cache lines
        // per load); consume_step re-lays them in the MFMA operand order
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const unsigned rmask = tmask | (tp + 4 * q + g < end ? 0u : kAbsent);
          st.k[t][q] = buffer_h8<MODE == 0>(rk, (tb + (unsigned)(4 * q + g) * 256u + 16u * j) | rmask);
        }
      } else {
        const unsigned kmask = tmask | (tp + j < end ? 0u : kAbsent);
#pragma unroll
        for (int s = 0; s < 4; ++s)
          st.k[t][s] = buffer_h8<MODE == 0>(rk, (tb + (unsigned)j * 256u + 16u * (4 * s + g)) | kmask);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const unsigned vmask = tmask | (tp + 4 * i + g < end ? 0u : kAbsent);
        st.v[t][i] = buffer_h8<MODE == 0>(rv, (tb + (unsigned)(4 * i + g) * 256u + 16u * j) | vmask);
      }
    } else {
      st.tile[t] = tp < end ? 0 : -1;
      const long krow = paged_offset(p, s_pages, page0, kvh, tp + j, end);
#pragma unroll
      for (int s = 0; s < 4; ++s)
        st.k[t][s] = krow >= 0 ? load_h8(p.k + krow + 8 * (4 * s + g)) : zero;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const long vrow = paged_offset(p, s_pages, page0, kvh, tp + 4 * i + g, end);
        st.v[t][i] = vrow >= 0 ? load_h8(p.v + vrow + 8 * j) : zero;
      }
    }
  }
}

template <int GROUP, int MODE, bool VIA = false>
__device__ __forceinline__ void consume_step(const AttnParams& p, const int* s_pages, int page0,
                                             const KvStep<MODE>& st, const h8 (&qb)[4], int p0,
                                             int end, int j, int g, float (*s_pw)[GROUP],
                                             float& m, float& lsum, float (&o)[GROUP][8],
                                             h8* s_k = nullptr) {
  float sc[kMfmaTiles][4];
  float tile_max = -INFINITY;
  h8 kf[kMfmaTiles][4];
  if constexpr (VIA) {
    // this wave's LDS slice, 16 rows x 16 chunks per tile; chunk c of row r
    // at slot c ^ r, so the row-wise stores and the column-wise operand
    // reads both touch 16 distinct bank groups per 16 lanes
#pragma unroll
    for (int t = 0; t < kMfmaTiles; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = 4 * q + g;
        s_k[t * 256 + r * 16 + (j ^ r)] = st.k[t][q];
      }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int t = 0; t < kMfmaTiles; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s) kf[t][s] = s_k[t * 256 + j * 16 + ((4 * s + g) ^ j)];
    __builtin_amdgcn_wave_barrier();
  } else {
#pragma unroll
    for (int t = 0; t < kMfmaTiles; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s) kf[t][s] = st.k[t][s];
  }
#pragma unroll
  for (int t = 0; t < kMfmaTiles; ++t) {
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[t][s], qb[s], acc, 0, 0, 0);
    const int tp = p0 + 16 * t;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int pos = tp + 4 * g + r;
      bool ok = st.tile[t] >= 0 && pos < end;
      if constexpr (MODE == 2) ok = ok && page_ok<2>(p, s_pages[page_of(p, pos) - page0]);
      sc[t][r] = ok ? acc[r] * p.scale_log2 : -INFINITY;
      tile_max = fmaxf(tile_max, sc[t][r]);
    }
  }
  tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 16, kWave));
  tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32, kWave));
  const float next = fmaxf(m, tile_max);
  const float alpha = next == -INFINITY ? 1.0f : fast_exp2(m - next);
  float psum = 0.0f;
#pragma unroll
  for (int t = 0; t < kMfmaTiles; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pr = sc[t][r] == -INFINITY ? 0.0f : fast_exp2(sc[t][r] - next);
      psum += pr;
      if (j < GROUP) s_pw[16 * t + 4 * g + r][j] = pr;
    }
  lsum = lsum * alpha + psum;
  m = next;
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int h = 0; h < GROUP; ++h) {
    const float ah = readlane(alpha, h);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] *= ah;
  }
#pragma unroll
  for (int t = 0; t < kMfmaTiles; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float pv[GROUP];
#pragma unroll
      for (int h = 0; h < GROUP; ++h) pv[h] = s_pw[16 * t + 4 * i + g][h];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = (float)st.v[t][i][e];
#pragma unroll
        for (int h = 0; h < GROUP; ++h) o[h][e] += pv[h] * v;
      }
    }
  __builtin_amdgcn_wave_barrier();
}

// One step of the whole-row forms (MODE 0 / 1) with PV on the MFMA as well.
// K goes through the wave's LDS slice as in consume_step; then V's 32 rows go
// through the same slice (the 32-byte units of row R at unit slot u ^ (R & 7)),
// and ds_read_b64_tr_b16 gives each lane the B operand of
// v_mfma_f32_16x16x32_f16 with positions as k: a 16-lane group's result lane
// n, element e, is the n-th 16-bit value of the 8-byte run its source lane
// 4e + n/4 points at, so source lane s of group g points at position
// (16h + 4g + s/4), dims 16db + 4(s%4): result lane (n, g) gets dims
// 16db + n of positions 16h + 4g .. +3.  The probabilities are the A operand
// just as the score MFMA left them: lane (head j, group g) holds positions
// 4g .. 4g+3 of both 16-position tiles, the same k order.  oacc[db][r] is
// O[head 4g + r][16 db + j], summed over the positions of the steps so far.
template <int GROUP, int MODE>
__device__ __forceinline__ void consume_step_pvm(const AttnParams& p, const KvStep<MODE>& st,
                                                 const h8 (&qb)[4], int p0, int end, int j, int g,
                                                 float& m, float& lsum, f4 (&oacc)[8], h8* s_k) {
  static_assert(MODE != 2 && GROUP <= 16, "whole-row K/V forms, at most 16 heads per kv head");
  typedef half_t v4h __attribute__((ext_vector_type(4)));
  typedef __fp16 v4fp16 __attribute__((__vector_size__(8)));
  float sc[kMfmaTiles][4];
  float tile_max = -INFINITY;
  h8 kf[kMfmaTiles][4];
#pragma unroll
  for (int t = 0; t < kMfmaTiles; ++t)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = 4 * q + g;
      s_k[t * 256 + r * 16 + (j ^ r)] = st.k[t][q];
    }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int t = 0; t < kMfmaTiles; ++t)
#pragma unroll
    for (int s = 0; s < 4; ++s) kf[t][s] = s_k[t * 256 + j * 16 + ((4 * s + g) ^ j)];
  __builtin_amdgcn_wave_barrier();
  // V row R = 16t + 4i + g, 16-byte chunk j: unit j/2 at slot (j/2) ^ (R & 7)
  char* vb = reinterpret_cast<char*>(s_k);
#pragma unroll
  for (int t = 0; t < kMfmaTiles; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int R = 16 * t + 4 * i + g;
      *reinterpret_cast<h8*>(vb + R * 256 + (((j >> 1) ^ (R & 7)) << 5) + ((j & 1) << 4)) =
          st.v[t][i];
    }
#pragma unroll
  for (int t = 0; t < kMfmaTiles; ++t) {
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[t][s], qb[s], acc, 0, 0, 0);
    const int tp = p0 + 16 * t;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = st.tile[t] >= 0 && tp + 4 * g + r < end;
      sc[t][r] = ok ? acc[r] * p.scale_log2 : -INFINITY;
      tile_max = fmaxf(tile_max, sc[t][r]);
    }
  }
  tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 16, kWave));
  tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32, kWave));
  const float next = fmaxf(m, tile_max);
  const float alpha = next == -INFINITY ? 1.0f : fast_exp2(m - next);
  float psum = 0.0f;
  h8 pa;
#pragma unroll
  for (int t = 0; t < kMfmaTiles; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pr = sc[t][r] == -INFINITY ? 0.0f : fast_exp2(sc[t][r] - next);
      psum += pr;
      pa[4 * t + r] = (half_t)(j < GROUP ? pr : 0.0f);
    }
  lsum = lsum * alpha + psum;
  m = next;
  // rows 4g .. 4g+3 of the accumulator are heads 4g + r: their alpha
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float ar = __shfl(alpha, 4 * g + r, kWave);
#pragma unroll
    for (int db = 0; db < 8; ++db) oacc[db][r] *= ar;
  }
  __builtin_amdgcn_wave_barrier();
  const int s16 = j;  // source lane within the 16-lane group
#pragma unroll
  for (int db = 0; db < 8; ++db) {
    v4h half_b[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int R = 16 * h + 4 * g + (s16 >> 2);
      half_b[h] = __builtin_bit_cast(v4h, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
          reinterpret_cast<__attribute__((address_space(3))) v4fp16*>(
              (__attribute__((address_space(3))) char*)vb + R * 256 + ((db ^ (R & 7)) << 5) +
              ((s16 & 3) << 3))));
    }
    const h8 bv = __builtin_shufflevector(half_b[0], half_b[1], 0, 1, 2, 3, 4, 5, 6, 7);
    oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, bv, oacc[db], 0, 0, 0);
  }
  __builtin_amdgcn_wave_barrier();
}

// Split merge inside the partial kernel (D = 128, GQA group <= 4: each
// thread takes GROUP * 128 / threads outputs and issues the slot loads of
// all of them before using any, one memory round trip per 8 splits; on C4,
// group 4, 40.5 -> 40.0 us against the merge launch, which a one-output-
// per-pass loop here had lost by 0.6%; wider groups keep the launch).
// Every split block of a
// (request, kv head) row has written its slots with agent-scope stores;
// once they have completed it counts itself in the row's arrival counter,
// and the block that arrives last merges the row's GROUP heads exactly as
// attn_combine_kernel does (slots in split order, agent-scope loads, a
// marked slot leaves the output untouched) and resets the counter.  No
// block waits for another and no cache writeback or invalidate is needed:
// every shared word is written and read with agent-scope operations.
template <int GROUP, bool PAGED, int WAVES>
__device__ void merge_if_last(const AttnParams& p, int b, int kvh, int nsplit) {
  constexpr int D = 128;
  __shared__ int s_last;
  int* counter = p.arrivals + (size_t)b * p.kv_heads + kvh;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's slot stores have completed
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             nsplit - 1;
  __syncthreads();
  if (!s_last) return;
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // R outputs per thread, all their slot loads of a pass issued before any
  // is used (one memory round trip per 8 splits, whatever the group)
  constexpr int T = WAVES * kWave;
  constexpr int R = (GROUP * D + T - 1) / T;
  float mx[R], lsum[R], osum[R];
  bool bad[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    mx[r] = -INFINITY;
    lsum[r] = 0.0f;
    osum[r] = 0.0f;
    bad[r] = false;
  }
  const int live = GROUP * D;
  for (int s0 = 0; s0 < nsplit; s0 += 8) {
    float ms[R][8], ls[R][8], os[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int idx = min((int)threadIdx.x + r * T, live - 1);
      const int qh = kvh * GROUP + idx / D, d = idx % D;
      const float* base = p.ws + ((size_t)b * p.q_heads + qh) * p.max_splits * (D + 2);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float* slot = base + (size_t)min(s0 + k, nsplit - 1) * (D + 2);
        ms[r][k] = __hip_atomic_load(slot + D, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ls[r][k] = __hip_atomic_load(slot + D + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        os[r][k] = __hip_atomic_load(slot + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (s0 + k >= nsplit) {
          ms[r][k] = -INFINITY;
          ls[r][k] = 0.0f;
          os[r][k] = 0.0f;
        } else {
          bad[r] |= ls[r][k] < 0.0f;
        }
      float next = mx[r];
#pragma unroll
      for (int k = 0; k < 8; ++k) next = fmaxf(next, ms[r][k]);
      const float alpha = mx[r] == -INFINITY ? 0.0f : fast_exp2(mx[r] - next);
      lsum[r] *= alpha;
      osum[r] *= alpha;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float scale = ms[r][k] == -INFINITY ? 0.0f : fast_exp2(ms[r][k] - next);
        lsum[r] += scale * ls[r][k];
        osum[r] += scale * os[r][k];
      }
      mx[r] = next;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int idx = (int)threadIdx.x + r * T;
    if (idx >= live || (PAGED && bad[r])) continue;
    const int qh = kvh * GROUP + idx / D, d = idx % D;
    p.out[out_index(p, b, qh * D + d, p.q_heads * D)] = (half_t)(osum[r] / lsum[r]);
  }
}

template <int GROUP, int MODE, int WAVES>
__global__ __launch_bounds__(WAVES * kWave) void attn_mfma_kernel(AttnParams p) {
  constexpr int D = 128;
  constexpr bool PAGED = MODE != 0;
  __shared__ float s_m[WAVES][GROUP];
  __shared__ float s_l[WAVES][GROUP];
  __shared__ float s_o[WAVES][GROUP][D];
  // PV on the MFMA (consume_step_pvm) for the whole-row forms (MODE 0, 1) of
  // GQA groups of 4 and more below 16 waves, else on VALU with the
  // probabilities passed through s_p.  The MFMA computes 16 head rows
  // whatever the group, so for 1 or 2 heads the VALU form does less work with
  // fewer registers (C3, MHA: 15.3 against 16.6 us with the MFMA form; C4,
  // group 4: 37.5 -> 36.1 us); the 16-wave blocks would spill at their
  // 128-register bound.
  constexpr bool kPvm = MODE != 2 && WAVES != kWideWaves && GROUP >= 4;
  __shared__ float s_p[kPvm ? 1 : WAVES][kMfmaStep][GROUP];
  __shared__ int s_pages[PAGED ? kMfmaMaxChunk + 1 : 1];
  // 16-position tiles (MODE 0, MODE 1) load K as whole rows and re-lay them
  // for the MFMA through 8 KiB of LDS per wave.  Measured against the
  // MFMA-order loads (16 positions x 64 bytes per load instruction): C4
  // 38.7 -> 37.9 us, batch-16 MHA (8-wave blocks) 22.1 -> 21.5 us, paged
  // batch 1 (16-wave one-split blocks) at L 200 6.05 -> 5.45 us and at L 900
  // 12.4 -> 10.2 us, contiguous batch 1 at capacity 1024, L 900 16.4 ->
  // 12.4 us, contiguous C3 at L 1025 12.3 -> 11.0 us and at L 4095 the same
  // 15.2-15.4 us as the direct loads with two steps in flight, which this
  // replaces.  MODE 2 looks up every position and keeps the direct loads.
  constexpr bool kVia = MODE != 2;
  __shared__ h8 s_k[kVia ? WAVES : 1][kVia ? kMfmaTiles * 256 : 1];

  const int kvh = blockIdx.x;
  constexpr bool TL = TMC_ATTN_TIMELINE && MODE != 2 && (WAVES == kWaves || WAVES == kMidWaves);
  if constexpr (TL) {
    timeline_put<TL>(0, __builtin_amdgcn_s_memrealtime());
    timeline_put<TL>(3, shader_clock());
    timeline_put<TL>(2, (unsigned long long)__builtin_amdgcn_s_getreg(4 | (31 << 11)) |
                            ((unsigned long long)__builtin_amdgcn_s_getreg(20 | (15 << 11)) << 32));
    timeline_put<TL>(8, 99);
  }
  // One-split blocks (the whole row, max_pages <= the block's threads): each
  // thread fetches one block-table entry together with the row's length, so
  // the K/V addresses wait on one memory round trip instead of two.
  int b = blockIdx.z, split = blockIdx.y;
  if constexpr (PAGED && (WAVES == kWaves || WAVES == kMidWaves)) {
    const int unit = dealt_unit(p, split + (int)gridDim.y * b, (int)gridDim.z, (int)gridDim.y,
                                p.chunk, 256 / (int)gridDim.x);
    b = unit / (int)gridDim.y;
    split = unit % (int)gridDim.y;
  }
  if constexpr (TL) timeline_put<TL>(9, shader_clock());
  int early_page = -1;
  if constexpr (PAGED && WAVES == kWideWaves) {
    if ((int)threadIdx.x < p.max_pages)
      early_page = p.tables[(size_t)b * p.max_pages + threadIdx.x];
  }
  // the active count and the length are read together (both in bounds)
  const int active_rows = PAGED && p.active ? p.active[0] : INT_MAX;
  const int valid = valid_length<PAGED>(p, b);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int j = lane & 15;
  const int g = lane >> 4;
  const h8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  h8 qb[4];
  {
    const half_t* qrow = p.q + ((size_t)b * p.q_heads + kvh * GROUP + (j < GROUP ? j : 0)) * D;
#pragma unroll
    for (int s = 0; s < 4; ++s) qb[s] = j < GROUP ? load_h8(qrow + 8 * (4 * s + g)) : zero;
  }
  if (b >= active_rows) return;
  if (valid < 1 || valid > p.capacity) return;
  const int CHUNK = mfma_chunk<PAGED>(p, valid);
  const int nsplit = (valid + CHUNK - 1) / CHUNK;
  if (split >= nsplit) return;
  const int begin = split * CHUNK;
  const int end = min(valid, begin + CHUNK);

  int page0 = 0;
  bool bad = false;
  if constexpr (PAGED) {
    page0 = page_of(p, begin);
    const int entries = page_of(p, end - 1) - page0 + 1;
    int bad_page = 0;
    if constexpr (WAVES == kWideWaves) {  // one split: page0 == 0
      if ((int)threadIdx.x < entries) {
        s_pages[threadIdx.x] = early_page;
        bad_page = early_page < 0 || (p.pool_pages > 0 && early_page >= p.pool_pages);
      }
    } else {
      for (int i = threadIdx.x; i < entries; i += WAVES * kWave) {
        const int page = p.tables[(size_t)b * p.max_pages + page0 + i];
        s_pages[i] = page;
        bad_page |= page < 0 || (p.pool_pages > 0 && page >= p.pool_pages);
      }
    }
    bad = __syncthreads_or(bad_page) != 0;
  }
  float m = -INFINITY, lsum = 0.0f;
  // kPvm: oacc[db][r] = O[head 4g + r][16 db + j]; else o[h][e] = this lane's
  // share of O[head h][8 j + e]
  float o[kPvm ? 1 : GROUP][8];
  f4 oacc[kPvm ? 8 : 1];
#pragma unroll
  for (int h = 0; h < (kPvm ? 1 : GROUP); ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = 0.0f;
#pragma unroll
  for (int db = 0; db < (kPvm ? 8 : 1); ++db) oacc[db] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  const size_t cbase = ((size_t)b * p.kv_heads + kvh) * (size_t)p.capacity * D;
  const __amdgpu_buffer_rsrc_t rk = buffer_of(p.k, p.kv_bytes);
  const __amdgpu_buffer_rsrc_t rv = buffer_of(p.v, p.kv_bytes);
  float (*s_pw)[GROUP] = s_p[kPvm ? 0 : wave];

  constexpr int kStride = kMfmaStep * WAVES;
  int steps = 0;
  if constexpr (TL) timeline_put<TL>(4, shader_clock());
  for (int p0 = begin + kMfmaStep * wave; p0 < end; p0 += kStride) {
    KvStep<MODE> st;
    if constexpr (TL) if (steps < 12) timeline_put<TL>(10 + 3 * steps, shader_clock());
    issue_step<MODE, kVia>(p, s_pages, page0, cbase, kvh, p0, end, j, g, rk, rv, st);
    if constexpr (TL) {
      __builtin_amdgcn_s_waitcnt(0);
      if (steps < 12) timeline_put<TL>(11 + 3 * steps, shader_clock());
    }
    if constexpr (kPvm)
      consume_step_pvm<GROUP, MODE>(p, st, qb, p0, end, j, g, m, lsum, oacc, s_k[wave]);
    else
      consume_step<GROUP, MODE, kVia>(p, s_pages, page0, st, qb, p0, end, j, g, s_pw, m, lsum, o,
                                      s_k[kVia ? wave : 0]);
    if constexpr (TL) if (steps < 12) timeline_put<TL>(12 + 3 * steps, shader_clock());
    ++steps;
  }
  if constexpr (TL) {
    timeline_put<TL>(8, steps);
    timeline_put<TL>(5, shader_clock());
  }

  lsum = cross_sum<16>(lsum);
  if constexpr (kPvm) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (4 * g + r < GROUP)
#pragma unroll
        for (int db = 0; db < 8; ++db) s_o[wave][4 * g + r][16 * db + j] = oacc[db][r];
  } else {
#pragma unroll
    for (int h = 0; h < GROUP; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] = cross_sum<16>(o[h][e]);
    if (g == 0)
#pragma unroll
      for (int h = 0; h < GROUP; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) s_o[wave][h][8 * j + e] = o[h][e];
  }
  if (g == 0 && j < GROUP) {
    s_m[wave][j] = m;
    s_l[wave][j] = lsum;
  }
  __syncthreads();
  finish_split<D, GROUP, PAGED, WAVES>(p, b, kvh, split, nsplit, bad, s_m, s_l, s_o);
  if constexpr (TL) timeline_put<TL>(6, shader_clock());
  if (nsplit > 1 && p.arrivals) merge_if_last<GROUP, PAGED, WAVES>(p, b, kvh, nsplit);
  if constexpr (TL) {
    timeline_put<TL>(7, shader_clock());
    timeline_put<TL>(1, __builtin_amdgcn_s_memrealtime());
  }
}

template <int D, int GROUP, bool PAGED>
int launch_group(const AttnParams& params, int batch, hipStream_t stream) {
  AttnParams p = params;
#if TMC_ATTN_MERGE_LAUNCH
  p.arrivals = nullptr;  // build switch: every split merge in its own launch
#endif
  if (D != 128 || GROUP > 4) p.arrivals = nullptr;  // merge launch (see merge_if_last)
  const dim3 grid((unsigned)p.kv_heads, (unsigned)p.max_splits, (unsigned)batch);
  if constexpr (D == 128) {
    if (p.waves == kWideWaves) {
      if constexpr (GROUP <= kWideMaxGroup) {
        const dim3 block(kWideWaves * kWave);
        if (p.kv_bytes != 0 && !PAGED)
          hipLaunchKernelGGL((attn_mfma_kernel<GROUP, 0, kWideWaves>), grid, block, 0, stream, p);
        else if (p.kv_bytes != 0 && p.page_size % 16 == 0)
          hipLaunchKernelGGL((attn_mfma_kernel<GROUP, 1, kWideWaves>), grid, block, 0, stream, p);
        else if (PAGED)
          hipLaunchKernelGGL((attn_mfma_kernel<GROUP, 2, kWideWaves>), grid, block, 0, stream, p);
        else
          return fail("Attention: contiguous caches of 4 GiB or more are not supported.");
      } else {
        return fail("Attention: internal error (wide blocks for a large GQA group).");
      }
    } else if (p.waves == kMidWaves) {
      if constexpr (GROUP == 1) {
        const dim3 block(kMidWaves * kWave);
        if (p.kv_bytes != 0 && !PAGED)
          hipLaunchKernelGGL((attn_mfma_kernel<1, 0, kMidWaves>), grid, block, 0, stream, p);
        else if (p.kv_bytes != 0 && p.page_size % 16 == 0)
          hipLaunchKernelGGL((attn_mfma_kernel<1, 1, kMidWaves>), grid, block, 0, stream, p);
        else if (PAGED)
          hipLaunchKernelGGL((attn_mfma_kernel<1, 2, kMidWaves>), grid, block, 0, stream, p);
        else
          return fail("Attention: contiguous caches of 4 GiB or more are not supported.");
      } else {
        return fail("Attention: internal error (8-wave blocks for a GQA group).");
      }
    } else if (p.kv_bytes != 0 && !PAGED)
      hipLaunchKernelGGL((attn_mfma_kernel<GROUP, 0, kWaves>), grid, dim3(kThreads), 0, stream, p);
    else if (p.kv_bytes != 0 && p.page_size % 16 == 0)
      hipLaunchKernelGGL((attn_mfma_kernel<GROUP, 1, kWaves>), grid, dim3(kThreads), 0, stream, p);
    else if (PAGED)
      hipLaunchKernelGGL((attn_mfma_kernel<GROUP, 2, kWaves>), grid, dim3(kThreads), 0, stream, p);
    else
      return fail("Attention: contiguous caches of 4 GiB or more are not supported.");
  } else {
    hipLaunchKernelGGL((attn_partial_kernel<D, GROUP, PAGED>), grid, dim3(kThreads), 0, stream, p);
  }
  if (check_launch("attention kernel")) return 1;
  if (p.max_splits > 1 && !p.arrivals) {  // else merged in the partial kernel
    hipLaunchKernelGGL((attn_combine_kernel<D, PAGED>),
                       dim3((unsigned)p.q_heads, (unsigned)batch), dim3(D), 0, stream, p);
    return check_launch("attn_combine_kernel");
  }
  return 0;
}

template <int D, bool PAGED>
int launch_attention(const AttnParams& p, int batch, hipStream_t stream) {
  switch (p.q_heads / p.kv_heads) {
  case 1: return launch_group<D, 1, PAGED>(p, batch, stream);
  case 2: return launch_group<D, 2, PAGED>(p, batch, stream);
  case 4: return launch_group<D, 4, PAGED>(p, batch, stream);
  case 8: return launch_group<D, 8, PAGED>(p, batch, stream);
  default: return fail("Attention: q_heads / kv_heads must be 1, 2, 4 or 8.");
  }
}

int page_shift_of(int64_t page_size) {
  if (page_size <= 0 || (page_size & (page_size - 1))) return -1;
  int shift = 0;
  while ((1LL << shift) < page_size) ++shift;
  return shift;
}

// Positions per split for a launch.  D = 128: the largest power of two in
// [128, 1024] not above batch * kv_heads * capacity / 256 (one block per CU
// at full capacity); smaller heads use the VALU kernel's fixed split.
int chunk_for(int64_t head_dim, int64_t batch, int64_t kv_heads, int64_t capacity) {
  switch (head_dim) {
  case 16: return chunk_positions<16>();
  case 32: return chunk_positions<32>();
  case 64: return chunk_positions<64>();
  case 128: {
    // About one block per CU when every row fills its capacity: on MI355X
    // (256 CUs) this measured best for contiguous batch-1 attention at
    // L 4095 (chunk 512) and paged batch-16 GQA with L ~ U[64, 4096] (1024).
    const int64_t target = batch * kv_heads * capacity / 256;
    int chunk = kMfmaMinChunk;
    while (chunk < kMfmaMaxChunk && 2 * chunk <= target) chunk *= 2;
    return chunk;
  }
  default: return 0;
  }
}

bool head_dim_ok(int64_t head_dim) { return chunk_for(head_dim, 1, 1, 1) > 0; }

// Split geometry of a launch.  When the whole capacity fits one block
// (<= 1024 positions, D = 128, GQA group <= 2) and the (request, kv head)
// rows number at most one per CU (256 on MI355X), one block of 16 waves
// covers each row: no partial slots and no combine launch.  Measured on
// random 16-position pages, lengths U[33, 640]: batch 1 (L 300) 7.3 us in
// one launch against 5.8 + 4.7 us with the merge; batch 8 MHA 11.0 against
// 15.3 us; batch 16 GQA-2 11.7 against 16.1 us.  With more rows (batch 16
// MHA) the 4-wave blocks win (17.9 against 20.2 us).  A lone long row is
// slower in one block (batch 1, L 1024: 13.4 us) than split, the price of
// the short-context case.
constexpr int kWideMaxRows = 256;

struct SplitPlan {
  int chunk;
  int waves;
};

SplitPlan split_plan(int64_t head_dim, int64_t batch, int64_t q_heads, int64_t kv_heads,
                     int64_t capacity) {
  const int chunk = chunk_for(head_dim, batch, kv_heads, capacity);
  if (head_dim == 128 && chunk > 0 && capacity <= kMfmaMaxChunk &&
      batch * kv_heads <= kWideMaxRows && q_heads / kv_heads <= kWideMaxGroup)
    return {(int)((capacity + kMfmaStep - 1) / kMfmaStep * kMfmaStep), kWideWaves};
  if (head_dim == 128 && chunk >= capacity && q_heads == kv_heads)
    return {chunk, kMidWaves};
  return {chunk, kWaves};
}

template <bool PAGED>
int dispatch_attention(const AttnParams& p, int batch, int head_dim, hipStream_t stream) {
  switch (head_dim) {
  case 16: return launch_attention<16, PAGED>(p, batch, stream);
  case 32: return launch_attention<32, PAGED>(p, batch, stream);
  case 64: return launch_attention<64, PAGED>(p, batch, stream);
  default: return launch_attention<128, PAGED>(p, batch, stream);
  }
}

int common_checks(const void* q, const void* k, const void* v, const void* out, int dtype,
                  int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                  int64_t capacity) {
  TMC_REQUIRE(q && k && v && out, "Attention: null device pointer.");
  TMC_REQUIRE(dtype == TMC_F16, "Attention: the gfx950 kernel stores K/V in fp16.");
  TMC_REQUIRE(head_dim_ok(head_dim), "Attention: head_dim must be 16, 32, 64 or 128.");
  TMC_REQUIRE(q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0 &&
                  (q_heads / kv_heads) <= 8 && ((q_heads / kv_heads) & (q_heads / kv_heads - 1)) == 0,
              "Attention: q_heads / kv_heads must be 1, 2, 4 or 8.");
  TMC_REQUIRE(batch > 0 && batch < 65536 && q_heads > 0 && kv_heads > 0 && kv_heads < 65536 &&
                  q_heads % kv_heads == 0 && capacity > 0 && capacity < (1LL << 30),
              "Attention: invalid batch, head counts or capacity.");
  TMC_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v), "Attention: q, K and V must be 16-byte aligned.");
  const int chunk = split_plan(head_dim, batch, q_heads, kv_heads, capacity).chunk;
  TMC_REQUIRE((capacity + chunk - 1) / chunk <= 1024, "Attention: capacity exceeds 1024 splits.");
  return 0;
}

}  // namespace
}  // namespace tmc

using namespace tmc;

namespace tmc {
namespace {
// Workspace layout, the same for every head size and kernel: the rows'
// arrival counters ([batch][kv_heads] int) in a fixed 64 KiB area at the
// start (shapes with more than 16384 rows take rows * 4 bytes), then the
// partial slots.  Every launch leaves its counters at zero and no launch's
// slots overlap the counter area, so one zeroed workspace serves launches of
// any shapes with at most 16384 (request, kv head) rows, in any order.
constexpr size_t kCounterAreaBytes = 64u << 10;
size_t counter_bytes(int64_t batch, int64_t kv_heads) {
  const size_t rows = (size_t)batch * kv_heads * sizeof(int);
  return std::max(kCounterAreaBytes, (rows + 255) / 256 * 256);
}
size_t slot_bytes(int64_t batch, int64_t q_heads, int64_t head_dim, int64_t splits) {
  return (size_t)batch * q_heads * splits * (head_dim + 2) * sizeof(float);
}
int64_t split_count(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                    int64_t capacity) {
  const int chunk = split_plan(head_dim, batch, q_heads, kv_heads, capacity).chunk;
  return chunk > 0 ? (capacity + chunk - 1) / chunk : 0;
}
// Slot bytes a launch of this shape may use (0: no workspace needed).
size_t slots_needed(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                    int64_t capacity) {
  const int64_t splits = split_count(batch, q_heads, kv_heads, head_dim, capacity);
  return splits > 1 ? slot_bytes(batch, q_heads, head_dim, splits) : 0;
}
}  // namespace
}  // namespace tmc

extern "C" size_t tmc_attention_workspace_bytes(int64_t batch, int64_t q_heads, int64_t kv_heads,
                                                int64_t head_dim, int64_t capacity) {
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || capacity <= 0 || q_heads % kv_heads) return 0;
  const size_t slots = slots_needed(batch, q_heads, kv_heads, head_dim, capacity);
  return slots ? counter_bytes(batch, kv_heads) + slots : 0;
}

extern "C" int tmc_decode_attention(const void* q, const void* key_cache, const void* value_cache,
                                    const int32_t* valid_length, void* out, int dtype,
                                    int64_t batch, int64_t q_heads, int64_t kv_heads,
                                    int64_t head_dim, int64_t capacity, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  if (common_checks(q, key_cache, value_cache, out, dtype, batch, q_heads, kv_heads, head_dim,
                    capacity))
    return 1;
  TMC_REQUIRE(valid_length, "Attention: null valid-length pointer.");
  const size_t need = tmc_attention_workspace_bytes(batch, q_heads, kv_heads, head_dim, capacity);
  TMC_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
              "Attention: workspace is smaller than tmc_attention_workspace_bytes().");
  AttnParams p{};
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(key_cache);
  p.v = static_cast<const half_t*>(value_cache);
  p.out = static_cast<half_t*>(out);
  if (need > 0) {
    p.arrivals = static_cast<int*>(workspace);
    p.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + counter_bytes(batch, kv_heads));
  }
  p.valid = valid_length;
  p.q_heads = (int)q_heads;
  p.kv_heads = (int)kv_heads;
  p.capacity = (int)capacity;
  p.page_size = 1;
  p.page_shift = 0;
  {
    const uint64_t bytes = (uint64_t)batch * kv_heads * capacity * head_dim * 2;
    p.kv_bytes = bytes < kAbsent ? (unsigned)bytes : 0u;
  }
  const SplitPlan plan = split_plan(head_dim, batch, q_heads, kv_heads, capacity);
  p.chunk = plan.chunk;
  p.waves = plan.waves;
  p.max_splits = (int)((capacity + p.chunk - 1) / p.chunk);
  p.scale_log2 = (float)(1.0 / std::sqrt((double)head_dim)) * 1.4426950408889634f;
  return dispatch_attention<false>(p, (int)batch, (int)head_dim, as_stream(stream));
}

namespace tmc {
namespace {

// Paged attention with the split slots and the arrival counters given
// (either may be null when the limits need no workspace).
int paged_attention_impl(const void* q, const void* key_pool, const void* value_pool,
                         const int32_t* valid_lengths, const int32_t* block_tables,
                         const int32_t* active_count, void* out, int dtype, int64_t max_batch,
                         int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t page_size,
                         int64_t max_pages, int64_t pool_pages, int64_t page_stride,
                         int64_t head_stride, float* slots, int* arrivals, void* stream,
                         int layout = 0) {
  const int64_t capacity = page_size * max_pages;
  if (common_checks(q, key_pool, value_pool, out, dtype, max_batch, q_heads, kv_heads, head_dim,
                    capacity))
    return 1;
  TMC_REQUIRE(valid_lengths && block_tables, "Paged attention: null lengths or block tables.");
  TMC_REQUIRE(page_size > 0 && max_pages > 0 && page_stride > 0 && head_stride >= 0 &&
                  (page_stride % 8) == 0 && (head_stride % 8) == 0 && pool_pages >= 0 &&
                  pool_pages < (1LL << 31),
              "Paged attention: invalid page geometry (strides must be multiples of 8 elements).");
  TMC_REQUIRE(pool_pages == 0 || (kv_heads - 1) * head_stride + page_size * head_dim <= page_stride,
              "Paged attention: a page's kv heads overrun the page stride.");
  AttnParams p{};
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(key_pool);
  p.v = static_cast<const half_t*>(value_pool);
  p.out = static_cast<half_t*>(out);
  p.ws = slots;
  p.arrivals = arrivals;
  TMC_REQUIRE(layout == 0 || (layout == TMC_LAYOUT_Y_PACKED && dtype == TMC_F16 && aligned16(out)),
              "Paged attention: layout must be 0 or TMC_LAYOUT_Y_PACKED (fp16, 16-byte aligned "
              "output).");
  if (layout) p.out_pass = (long)((q_heads * head_dim + 31) / 32) * 512;
  p.valid = valid_lengths;
  p.tables = block_tables;
  p.active = active_count;
  p.page_stride = (long)page_stride;
  p.head_stride = (long)head_stride;
  p.q_heads = (int)q_heads;
  p.kv_heads = (int)kv_heads;
  p.capacity = (int)capacity;
  p.page_size = (int)page_size;
  p.page_shift = page_shift_of(page_size);
  p.pool_pages = (long)pool_pages;
  {
    const uint64_t bytes = (uint64_t)pool_pages * page_stride * 2;
    p.kv_bytes = pool_pages > 0 && bytes < kAbsent ? (unsigned)bytes : 0u;
  }
  p.max_pages = (int)max_pages;
  const SplitPlan plan = split_plan(head_dim, max_batch, q_heads, kv_heads, capacity);
  p.chunk = plan.chunk;
  p.waves = plan.waves;
  p.max_splits = (int)((capacity + p.chunk - 1) / p.chunk);
  p.scale_log2 = (float)(1.0 / std::sqrt((double)head_dim)) * 1.4426950408889634f;
  return dispatch_attention<true>(p, (int)max_batch, (int)head_dim, as_stream(stream));
}

}  // namespace
}  // namespace tmc

extern "C" int tmc_paged_decode_attention_ex(
    const void* q, const void* key_pool, const void* value_pool, const int32_t* valid_lengths,
    const int32_t* block_tables, const int32_t* active_count, void* out, int dtype,
    int64_t max_batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t page_size,
    int64_t max_pages, int64_t pool_pages, int64_t page_stride, int64_t head_stride,
    void* workspace, size_t workspace_bytes, int layout, void* stream) {
  TMC_REQUIRE(page_size > 0 && max_pages > 0 && max_pages <= (INT64_MAX / page_size),
              "Paged attention: invalid page geometry.");
  const size_t need = tmc_attention_workspace_bytes(max_batch, q_heads, kv_heads, head_dim,
                                                    page_size * max_pages);
  TMC_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
              "Paged attention: workspace is smaller than tmc_attention_workspace_bytes().");
  float* slots = nullptr;
  int* arrivals = nullptr;
  if (need > 0) {
    arrivals = static_cast<int*>(workspace);
    slots = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                     counter_bytes(max_batch, kv_heads));
  }
  return paged_attention_impl(q, key_pool, value_pool, valid_lengths, block_tables, active_count,
                              out, dtype, max_batch, q_heads, kv_heads, head_dim, page_size,
                              max_pages, pool_pages, page_stride, head_stride, slots, arrivals,
                              stream, layout);
}

extern "C" int tmc_paged_decode_attention(const void* q, const void* key_pool,
                                          const void* value_pool, const int32_t* valid_lengths,
                                          const int32_t* block_tables,
                                          const int32_t* active_count, void* out, int dtype,
                                          int64_t max_batch, int64_t q_heads, int64_t kv_heads,
                                          int64_t head_dim, int64_t page_size, int64_t max_pages,
                                          int64_t pool_pages, int64_t page_stride,
                                          int64_t head_stride, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  return tmc_paged_decode_attention_ex(q, key_pool, value_pool, valid_lengths, block_tables,
                                       active_count, out, dtype, max_batch, q_heads, kv_heads,
                                       head_dim, page_size, max_pages, pool_pages, page_stride,
                                       head_stride, workspace, workspace_bytes, 0, stream);
}

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kScratchDevices];  // per-device address of `scratch`, filled on first use

// The current device's address of `scratch` (looked up once per device,
// with that device current).  Returns 0 or sets the error text.
int scratch_address(void** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(std::string("Attention scratch: ") + hipGetErrorString(err));
  TMC_REQUIRE(device >= 0 && device < kScratchDevices, "Attention scratch: device index too large.");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[device]) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr)
      return fail(std::string("Attention scratch: hipGetSymbolAddress failed: ") +
                  hipGetErrorString(err));
    g_scratch[device] = ptr;
  }
  *out = g_scratch[device];
  return 0;
}

}  // namespace

extern "C" size_t tmc_attention_scratch_bytes(void) { return kScratchBytes; }

extern "C" int tmc_attention_timeline(uint64_t* events, int64_t waves) {
  clear_error();
#if TMC_ATTN_TIMELINE
  TMC_REQUIRE(events && waves > 0 && waves <= kTimelineWaves,
              "Attention timeline: events must hold 1 .. " + std::to_string(kTimelineWaves) +
                  " waves.");
  const size_t bytes = (size_t)waves * kTimelineEvents * sizeof(uint64_t);
  hipError_t err = hipDeviceSynchronize();
  if (err == hipSuccess) err = hipMemcpyFromSymbol(events, HIP_SYMBOL(timeline), bytes);
  if (err != hipSuccess)
    return fail(std::string("Attention timeline: ") + hipGetErrorString(err));
  return 0;
#else
  (void)events;
  (void)waves;
  return fail("Attention timeline: this library was built without TMC_ATTN_TIMELINE=1 "
              "(libtmc_hip_timeline.so has it).");
#endif
}

extern "C" int tmc_paged_decode_attention_noalloc(
    const void* q, const void* key_pool, const void* value_pool, const int32_t* valid_lengths,
    const int32_t* block_tables, const int32_t* active_count, void* out, int dtype,
    int64_t max_batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t page_size,
    int64_t max_pages, int64_t pool_pages, int64_t page_stride, int64_t head_stride,
    void* stream) {
  clear_error();
  TMC_REQUIRE(page_size > 0 && max_pages > 0 && max_pages <= (INT64_MAX / page_size),
              "Paged attention (no-alloc): invalid page geometry.");
  const size_t need = tmc_attention_workspace_bytes(max_batch, q_heads, kv_heads, head_dim,
                                                    page_size * max_pages);
  // The scratch keeps the merge counters in a fixed area at its start, which
  // no call's slots overlap: every call leaves its counters at zero, so the
  // next call, whatever its shape, finds them zero.
  const size_t counters = counter_bytes(max_batch, kv_heads);
  const size_t slot_need = need > 0 ? need - counters : 0;
  if (counters > kScratchCounterBytes || slot_need > kScratchBytes - kScratchCounterBytes)
    return fail("Paged attention (no-alloc): these limits need " + std::to_string(need) +
                " bytes of split workspace; the static scratch holds " +
                std::to_string(kScratchBytes - kScratchCounterBytes) + " bytes of slots and " +
                std::to_string(kScratchCounterBytes / 4) +
                " merge counters (use tmc_paged_decode_attention).");
  void* ws = nullptr;
  if (need > 0 && scratch_address(&ws)) return 1;
  int* arrivals = need > 0 ? static_cast<int*>(ws) : nullptr;
  float* slots =
      need > 0 ? reinterpret_cast<float*>(static_cast<char*>(ws) + kScratchCounterBytes) : nullptr;
  return paged_attention_impl(q, key_pool, value_pool, valid_lengths, block_tables, active_count,
                              out, dtype, max_batch, q_heads, kv_heads, head_dim, page_size,
                              max_pages, pool_pages, page_stride, head_stride, slots, arrivals,
                              stream);
}

// ------------------------------------------------------------ gather probe
// Bandwidth probe of the paged decode-attention access pattern: reads the K
// and V bytes a launch of tmc_paged_decode_attention (D = 128) reads, page by
// page through the same block tables, and nothing else (no scores, no
// partials).  Block (kv head, 128-position split, request); 16 lanes cover a
// position's 256 bytes, and each thread keeps four 16-byte loads of K and of
// V in flight.  Pages hold a multiple of 16 positions.  The xor of the loaded words reaches `sink` only when it equals
// a fixed constant, which keeps the loads without writing memory.
namespace tmc {
namespace {

constexpr int kProbeChunk = 128;
constexpr int kProbeDepth = 4;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void gather_probe_kernel(
    const u32x4* k, const u32x4* v, const int32_t* lengths, const int32_t* tables, int max_pages,
    int page_size, long page_stride, long head_stride, long pool_pages, uint32_t* sink) {
  const int kvh = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
  const int length = lengths[b];
  const int begin = split * kProbeChunk;
  if (length < 1 || length > max_pages * page_size || begin >= length) return;
  const int end = min(length, begin + kProbeChunk);
  const int c = threadIdx.x & 15, row = threadIdx.x >> 4;  // 16 positions per pass
  uint32_t acc = 0;
  for (int p0 = begin; p0 < end; p0 += 16 * kProbeDepth) {
    u32x4 a[kProbeDepth], bv[kProbeDepth];
#pragma unroll
    for (int u = 0; u < kProbeDepth; ++u) {
      // 16 positions from a multiple of 16 lie in one page: one table entry,
      // the same for the whole block (a scalar load)
      const int p16 = p0 + 16 * u;
      const int page = p16 < end ? tables[(size_t)b * max_pages + p16 / page_size] : -1;
      const int pos = p16 + row;
      const bool ok = pos < end && page >= 0 && (pool_pages == 0 || page < pool_pages);
      const size_t off = ok ? ((size_t)page * page_stride + (size_t)kvh * head_stride +
                               (size_t)(pos % page_size) * 128) / 8 + c
                            : 0;
      const u32x4 none = {0u, 0u, 0u, 0u};
      a[u] = ok ? __builtin_nontemporal_load(k + off) : none;
      bv[u] = ok ? __builtin_nontemporal_load(v + off) : none;
    }
#pragma unroll
    for (int u = 0; u < kProbeDepth; ++u) acc ^= a[u].x ^ a[u].w ^ bv[u].y ^ bv[u].z;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace
}  // namespace tmc

extern "C" int tmc_paged_gather_probe(const void* key_pool, const void* value_pool,
                                      const int32_t* valid_lengths, const int32_t* block_tables,
                                      int64_t batch, int64_t kv_heads, int64_t head_dim,
                                      int64_t page_size, int64_t max_pages, int64_t pool_pages,
                                      int64_t page_stride, int64_t head_stride, void* sink,
                                      void* stream) {
  TMC_REQUIRE(key_pool && value_pool && valid_lengths && block_tables && sink,
              "Gather probe: null pointer.");
  TMC_REQUIRE(head_dim == 128, "Gather probe: head_dim must be 128.");
  TMC_REQUIRE(page_size % 16 == 0, "Gather probe: page_size must be a multiple of 16.");
  TMC_REQUIRE(batch > 0 && batch < 65536 && kv_heads > 0 && kv_heads < 65536 && page_size > 0 &&
                  max_pages > 0 && page_size * max_pages < (1LL << 30) && pool_pages >= 0 &&
                  page_stride > 0 && head_stride >= 0 && page_stride % 8 == 0 &&
                  head_stride % 8 == 0,
              "Gather probe: invalid geometry.");
  TMC_REQUIRE(aligned16(key_pool) && aligned16(value_pool),
              "Gather probe: pools must be 16-byte aligned.");
  const int64_t splits = (page_size * max_pages + kProbeChunk - 1) / kProbeChunk;
  TMC_REQUIRE(splits < 65536, "Gather probe: capacity too large.");
  hipLaunchKernelGGL(gather_probe_kernel, dim3((unsigned)kv_heads, (unsigned)splits, (unsigned)batch),
                     dim3(kThreads), 0, as_stream(stream), static_cast<const u32x4*>(key_pool),
                     static_cast<const u32x4*>(value_pool), valid_lengths, block_tables,
                     (int)max_pages, (int)page_size, (long)page_stride, (long)head_stride,
                     (long)pool_pages, static_cast<uint32_t*>(sink));
  return check_launch("gather_probe_kernel");
}

// ------------------------------------------------ attention + o projection
// Batch-1 decode: the paged attention of every head and the output
// projection y = Wo . context (+ residual) in one launch.  Reference: the
// fusion candidate emitPagedAttentionOutputProjection
// (DecoderLLMMetalEmitter.cpp:623-698, one threadgroup walks every head and
// then every output row), admitted by the decoder only when it times faster
// (DecoderLLMExecutor.cpp:648-713); the optional residual add is the one of
// emitLinearResidual (:604-621).
//
// Block (kv head h, slice s), 16 waves.  Waves 0-7 compute the attention of
// the GROUP query heads of h over the whole row with the MFMA steps of
// attn_mfma_kernel.  Meanwhile waves 8-15 load the block's weight slice, rows
// [s*ROWS, (s+1)*ROWS) x the GROUP*128 columns of those heads, into
// registers (a load retires in issue order per wave, so separate waves keep
// the attention's loads from waiting behind their own weights).  The
// context is rounded to fp16, as the attention kernel stores it, and the
// weight waves form the block's partial sums over its columns.  The two
// roles run in separate wave-uniform branches that pass the same LDS
// barriers, so the held weights never share registers with the attention.
//
// Cross-block sum: each block writes its ROWS partials to the workspace with
// agent-scope stores (written through to memory), waits until they have
// completed, and then counts itself in the slice's arrival counter.  The
// block that arrives last loads the kv heads' partials with agent-scope
// loads, sums them in head order (so the result does not depend on which
// block is last), rounds, adds the residual, stores y and resets the
// counter.  No block waits for another, and since every shared word is
// written and read with agent-scope operations no L2 writeback or
// invalidate is needed.  Blocks are dealt to the 8 XCDs round robin; the
// slices of one kv head are placed on one XCD, so its K/V comes from memory
// once and from that XCD's L2 for the other slices.
//
// Measured on MI355X at Llama-7B widths (32 heads, hidden 4096, 16 rotating
// weight copies, HIP graph): 14.6 us per launch at 132 positions against
// 13.1 us for the attention kernel followed by the residual GEMV, 22.1
// against 20.1 us at 1024.  The weight stream alone takes 7.5 us in this
// form, the cross-block sum 3.4 us, and the attention 3.4 us more: cross-CU
// handoffs cost about what a kernel boundary does on this chip.  A form with
// separate attention and weight blocks (no cross-block sum, a bounded wait
// for the context) measured 16.5 us: 128 weight CUs stream too slowly, and
// CUs shared with weights delay the attention's loads.
namespace tmc {
namespace {

constexpr int kAoWaves = 16;
constexpr int kAoAttnWaves = 8;
constexpr int kAoWeightWaves = kAoWaves - kAoAttnWaves;
constexpr int kAoMaxPages = kMfmaMaxChunk / 16;  // one-split rows, pages of >= 16 positions
constexpr int kAoSumBatch = 32;                   // kv-head partials loaded together

struct AttnOutParams {
  AttnParams a;
  const half_t* w;         // [n_out][in_features]
  const half_t* residual;  // [n_out] or null
  half_t* y;               // [n_out]
  float* partial;          // [kv_heads][n_out]
  int* arrivals;           // [slices]
  int n_out, in_features;
  int xcd_heads;           // kv heads per XCD when slices are grouped by XCD, else 0
};

// Output rows per block: 8 weight waves x NL loads x (64 / lanes per row).
template <int GROUP, int NL> constexpr int ao_rows() { return kAoWeightWaves * NL * (4 / GROUP); }

template <int GROUP, int NL>
__global__ __launch_bounds__(kAoWaves * kWave) void attn_out_kernel(AttnOutParams P) {
  constexpr int D = 128;
  constexpr int LPR = GROUP * 16;  // lanes per weight row (16-byte chunks of GROUP*128 columns)
  constexpr int RPL = kWave / LPR;  // rows per wave load
  constexpr int ROWS = ao_rows<GROUP, NL>();
  constexpr int WAVES = kAoAttnWaves;
  __shared__ float s_m[WAVES][GROUP];
  __shared__ float s_l[WAVES][GROUP];
  __shared__ float s_o[WAVES][GROUP][D];
  __shared__ float s_p[WAVES][kMfmaStep][GROUP];
  __shared__ int s_pages[kAoMaxPages];
  __shared__ __align__(16) half_t s_ctx[GROUP * D];
  __shared__ float s_part[ROWS];
  __shared__ int s_bad, s_last;

  const AttnParams& p = P.a;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  int kvh, slice;
  if (P.xcd_heads > 0) {
    const int xcd = blockIdx.x & 7, local = blockIdx.x >> 3;
    kvh = xcd + 8 * (local % P.xcd_heads);
    slice = local / P.xcd_heads;
  } else {
    kvh = blockIdx.x % p.kv_heads;
    slice = blockIdx.x / p.kv_heads;
  }
  const int row0 = slice * ROWS;

  // Barriers shared by both roles: (1) pages known, (2) wave partials in
  // LDS, (3) context in LDS; the weight waves then write the block's sums.
  if (wave < WAVES) {
    const int j = lane & 15, g = lane >> 4;
    // What the attention waits on goes out in one round trip, unconditionally
    // (clamped addresses; a conditional load becomes a branch whose join
    // waits for it): the block table (at most 64 pages), the active count,
    // the length and q.  MFMA column j >= GROUP repeats head GROUP-1; those
    // score columns are never read (each column of the product is
    // independent).
    const int early_page = p.tables[min(lane, p.max_pages - 1)];
    const int active_word = (p.active ? p.active : p.valid)[0];
    const int valid = p.valid[0];
    h8 qb[4];
    {
      const half_t* qrow = p.q + (size_t)(kvh * GROUP + min(j, GROUP - 1)) * D;
#pragma unroll
      for (int s = 0; s < 4; ++s) qb[s] = load_h8(qrow + 8 * (4 * s + g));
    }
    // An inactive row, an invalid length or a missing page leaves y
    // untouched (the attention kernel leaves its output untouched then).
    // Every attention wave checks the pages (the same ballot), so that no
    // load is sunk into wave 0's branch behind another's wait.
    const int active_rows = p.active ? active_word : INT_MAX;
    const bool run = active_rows > 0 && valid >= 1 && valid <= p.capacity;
    const int entries = run ? page_of(p, valid - 1) + 1 : 0;
    const bool mine = lane < entries;
    const bool bad = !run || __ballot(mine && !page_ok<1>(p, early_page)) != 0;
    if (wave == 0) {
      if (mine) s_pages[lane] = early_page;
      if (lane == 0) s_bad = bad;
    }
    lds_barrier();  // (1)
    float m = -INFINITY, lsum = 0.0f;
    float o[GROUP][8];
#pragma unroll
    for (int h = 0; h < GROUP; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] = 0.0f;
    if (!bad) {
      const __amdgpu_buffer_rsrc_t rk = buffer_of(p.k, p.kv_bytes);
      const __amdgpu_buffer_rsrc_t rv = buffer_of(p.v, p.kv_bytes);
      float (*s_pw)[GROUP] = s_p[wave];
      for (int p0 = kMfmaStep * wave; p0 < valid; p0 += kMfmaStep * WAVES) {
        KvStep<1> st;
        issue_step<1>(p, s_pages, 0, 0, kvh, p0, valid, j, g, rk, rv, st);
        consume_step<GROUP, 1>(p, s_pages, 0, st, qb, p0, valid, j, g, s_pw, m, lsum, o);
      }
    }
#pragma unroll
    for (int h = 0; h < GROUP; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] = cross_sum<16>(o[h][e]);
    lsum = cross_sum<16>(lsum);
    if (g == 0) {
#pragma unroll
      for (int h = 0; h < GROUP; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) s_o[wave][h][8 * j + e] = o[h][e];
      if (j < GROUP) {
        s_m[wave][j] = m;
        s_l[wave][j] = lsum;
      }
    }
    lds_barrier();  // (2)
    // Context of query head kvh*GROUP + h, column d (the merge of
    // finish_split), rounded to fp16.
    if ((int)threadIdx.x < GROUP * D) {
      const int h = threadIdx.x / D, d = threadIdx.x % D;
      float mx = s_m[0][h];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) mx = fmaxf(mx, s_m[w][h]);
      float l = 0.0f, acc = 0.0f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        const float scale = s_m[w][h] == -INFINITY ? 0.0f : fast_exp2(s_m[w][h] - mx);
        l += scale * s_l[w][h];
        acc += scale * s_o[w][h][d];
      }
      s_ctx[threadIdx.x] = (half_t)(acc / l);
    }
    lds_barrier();  // (3)
  } else {
    // The block's weight slice: lane (row r of each load, 16-byte chunk c).
    const int r = lane / LPR, c = lane % LPR;
    const int first = (wave - WAVES) * NL * RPL + r;
    const half_t* base = P.w + (size_t)(row0 + first) * P.in_features +
                         (size_t)kvh * GROUP * D + 8 * c;
    h8 wt[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) wt[i] = load_h8_stream(base + (size_t)i * RPL * P.in_features);
    lds_barrier();  // (1)
    lds_barrier();  // (2)
    lds_barrier();  // (3)
    const h8 cx = *reinterpret_cast<const h8*>(s_ctx + 8 * c);
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      float s = group_sum<16>(dot8(wt[i], cx, 0.0f));
      if constexpr (LPR == 32) s += __shfl_xor(s, 16, kWave);
      if (c == 0) s_part[first + RPL * i] = s;
    }
  }
  __syncthreads();
  const bool bad = s_bad != 0;

  float* part = P.partial + (size_t)kvh * P.n_out + row0;
  for (int t = threadIdx.x; t < ROWS; t += kAoWaves * kWave)
    __hip_atomic_store(part + t, s_part[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(P.arrivals + slice, 1, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) == p.kv_heads - 1;
  __syncthreads();
  if (!s_last) return;
  if (threadIdx.x == 0)
    __hip_atomic_store(P.arrivals + slice, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (bad) return;
  // kAoSumBatch partials per round trip (indices clamped, extra ones
  // ignored); the residual load is unconditional (y stands in when absent).
  const half_t* res_row = P.residual ? P.residual : P.y;
  for (int t = threadIdx.x; t < ROWS; t += kAoWaves * kWave) {
    const int row = row0 + t;
    const float res = (float)res_row[row];
    const float* col = P.partial + row;
    float acc = 0.0f;
    for (int h0 = 0; h0 < p.kv_heads; h0 += kAoSumBatch) {
      float v[kAoSumBatch];
#pragma unroll
      for (int u = 0; u < kAoSumBatch; ++u)
        v[u] = __hip_atomic_load(col + (size_t)min(h0 + u, p.kv_heads - 1) * P.n_out,
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int u = 0; u < kAoSumBatch; ++u) acc += h0 + u < p.kv_heads ? v[u] : 0.0f;
    }
    const half_t out = (half_t)acc;
    P.y[row] = P.residual ? (half_t)(res + (float)out) : out;
  }
}

struct AoShape {
  int nl;      // weight loads per lane (16, 8 or 4), 0 when none fits
  int rows;    // output rows per block
  int slices;  // blocks per kv head
};

AoShape ao_shape(int64_t group, int64_t out_features) {
  for (int nl : {16, 8, 4}) {
    const int rows = kAoWeightWaves * nl * (int)(4 / group);
    if (out_features > 0 && out_features % rows == 0)
      return {nl, rows, (int)(out_features / rows)};
  }
  return {0, 0, 0};
}

// Workspace: the slices' arrival counters (256-byte aligned), then the
// partial sums [kv_heads][out_features] in fp32.
size_t ao_counter_bytes(int slices) { return ((size_t)slices * sizeof(int) + 255) / 256 * 256; }

template <int GROUP>
void launch_attn_out(const AttnOutParams& P, int nl, unsigned blocks, hipStream_t stream) {
  const dim3 block(kAoWaves * kWave);
  if (nl == 16)
    hipLaunchKernelGGL((attn_out_kernel<GROUP, 16>), dim3(blocks), block, 0, stream, P);
  else if (nl == 8)
    hipLaunchKernelGGL((attn_out_kernel<GROUP, 8>), dim3(blocks), block, 0, stream, P);
  else
    hipLaunchKernelGGL((attn_out_kernel<GROUP, 4>), dim3(blocks), block, 0, stream, P);
}

}  // namespace
}  // namespace tmc

extern "C" size_t tmc_attention_output_workspace_bytes(int64_t q_heads, int64_t kv_heads,
                                                       int64_t out_features) {
  if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || q_heads / kv_heads > 2) return 0;
  const AoShape shape = ao_shape(q_heads / kv_heads, out_features);
  if (shape.nl == 0) return 0;
  return ao_counter_bytes(shape.slices) + (size_t)kv_heads * out_features * sizeof(float);
}

extern "C" int tmc_paged_attention_output_f16(
    const void* q, const void* key_pool, const void* value_pool, const int32_t* valid_lengths,
    const int32_t* block_tables, const int32_t* active_count, const void* weight,
    const void* residual, void* y, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
    int64_t page_size, int64_t max_pages, int64_t pool_pages, int64_t page_stride,
    int64_t head_stride, int64_t out_features, void* workspace, size_t workspace_bytes,
    void* stream) {
  clear_error();
  TMC_REQUIRE(q && key_pool && value_pool && valid_lengths && block_tables && weight && y,
              "Paged attention/output fusion: null device pointer.");
  TMC_REQUIRE(head_dim == 128, "Paged attention/output fusion: head_dim must be 128.");
  TMC_REQUIRE(q_heads > 0 && kv_heads > 0 && q_heads < 65536 && q_heads % kv_heads == 0 &&
                  (q_heads / kv_heads == 1 || q_heads / kv_heads == 2),
              "Paged attention/output fusion: q_heads / kv_heads must be 1 or 2.");
  TMC_REQUIRE(page_size >= 16 && page_size % 16 == 0 && max_pages > 0 &&
                  page_size * max_pages <= kMfmaMaxChunk,
              "Paged attention/output fusion: pages must hold a multiple of 16 positions and the "
              "capacity (page_size * max_pages) at most 1024.");
  TMC_REQUIRE(page_stride > 0 && head_stride >= 0 && page_stride % 8 == 0 &&
                  head_stride % 8 == 0 &&
                  (kv_heads - 1) * head_stride + page_size * head_dim <= page_stride,
              "Paged attention/output fusion: invalid page geometry (strides must be multiples "
              "of 8 elements and a page's kv heads must fit its stride).");
  TMC_REQUIRE(pool_pages > 0 && (uint64_t)pool_pages * (uint64_t)page_stride * 2 < kAbsent,
              "Paged attention/output fusion: each pool must hold a known number of pages and "
              "less than 4 GiB.");
  const AoShape shape = ao_shape(q_heads / kv_heads, out_features);
  TMC_REQUIRE(shape.nl > 0 && out_features < (1LL << 24),
              "Paged attention/output fusion: out_features must be a multiple of " +
                  std::to_string(kAoWeightWaves * 4 * (4 / (q_heads / kv_heads))) + ".");
  TMC_REQUIRE(aligned16(q) && aligned16(key_pool) && aligned16(value_pool) && aligned16(weight),
              "Paged attention/output fusion: q, pools and weight must be 16-byte aligned.");
  const size_t need = tmc_attention_output_workspace_bytes(q_heads, kv_heads, out_features);
  TMC_REQUIRE(workspace && workspace_bytes >= need,
              "Paged attention/output fusion: workspace is smaller than "
              "tmc_attention_output_workspace_bytes().");
  AttnOutParams P{};
  AttnParams& p = P.a;
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(key_pool);
  p.v = static_cast<const half_t*>(value_pool);
  p.valid = valid_lengths;
  p.tables = block_tables;
  p.active = active_count;
  p.page_stride = (long)page_stride;
  p.head_stride = (long)head_stride;
  p.q_heads = (int)q_heads;
  p.kv_heads = (int)kv_heads;
  p.capacity = (int)(page_size * max_pages);
  p.page_size = (int)page_size;
  p.page_shift = page_shift_of(page_size);
  p.pool_pages = (long)pool_pages;
  p.kv_bytes = (unsigned)((uint64_t)pool_pages * page_stride * 2);
  p.max_pages = (int)max_pages;
  p.chunk = p.capacity;
  p.max_splits = 1;
  p.waves = kAoAttnWaves;
  p.scale_log2 = (float)(1.0 / std::sqrt((double)head_dim)) * 1.4426950408889634f;
  P.w = static_cast<const half_t*>(weight);
  P.residual = static_cast<const half_t*>(residual);
  P.y = static_cast<half_t*>(y);
  P.arrivals = static_cast<int*>(workspace);
  P.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                       ao_counter_bytes(shape.slices));
  P.n_out = (int)out_features;
  P.in_features = (int)(q_heads * head_dim);
  const int64_t blocks = kv_heads * shape.slices;
  TMC_REQUIRE(blocks < (1LL << 31), "Paged attention/output fusion: too many blocks.");
  P.xcd_heads = kv_heads % 8 == 0 ? (int)(kv_heads / 8) : 0;
  if (q_heads == kv_heads)
    launch_attn_out<1>(P, shape.nl, (unsigned)blocks, as_stream(stream));
  else
    launch_attn_out<2>(P, shape.nl, (unsigned)blocks, as_stream(stream));
  return check_launch("attn_out_kernel");
}
