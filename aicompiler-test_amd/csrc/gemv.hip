// Decode GEMV family for gfx950: fp16 weights [out, in] row-major, fp32
// accumulation.  The fast algorithms stream every weight byte once:
//
//  * Wave64 split-K dot (algorithm 1, batch <= 8).  A wave owns RPW output
//    rows; its 64 lanes split K in 16-byte chunks (lane l reads chunks
//    l, l+64, ...: coalesced 1 KiB per wave per load), issue U*RPW chunk loads
//    before any math, accumulate with v_dot2_f32_f16 and reduce the 64 lane
//    partials with DPP row sums + v_readlane.  KS waves of a block may share
//    a row group (each takes every KS-th chunk) and meet in LDS, which keeps
//    enough waves in flight when N is small.  (Reference: emitDecodeGEMV,
//    DecodeGEMVMetalEmitter.cpp:68-132, one threadgroup per output.)
//  * MFMA skinny GEMM (algorithm 2, any batch): v_mfma_f32_16x16x32_f16 over
//    16 output rows x 16*MT batch rows; KS waves of a block split K in
//    128-element tiles, U tiles of loads in flight per wave, partials summed
//    in LDS.  The x operand costs one 16-byte load per weight load whatever
//    the batch, so it is the path for batch > 1.
//
//  * Linear baseline (algorithm 4): one thread per output, the reference
//    tuner's baseline kept as the tuners' fallback.
//
//  * MFMA row-tile GEMM (algorithm 3, batch <= 16 per pass): the same
//    instruction, but a wave owns RT 16-row output tiles (one activation
//    fragment serves RT weight fragments) and every operand is read with raw
//    buffer loads: rows past N, batch rows past B and k past K get an
//    offset beyond the buffer, which reads as zero, so no load is
//    predicated.  KS waves of a block split K; all waves share the LDS
//    reduction.
//
// The gated MLP (emitDecoderGatedMLP, DecoderLLMMetalEmitter.cpp:479-536)
// runs either algorithm over the Wg and Wu rows of each feature and finishes
// with the reference rounding points h(h(silu(h(g))) * h(u)).
#include <algorithm>
#include <cmath>

#include "tmc_abi.hpp"
#include "tmc_device.hpp"

namespace tmc {
namespace {

__device__ __forceinline__ half_t silu_mul_h(float gate_sum, float up_sum) {
  const float g = through<half_t>(gate_sum);
  const float u = through<half_t>(up_sum);
  const float activated = through<half_t>(g / (1.0f + expf(-g)));
  return (half_t)(activated * u);
}

// Output writer shared by the plain GEMV and the gated MLP: MATS = 1 writes
// y = OutT(acc0); MATS = 2 writes y = silu_mul_h(acc0, acc1).
template <int MATS, typename OutT>
__device__ __forceinline__ void write_out(OutT* y, size_t i, float a0, float a1) {
  if constexpr (MATS == 1) {
    y[i] = from_float<OutT>(a0);
  } else {
    y[i] = silu_mul_h(a0, a1);
  }
}

// ---------------------------------------------------------------- wave64 dot
// Fusions of the batch-1 dot GEMV:
//  * kFuseAddNorm / kFuseNorm (gemv_norm_kernel): the input is x = h(s *
//    rsqrt(mean(s^2) + eps) * gamma) of a stored row s (kFuseAddNorm: s =
//    h(residual + update), stored to sum_out by block 0; kFuseNorm: s =
//    residual), computed in the kernel instead of by a norm launch.  The sum
//    of squares runs in the order of norm_vec_kernel with one 16-byte chunk
//    per thread: thread t owns chunk t, its 8 squares are added in order,
//    each group of 64 chunks is reduced by wave_sum, and the group totals are
//    added in group order.  That order does not depend on the thread count
//    once every thread holds at most one chunk (idle threads add exact
//    zeros), so x equals tmc_rmsnorm / tmc_add_rmsnorm at any thread count
//    >= k / 8 bit for bit.
//  * kFuseResidual (gemv_dot_kernel): the output is h(residual + h(W x)), the
//    residual add of emitLinearResidual (DecoderLLMMetalEmitter.cpp:604-622),
//    so the add no longer needs the norm kernel that follows.
enum Fuse { kFuseNone = 0, kFuseAddNorm = 1, kFuseNorm = 2, kFuseResidual = 3 };

struct NormArgs {
  const half_t* x = nullptr;  // kFuseNone / kFuseResidual in gemv_norm_kernel: the input row
  const half_t* residual = nullptr;
  const half_t* update = nullptr;
  const half_t* gamma = nullptr;
  half_t* sum_out = nullptr;
  float eps = 0.0f;
};

// Streaming 16-byte weight load through a buffer resource (non-temporal).
__device__ __forceinline__ h8 buffer_stream_h8(__amdgpu_buffer_rsrc_t r, unsigned byte_offset) {
  return __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_offset, 0, 2));
}

template <int MATS, int FUSE, typename OutT>
__device__ __forceinline__ void store_out(OutT* y, size_t i, float a0, float a1,
                                          const NormArgs& na) {
  if constexpr (FUSE == kFuseResidual) {
    static_assert(MATS == 1, "the residual epilogue follows a plain projection");
    const float projected = to_float<half_t>(from_float<half_t>(a0));
    y[i] = from_float<half_t>(to_float<half_t>(na.residual[i]) + projected);
  } else {
    write_out<MATS>(y, i, a0, a1);
  }
}

template <int MATS, int NB, int RPW, int U, int KS, typename OutT, int FUSE = kFuseNone,
          bool ROPE = false>
__global__ __launch_bounds__(256) void gemv_dot_kernel(const half_t* __restrict__ x,
                                                      const half_t* __restrict__ w0,
                                                      const half_t* __restrict__ w1,
                                                      OutT* __restrict__ y, int n_out, int k_in,
                                                      NormArgs na, RopeArgs ra) {
  static_assert(!ROPE || (MATS == 1 && NB == 1 && RPW == 2),
                "the RoPE epilogue takes one projection row pair per wave at batch 1");
  static_assert(FUSE == kFuseNone || FUSE == kFuseResidual, "norm fusions run gemv_norm_kernel");
  static_assert(FUSE != kFuseResidual || (NB == 1 && !ROPE && MATS == 1),
                "the residual epilogue serves a batch-1 projection");
  constexpr int kWaves = 4;
  constexpr int kGroups = kWaves / KS;
  __shared__ float partial[kWaves][MATS][RPW][NB];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int group = wave / KS;
  const int part = wave % KS;
  const int row0 = (blockIdx.x * kGroups + group) * RPW;
  const bool live = row0 < n_out;  // wave-uniform; dead waves still meet the barrier
  const int chunks = k_in >> 3;
  const half_t* wrow[MATS][RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const size_t off = (size_t)min(row0 + r, n_out - 1) * k_in;
    wrow[0][r] = w0 + off;
    if constexpr (MATS == 2) wrow[1][r] = w1 + off;
  }
  float acc[MATS][RPW][NB];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[m][r][b] = 0.0f;

  constexpr int stride = kWave * KS;
  int c = live ? lane + kWave * part : chunks;
  for (; c + stride * (U - 1) < chunks; c += stride * U) {
    h8 wv[U][MATS][RPW];
    h8 xv[U][NB];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int r = 0; r < RPW; ++r) wv[u][m][r] = load_h8_stream(wrow[m][r] + 8 * (c + stride * u));
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int b = 0; b < NB; ++b) xv[u][b] = load_h8(x + (size_t)b * k_in + 8 * (c + stride * u));
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
          for (int b = 0; b < NB; ++b) acc[m][r][b] = dot8(wv[u][m][r], xv[u][b], acc[m][r][b]);
  }
  for (; c < chunks; c += stride) {
    h8 xv[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) xv[b] = load_h8(x + (size_t)b * k_in + 8 * c);
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const h8 w = load_h8_stream(wrow[m][r] + 8 * c);
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[m][r][b] = dot8(w, xv[b], acc[m][r][b]);
      }
  }
  if constexpr (ROPE && KS == 1) {
    const float even = wave_sum(acc[0][0][0]);
    const float odd = wave_sum(acc[0][1][0]);
    if (lane == 0 && live) rope_append_pair(ra, 0, row0, even, odd);
  } else if constexpr (KS == 1) {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float a0 = wave_sum(acc[0][r][b]);
        const float a1 = MATS == 2 ? wave_sum(acc[MATS - 1][r][b]) : 0.0f;
        if (lane == 0 && live && row0 + r < n_out)
          store_out<MATS, FUSE>(y, (size_t)b * n_out + row0 + r, a0, a1, na);
      }
  } else {
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const float total = wave_sum(acc[m][r][b]);
          if (lane == 0) partial[wave][m][r][b] = total;
        }
    __syncthreads();
    if constexpr (ROPE) {
      if (part == 0 && live && lane == 0) {
        float even = 0.0f, odd = 0.0f;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          even += partial[wave + s][0][0][0];
          odd += partial[wave + s][0][1][0];
        }
        rope_append_pair(ra, 0, row0, even, odd);
      }
    } else if (part == 0 && live) {
      for (int idx = lane; idx < RPW * NB; idx += kWave) {
        const int r = idx / NB, b = idx % NB;
        float a[2] = {0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < MATS; ++m)
#pragma unroll
          for (int s = 0; s < KS; ++s) a[m] += partial[wave + s][m][r][b];
        if (row0 + r < n_out) store_out<MATS, FUSE>(y, (size_t)b * n_out + row0 + r, a[0], a[1], na);
      }
    }
  }
}

// Batch-1 dot GEMV (or gated MLP, or q.k.v + RoPE + append) of a normalized
// stored row, as a persistent kernel: the grid holds as many blocks as run at
// once, and block b computes row groups (RPW rows each) b, b + G, b + 2G, ...
// A block's 4 waves split K like the dot GEMV at k split 4: wave p holds the
// 16-byte chunks p*64 + lane + 256*i (i < NC, K <= 2048 * NC), which are also
// the 64-chunk groups p + 4*i of the norm's reduction.  The block loads its
// row chunks and gamma once, and the weights of its first row groups;
// reduces its norm groups (one wave_sum each) and meets the other waves at
// one LDS barrier (the weight loads stay in flight); normalizes its chunks
// once, into registers; then streams its row groups two or three deep, the
// loads of group j + depth issued as group j is consumed.  Weights are read with raw
// buffer loads, a group past the matrix with an out-of-range offset (zeros,
// no memory traffic), so the stream has no branches.  Per-row partials wait
// in LDS until the end and are summed in wave order as in the dot GEMV, so
// results equal the norm kernel followed by tmc_gemv_f16 at k split 4 bit for
// bit.
constexpr int kNormMaxChunks = 1024;  // normalized rows: K <= 8192, four chunks per lane
constexpr int kNormMaxSlots = 35;     // row groups per block (grid >= groups / 32), + overshoot
// Build parameter: blocks of the persistent grid per resident block slot
// (1 = one wave of blocks; 2 = twice as many, each with half the groups).
#ifndef TMC_NORM_GRID_FACTOR
#define TMC_NORM_GRID_FACTOR 1
#endif

template <int FUSE>
__device__ __forceinline__ h8 norm_source(const NormArgs& na, int c) {
  h8 a = load_h8(na.residual + 8 * c);
  if constexpr (FUSE == kFuseAddNorm) {
    const h8 b = load_h8(na.update + 8 * c);
#pragma unroll
    for (int t = 0; t < 8; ++t) a[t] = from_float<half_t>(to_float<half_t>(a[t]) + to_float<half_t>(b[t]));
  }
  return a;
}


// ARGMAX (the token-only LM head, emitLMHeadPartialArgmax,
// DecoderLLMMetalEmitter.cpp:700-728): y is a partial-argmax workspace
// (argmax_partials, one row of n_out slots): instead of storing the block's
// logits, wave 0 keeps the greatest (value, row) of them in the greedy-token
// order and writes it to slot blockIdx.x; block 0 writes the slot count.
// The values are the logits the plain form stores, so the final argmax over
// the slots is the argmax of those logits, ties and NaN included.
template <int MATS, int RPW, int NC, typename OutT, int FUSE, bool ROPE = false,
          bool ARGMAX = false>
__global__ __launch_bounds__(256) void gemv_norm_kernel(const half_t* __restrict__ w0,
                                                       const half_t* __restrict__ w1,
                                                       OutT* __restrict__ y, int n_out, int k_in,
                                                       NormArgs na, RopeArgs ra) {
  // kFuseNone / kFuseResidual: the same stream over a stored input row (no
  // norm prologue, no barrier before the stream), the plain or residual
  // batch-1 GEMV (algorithm 5, "persistent dot")
  constexpr bool kNorm = FUSE == kFuseAddNorm || FUSE == kFuseNorm;
  static_assert(!ROPE || (MATS == 1 && RPW == 2), "the RoPE epilogue takes one row pair");
  static_assert(!ARGMAX || (MATS == 1 && !ROPE), "the argmax epilogue follows one matrix");
  static_assert(FUSE != kFuseResidual || (MATS == 1 && !ROPE && !ARGMAX),
                "the residual epilogue follows one projection");
  static_assert(NC == 1 || NC == 2 || NC == 4 || (!kNorm && (NC == 6 || NC == 8)),
                "1, 2 or 4 chunks per lane (6 or 8 without the norm)");
  // row groups in flight per wave, measured on the 7B shapes: 3 for the gated
  // pair (gate/up 28.2 against 30.5 us at 2), 2 for one matrix (q.k.v 16.4
  // against 16.9 us at 3)
  constexpr int kNormDepth = MATS == 2 ? 3 : 2;
  constexpr int kWaves = 4;
  __shared__ float totals[kNormMaxChunks / kWave];
  __shared__ float partial[kWaves][kNormMaxSlots][MATS][RPW];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int chunks = k_in >> 3;
  const int groups = (n_out + RPW - 1) / RPW;
  const int grid = (int)gridDim.x;
  const unsigned bytes = (unsigned)n_out * (unsigned)k_in * 2u;
  const __amdgpu_buffer_rsrc_t rw0 = buffer_resource(w0, bytes);
  const __amdgpu_buffer_rsrc_t rw1 = buffer_resource(MATS == 2 ? w1 : w0, bytes);
  int c[NC];
  bool ok[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    c[i] = wave * kWave + lane + 4 * kWave * i;
    ok[i] = c[i] < chunks;
  }
  // the row and gamma first (clamped addresses, no branch; chunks past the
  // row are zeroed where they are used, so no select waits on these loads
  // before the weight loads are issued)
  h8 src[NC], gam[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int at = min(c[i], chunks - 1);
    if constexpr (kNorm) {
      src[i] = norm_source<FUSE>(na, at);
      gam[i] = load_h8(na.gamma + 8 * at);
    } else {
      src[i] = load_h8(na.x + 8 * at);
    }
  }
  // weights of row group g: rows past the matrix (clamped to row n_out, so
  // at or past the resource's end) and chunks past the row read as zero.  No
  // select on the block-uniform row test: the compiler would branch on it,
  // and the wait counters are counted conservatively at the join.
  auto load_group = [&](h8 (&w)[NC][MATS][RPW], int g) {
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const unsigned row = (unsigned)min(g * RPW + r, n_out);
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const unsigned off =
            ok[i] ? (row * (unsigned)k_in + 8u * (unsigned)c[i]) * 2u : kBufferAbsent;
        w[i][0][r] = buffer_stream_h8(rw0, off);
        if constexpr (MATS == 2) w[i][1][r] = buffer_stream_h8(rw1, off);
      }
    }
  };
  h8 wa[NC][MATS][RPW], wb[NC][MATS][RPW], wc[NC][MATS][RPW];
  int g = (int)blockIdx.x;
  // keep the row loads ahead of the weight loads (loads return in issue
  // order, so the norm then waits for the row only)
  __builtin_amdgcn_sched_barrier(0);
  load_group(wa, g);
  load_group(wb, g + grid);
  if constexpr (kNormDepth == 3) load_group(wc, g + 2 * grid);
  h8 xn[NC];
  if constexpr (kNorm) {
    // norm: group wave + 4i (past the row: zero); block 0 stores the sums
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      src[i] = ok[i] ? src[i] : h8{};
      float squares = 0.0f;
#pragma unroll
      for (int t = 0; t < 8; ++t) squares += to_float<half_t>(src[i][t]) * to_float<half_t>(src[i][t]);
      const float total = wave_sum(squares);
      if (lane == 0) totals[wave + 4 * i] = total;
    }
    if (FUSE == kFuseAddNorm && blockIdx.x == 0) {
#pragma unroll
      for (int i = 0; i < NC; ++i)
        if (ok[i]) *reinterpret_cast<h8*>(na.sum_out + 8 * c[i]) = src[i];
    }
    lds_barrier();
    float total = 0.0f;
    for (int q = 0; q * kWave < chunks; ++q) total += totals[q];
    const float inverse = 1.0f / sqrtf(total / (float)k_in + na.eps);
#pragma unroll
    for (int i = 0; i < NC; ++i)
#pragma unroll
      for (int t = 0; t < 8; ++t)
        xn[i][t] = from_float<half_t>(to_float<half_t>(src[i][t]) * inverse * to_float<half_t>(gam[i][t]));
  } else {
    // chunks past the row: the weights read as zero there, the products are 0
#pragma unroll
    for (int i = 0; i < NC; ++i) xn[i] = ok[i] ? src[i] : h8{};
  }
  auto consume = [&](const h8 (&w)[NC][MATS][RPW], int slot) {
    float acc[MATS][RPW];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        acc[m][r] = 0.0f;
#pragma unroll
        for (int i = 0; i < NC; ++i) acc[m][r] = dot8(w[i][m][r], xn[i], acc[m][r]);
      }
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const float sum = wave_sum(acc[m][r]);
        if (lane == 0) partial[wave][slot][m][r] = sum;
      }
  };
  int slot = 0;
  for (; g < groups; g += kNormDepth * grid, slot += kNormDepth) {  // block-uniform
    consume(wa, slot);
    load_group(wa, g + kNormDepth * grid);
    consume(wb, slot + 1);
    load_group(wb, g + (kNormDepth + 1) * grid);
    if constexpr (kNormDepth == 3) {
      consume(wc, slot + 2);
      load_group(wc, g + 5 * grid);
    }
  }
  __syncthreads();
  // the block's rows: (slot, row of the group) pairs, wave 0
  if (wave != 0) return;
  if constexpr (ROPE) {
    for (int s = lane; s < slot; s += kWave) {
      const int gg = (int)blockIdx.x + s * grid;
      if (gg >= groups) continue;
      float even = 0.0f, odd = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        even += partial[w][s][0][0];
        odd += partial[w][s][0][1];
      }
      rope_append_pair(ra, 0, gg * RPW, even, odd);
    }
  } else if constexpr (ARGMAX) {
    float best = -INFINITY;
    int selected = -1;
    for (int idx = lane; idx < slot * RPW; idx += kWave) {
      const int s = idx / RPW, r = idx % RPW;
      const int row = ((int)blockIdx.x + s * grid) * RPW + r;
      if (row >= n_out) continue;
      float a = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) a += partial[w][s][0][r];
      if (argmax_better(a, row, best, selected)) {
        best = a;
        selected = row;
      }
    }
    argmax_wave(best, selected);
    if (lane == 0) {
      const ArgmaxPartials out = argmax_partials(y, 1, n_out);
      out.values[blockIdx.x] = best;
      out.indices[blockIdx.x] = selected;
      if (blockIdx.x == 0) *out.count = grid;
    }
  } else {
    for (int idx = lane; idx < slot * RPW; idx += kWave) {
      const int s = idx / RPW, r = idx % RPW;
      const int row = ((int)blockIdx.x + s * grid) * RPW + r;
      if (row >= n_out) continue;
      float a[2] = {0.0f, 0.0f};
#pragma unroll
      for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int w = 0; w < kWaves; ++w) a[m] += partial[w][s][m][r];
      if constexpr (FUSE == kFuseResidual)
        store_out<1, kFuseResidual>(y, (size_t)row, a[0], 0.0f, na);
      else
        write_out<MATS>(y, (size_t)row, a[0], a[1]);
    }
  }
}

// Any K (no 16-byte alignment): one wave per (row, feature), scalar loads.
template <int MATS, typename OutT>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const half_t* __restrict__ x,
                                                          const half_t* __restrict__ w0,
                                                          const half_t* __restrict__ w1,
                                                          OutT* __restrict__ y, int batch,
                                                          int n_out, int k_in) {
  const int lane = threadIdx.x & (kWave - 1);
  const long item = (long)blockIdx.x * 4 + threadIdx.x / kWave;
  if (item >= (long)batch * n_out) return;
  const int b = (int)(item / n_out), n = (int)(item % n_out);
  float a0 = 0.0f, a1 = 0.0f;
  for (int k = lane; k < k_in; k += kWave) {
    const float xv = (float)x[(size_t)b * k_in + k];
    a0 += xv * (float)w0[(size_t)n * k_in + k];
    if constexpr (MATS == 2) a1 += xv * (float)w1[(size_t)n * k_in + k];
  }
  a0 = wave_sum(a0);
  if constexpr (MATS == 2) a1 = wave_sum(a1);
  if (lane == 0) write_out<MATS>(y, (size_t)b * n_out + n, a0, a1);
}

// Linear baseline (algorithm 4), emitLinearBaseline
// (DecodeGEMVMetalEmitter.cpp:18-66): one thread per output element with a
// serial fp32 K loop.  It is the tuners' performance baseline and fallback,
// not a fast path: lanes of a wave read rows K elements apart.
template <int MATS, typename OutT>
__global__ __launch_bounds__(128) void gemv_linear_baseline_kernel(
    const half_t* __restrict__ x, const half_t* __restrict__ w0, const half_t* __restrict__ w1,
    OutT* __restrict__ y, int batch, int n_out, int k_in) {
  const long item = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= (long)batch * n_out) return;
  const int b = (int)(item / n_out), n = (int)(item % n_out);
  const half_t* xr = x + (size_t)b * k_in;
  float a0 = 0.0f, a1 = 0.0f;
  for (int k = 0; k < k_in; ++k) {
    const float xv = (float)xr[k];
    a0 += xv * (float)w0[(size_t)n * k_in + k];
    if constexpr (MATS == 2) a1 += xv * (float)w1[(size_t)n * k_in + k];
  }
  write_out<MATS>(y, (size_t)item, a0, a1);
}

// ---------------------------------------------------------------- MFMA
// D[i][j] = sum_k x[i][k] * w[n0+j][k] for MT 16-row tiles of x.  Lane l
// supplies row l%16 of both operands and k-group g = l/16.  A 128-wide K tile
// is 16 chunks of 8 k; MFMA s of the tile takes chunk 4s+g from group g, so
// the four lanes of a row read 64 contiguous bytes per load instruction.
// Both operands use the same (s, g) -> k assignment, so each MFMA sums
// exactly the tile's k values.
template <int MATS, int MT, int U, typename OutT>
__global__ __launch_bounds__(1024) void mfma_gemm_kernel(const half_t* __restrict__ x,
                                                        const half_t* __restrict__ w0,
                                                        const half_t* __restrict__ w1,
                                                        OutT* __restrict__ y, int m_rows,
                                                        int n_out, int k_in, int ntile_per_block,
                                                        int ksplit) {
  extern __shared__ float red[];  // [waves][MATS][MT][4][64]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nt = wave / ksplit;
  const int ks = wave % ksplit;
  const int j = lane & 15;
  const int g = lane >> 4;
  const int n0 = (blockIdx.x * ntile_per_block + nt) * 16;
  const size_t row_off = (size_t)min(n0 + j, n_out - 1) * k_in;
  const half_t* wrow0 = w0 + row_off;
  const half_t* wrow1 = MATS == 2 ? w1 + row_off : nullptr;
  f4 acc[MATS][MT];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[m][mt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  const h8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  const int tiles = (k_in + 127) / 128;
  const bool live = n0 < n_out;
  for (int t0 = live ? ks : tiles; t0 < tiles; t0 += ksplit * U) {
    h8 wv[U][MATS][4];
    h8 xv[U][MT][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kb = (t0 + u * ksplit) * 128 + 8 * g;
      const bool tile_ok = t0 + u * ksplit < tiles;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int k = kb + 32 * s;
        const bool ok = tile_ok && k < k_in;
        wv[u][0][s] = ok ? load_h8_stream(wrow0 + k) : zero;
        if constexpr (MATS == 2) wv[u][MATS - 1][s] = ok ? load_h8_stream(wrow1 + k) : zero;
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int row = mt * 16 + j;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int k = kb + 32 * s;
          xv[u][mt][s] = (tile_ok && row < m_rows && k < k_in)
                             ? load_h8(x + (size_t)row * k_in + k) : zero;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int s = 0; s < 4; ++s)
            acc[m][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv[u][mt][s], wv[u][m][s],
                                                                acc[m][mt], 0, 0, 0);
  }
  float* mine = red + (size_t)wave * MATS * MT * 4 * kWave;
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) mine[((m * MT + mt) * 4 + r) * kWave + lane] = acc[m][mt][r];
  __syncthreads();
  if (ks != 0 || !live) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float a[2] = {0.0f, 0.0f};
#pragma unroll
      for (int m = 0; m < MATS; ++m)
        for (int s = 0; s < ksplit; ++s)
          a[m] += red[(size_t)(wave + s) * MATS * MT * 4 * kWave + ((m * MT + mt) * 4 + r) * kWave +
                      lane];
      const int row = mt * 16 + 4 * g + r;
      const int col = n0 + j;
      if (row < m_rows && col < n_out) write_out<MATS>(y, (size_t)row * n_out + col, a[0], a[1]);
    }
}

// ---------------------------------------------------------------- MFMA row tiles
constexpr unsigned kNoData = 0xFFFFFFF0u;  // buffer offset that reads as zero

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ h8 rsrc_h8(__amdgpu_buffer_rsrc_t r, unsigned byte_offset) {
  return __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_offset, 0, 0));
}

// Block = KS waves over RT tiles of 16 output rows; wave ks takes a
// contiguous run of K tiles (128 k), U adjacent tiles per round trip.  Lane (j = l % 16,
// g = l / 16): A = activations (batch row j, k chunk 4s+g of the tile), B =
// weights (output row j of the tile, same k chunk); acc[r] = out[batch
// 4g + r][row j].
template <int MATS, int RT, int U, typename OutT>
__global__ __launch_bounds__(1024) void mfma_rows_kernel(const half_t* __restrict__ x,
                                                        const half_t* __restrict__ w0,
                                                        const half_t* __restrict__ w1,
                                                        OutT* __restrict__ y, int m_rows,
                                                        int n_out, int k_in, int ks_count) {
  extern __shared__ float red[];  // [ks][MATS][RT][4][64]
  const int lane = threadIdx.x & (kWave - 1);
  const int ks = threadIdx.x / kWave;
  const int j = lane & 15;
  const int g = lane >> 4;
  const int n0 = blockIdx.x * RT * 16;
  const unsigned x_bytes = (unsigned)m_rows * (unsigned)k_in * 2u;
  const unsigned w_bytes = (unsigned)n_out * (unsigned)k_in * 2u;
  const __amdgpu_buffer_rsrc_t rx = rsrc_of(x, x_bytes);
  const __amdgpu_buffer_rsrc_t rw0 = rsrc_of(w0, w_bytes);
  const __amdgpu_buffer_rsrc_t rw1 = rsrc_of(MATS == 2 ? w1 : w0, w_bytes);
  const unsigned x_row = j < m_rows ? (unsigned)j * (unsigned)k_in * 2u : kNoData;
  unsigned w_row[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = n0 + rt * 16 + j;
    w_row[rt] = row < n_out ? (unsigned)row * (unsigned)k_in * 2u : kNoData;
  }
  f4 acc[MATS][RT];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[m][rt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  // Wave ks owns the contiguous K tiles [first, last): the U tiles of one
  // round trip are adjacent, so each weight row is read in U*256-byte runs.
  const int tiles = (k_in + 127) / 128;
  const int per_wave = (tiles + ks_count - 1) / ks_count;
  const int first = ks * per_wave;
  const int last = min(tiles, first + per_wave);
  for (int t0 = first; t0 < last; t0 += U) {
    h8 xv[U][4], wv[U][MATS][RT][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int k = (t0 + u) * 128 + 32 * s + 8 * g;
        const bool kok = t0 + u < last && k < k_in;
        const unsigned kb = (unsigned)k * 2u;
        xv[u][s] = rsrc_h8(rx, kok && x_row != kNoData ? x_row + kb : kNoData);
        // default cache policy for the weights: the non-temporal hint
        // measured slower here (C2 at batch 8, row-major: 3.90 -> 3.71 TB/s)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const unsigned off = kok && w_row[rt] != kNoData ? w_row[rt] + kb : kNoData;
          wv[u][0][rt][s] = rsrc_h8(rw0, off);
          if constexpr (MATS == 2) wv[u][1][rt][s] = rsrc_h8(rw1, off);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int m = 0; m < MATS; ++m)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
            acc[m][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv[u][s], wv[u][m][rt][s],
                                                                acc[m][rt], 0, 0, 0);
  }
  constexpr int kValues = MATS * RT * 4;  // per lane
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        red[((size_t)ks * kValues + (m * RT + rt) * 4 + r) * kWave + lane] = acc[m][rt][r];
  __syncthreads();
  // Every thread finishes some (rt, r, lane) outputs: sum the KS partials.
  const int total = RT * 4 * kWave;
  for (int idx = threadIdx.x; idx < total; idx += ks_count * kWave) {
    const int l = idx % kWave, rt = (idx / kWave) / 4, r = (idx / kWave) % 4;
    float a[2] = {0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < MATS; ++m)
      for (int w = 0; w < ks_count; ++w)
        a[m] += red[((size_t)w * kValues + (m * RT + rt) * 4 + r) * kWave + l];
    const int row = 4 * (l >> 4) + r;       // batch row
    const int col = n0 + rt * 16 + (l & 15);  // output feature
    if (row < m_rows && col < n_out) write_out<MATS>(y, (size_t)row * n_out + col, a[0], a[1]);
  }
}

// ---------------------------------------------------------------- dispatch

struct Shape {
  const half_t* x;
  const half_t* w0;
  const half_t* w1;
  void* y;
  int y_dtype, batch, n, k;
};

template <int MATS, int NB, int RPW, int U, int KS, typename OutT, int FUSE = kFuseNone,
          bool ROPE = false>
int launch_dot(const Shape& s, const half_t* x, OutT* y, hipStream_t stream,
               const NormArgs& na = NormArgs{}, const RopeArgs& ra = RopeArgs{}) {
  const int rows_per_block = (4 / KS) * RPW;
  const dim3 grid((s.n + rows_per_block - 1) / rows_per_block);
  hipLaunchKernelGGL((gemv_dot_kernel<MATS, NB, RPW, U, KS, OutT, FUSE, ROPE>), grid, dim3(256), 0,
                     stream, x, s.w0, s.w1, y, s.n, s.k, na, ra);
  return check_launch("gemv_dot_kernel");
}

// Batch-1 dot GEMV with a fusion (norm prologue or residual epilogue), by
// configuration.
template <int MATS, typename OutT, int FUSE>
int launch_dot_fused(const Shape& s, OutT* y, const tmc_gemv_config& c, const NormArgs& na,
                     hipStream_t st) {
  const int key = (c.rows_per_wave == 2 ? 100 : 0) + (c.unroll == 2 ? 10 : 0) +
                  (c.k_split == 4 ? 2 : c.k_split == 2 ? 1 : 0);
  switch (key) {
  case 0: return launch_dot<MATS, 1, 1, 4, 1, OutT, FUSE>(s, s.x, y, st, na);
  case 1: return launch_dot<MATS, 1, 1, 4, 2, OutT, FUSE>(s, s.x, y, st, na);
  case 2: return launch_dot<MATS, 1, 1, 4, 4, OutT, FUSE>(s, s.x, y, st, na);
  case 10: return launch_dot<MATS, 1, 1, 2, 1, OutT, FUSE>(s, s.x, y, st, na);
  case 11: return launch_dot<MATS, 1, 1, 2, 2, OutT, FUSE>(s, s.x, y, st, na);
  case 12: return launch_dot<MATS, 1, 1, 2, 4, OutT, FUSE>(s, s.x, y, st, na);
  case 100: return launch_dot<MATS, 1, 2, 4, 1, OutT, FUSE>(s, s.x, y, st, na);
  case 101: return launch_dot<MATS, 1, 2, 4, 2, OutT, FUSE>(s, s.x, y, st, na);
  case 102: return launch_dot<MATS, 1, 2, 4, 4, OutT, FUSE>(s, s.x, y, st, na);
  case 110: return launch_dot<MATS, 1, 2, 2, 1, OutT, FUSE>(s, s.x, y, st, na);
  case 111: return launch_dot<MATS, 1, 2, 2, 2, OutT, FUSE>(s, s.x, y, st, na);
  default: return launch_dot<MATS, 1, 2, 2, 4, OutT, FUSE>(s, s.x, y, st, na);
  }
}

// Batch-1 GEMV / gated MLP / q.k.v + RoPE of a normalized stored row: the
// persistent grid holds at most the blocks resident at once (occupancy x
// CUs, measured once per instance and device) and gives each block the same
// number of row groups, at most 32 (its LDS partials).
template <int MATS, int RPW, int NC, typename OutT, int FUSE, bool ROPE, bool ARGMAX = false>
int launch_norm_gemv_nc(const Shape& s, OutT* y, const NormArgs& na, const RopeArgs& ra,
                        hipStream_t st) {
  auto kernel = gemv_norm_kernel<MATS, RPW, NC, OutT, FUSE, ROPE, ARGMAX>;
  static int resident[64] = {0};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64)
    return fail("gemv_norm_kernel: no current device.");
  if (resident[device] == 0) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        per_cu <= 0 || cus <= 0)
      return fail("gemv_norm_kernel: occupancy query failed.");
    resident[device] = per_cu * cus * TMC_NORM_GRID_FACTOR;
  }
  // as many row groups per block as the resident blocks need, then the
  // fewest blocks that cover the groups with that count, so that every block
  // streams the same number of groups (a block with one extra group would
  // run alone at the end)
  const int groups = (s.n + RPW - 1) / RPW;
  const int per_block = std::min((groups + resident[device] - 1) / resident[device], 32);
  const int grid = (groups + per_block - 1) / per_block;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), 0, st, s.w0, s.w1, y, s.n, s.k, na, ra);
  return check_launch("gemv_norm_kernel");
}

template <int MATS, int RPW, typename OutT, int FUSE, bool ROPE = false, bool ARGMAX = false>
int launch_norm_gemv_rpw(const Shape& s, OutT* y, const NormArgs& na, const RopeArgs& ra,
                         hipStream_t st) {
  const int chunks = s.k / 8;
  if (chunks <= 256)
    return launch_norm_gemv_nc<MATS, RPW, 1, OutT, FUSE, ROPE, ARGMAX>(s, y, na, ra, st);
  if (chunks <= 512)
    return launch_norm_gemv_nc<MATS, RPW, 2, OutT, FUSE, ROPE, ARGMAX>(s, y, na, ra, st);
  if constexpr (MATS == 1 && (FUSE == kFuseNone || FUSE == kFuseResidual)) {
    if (chunks > 1024) {
      if (chunks <= 1536)
        return launch_norm_gemv_nc<MATS, RPW, 6, OutT, FUSE, ROPE, ARGMAX>(s, y, na, ra, st);
      return launch_norm_gemv_nc<MATS, RPW, 8, OutT, FUSE, ROPE, ARGMAX>(s, y, na, ra, st);
    }
  }
  return launch_norm_gemv_nc<MATS, RPW, 4, OutT, FUSE, ROPE, ARGMAX>(s, y, na, ra, st);
}

template <int MATS, typename OutT, int FUSE>
int launch_norm_gemv(const Shape& s, OutT* y, int rows_per_block, const NormArgs& na,
                     hipStream_t st) {
  return rows_per_block == 2
             ? launch_norm_gemv_rpw<MATS, 2, OutT, FUSE>(s, y, na, RopeArgs{}, st)
             : launch_norm_gemv_rpw<MATS, 1, OutT, FUSE>(s, y, na, RopeArgs{}, st);
}

template <int MATS, int NB, typename OutT>
int dot_by_config(const Shape& s, const half_t* x, OutT* y, int rpw, int unroll, int ks,
                  hipStream_t st) {
  const int key = (rpw == 2 ? 100 : 0) + (unroll == 2 ? 10 : 0) + (ks == 4 ? 2 : ks == 2 ? 1 : 0);
  switch (key) {
  case 0: return launch_dot<MATS, NB, 1, 4, 1, OutT>(s, x, y, st);
  case 1: return launch_dot<MATS, NB, 1, 4, 2, OutT>(s, x, y, st);
  case 2: return launch_dot<MATS, NB, 1, 4, 4, OutT>(s, x, y, st);
  case 10: return launch_dot<MATS, NB, 1, 2, 1, OutT>(s, x, y, st);
  case 11: return launch_dot<MATS, NB, 1, 2, 2, OutT>(s, x, y, st);
  case 12: return launch_dot<MATS, NB, 1, 2, 4, OutT>(s, x, y, st);
  case 100: return launch_dot<MATS, NB, 2, 4, 1, OutT>(s, x, y, st);
  case 101: return launch_dot<MATS, NB, 2, 4, 2, OutT>(s, x, y, st);
  case 102: return launch_dot<MATS, NB, 2, 4, 4, OutT>(s, x, y, st);
  case 110: return launch_dot<MATS, NB, 2, 2, 1, OutT>(s, x, y, st);
  case 111: return launch_dot<MATS, NB, 2, 2, 2, OutT>(s, x, y, st);
  default: return launch_dot<MATS, NB, 2, 2, 4, OutT>(s, x, y, st);
  }
}

// Batches above 8 (or a remainder) are cut into chunks of 8/4/2/1 rows.
template <int MATS, typename OutT>
int run_dot(const Shape& s, const tmc_gemv_config& cfg, hipStream_t st) {
  OutT* y = static_cast<OutT*>(s.y);
  for (int r0 = 0; r0 < s.batch;) {
    const int left = s.batch - r0;
    const int nb = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
    const half_t* xs = s.x + (size_t)r0 * s.k;
    OutT* ys = y + (size_t)r0 * s.n;
    int rc;
    switch (nb) {
    case 8: rc = dot_by_config<MATS, 8, OutT>(s, xs, ys, cfg.rows_per_wave, cfg.unroll, cfg.k_split, st); break;
    case 4: rc = dot_by_config<MATS, 4, OutT>(s, xs, ys, cfg.rows_per_wave, cfg.unroll, cfg.k_split, st); break;
    case 2: rc = dot_by_config<MATS, 2, OutT>(s, xs, ys, cfg.rows_per_wave, cfg.unroll, cfg.k_split, st); break;
    default: rc = dot_by_config<MATS, 1, OutT>(s, xs, ys, cfg.rows_per_wave, cfg.unroll, cfg.k_split, st); break;
    }
    if (rc) return rc;
    r0 += nb;
  }
  return 0;
}

template <int MATS, int MT, int U, typename OutT>
int launch_mfma(const Shape& s, const half_t* x, OutT* y, int rows, int nt, int ks,
                hipStream_t st) {
  const int ntiles = (s.n + 15) / 16;
  const dim3 grid((ntiles + nt - 1) / nt);
  const size_t lds = (size_t)nt * ks * MATS * MT * 4 * kWave * sizeof(float);
  hipLaunchKernelGGL((mfma_gemm_kernel<MATS, MT, U, OutT>), grid, dim3(nt * ks * kWave), lds, st,
                     x, s.w0, s.w1, y, rows, s.n, s.k, nt, ks);
  return check_launch("mfma_gemm_kernel");
}

template <int MATS, typename OutT>
int run_mfma(const Shape& s, const tmc_gemv_config& cfg, hipStream_t st) {
  OutT* y = static_cast<OutT*>(s.y);
  for (int r0 = 0; r0 < s.batch; r0 += 64) {
    const int rows = min(64, s.batch - r0);
    const int mt = (rows + 15) / 16;
    // Keep the LDS reduction buffer within 64 KiB: shrink the k split (then
    // the n tiles per block) for the widest batch tiles.
    int ks = cfg.k_split, nt = cfg.rows_per_wave;  // n tiles per block for this algorithm
    const int mt_alloc = mt == 3 ? 4 : mt;
    while ((size_t)nt * ks * MATS * mt_alloc * 4 * kWave * sizeof(float) > 65536 && ks > 1) ks /= 2;
    while ((size_t)nt * ks * MATS * mt_alloc * 4 * kWave * sizeof(float) > 65536 && nt > 1) nt /= 2;
    const half_t* xs = s.x + (size_t)r0 * s.k;
    OutT* ys = y + (size_t)r0 * s.n;
    int rc;
    const bool u2 = cfg.unroll >= 2;
    switch (mt) {
    case 1: rc = u2 ? launch_mfma<MATS, 1, 2, OutT>(s, xs, ys, rows, nt, ks, st)
                    : launch_mfma<MATS, 1, 1, OutT>(s, xs, ys, rows, nt, ks, st); break;
    case 2: rc = u2 ? launch_mfma<MATS, 2, 2, OutT>(s, xs, ys, rows, nt, ks, st)
                    : launch_mfma<MATS, 2, 1, OutT>(s, xs, ys, rows, nt, ks, st); break;
    default: rc = launch_mfma<MATS, 4, 1, OutT>(s, xs, ys, rows, nt, ks, st); break;
    }
    if (rc) return rc;
  }
  return 0;
}

template <int MATS, int RT, int U, typename OutT>
int launch_rows(const Shape& s, const half_t* x, OutT* y, int rows, int ks, hipStream_t st) {
  const dim3 grid((unsigned)((s.n + RT * 16 - 1) / (RT * 16)));
  const size_t lds = (size_t)ks * MATS * RT * 4 * kWave * sizeof(float);
  hipLaunchKernelGGL((mfma_rows_kernel<MATS, RT, U, OutT>), grid, dim3(ks * kWave), lds, st, x,
                     s.w0, s.w1, y, rows, s.n, s.k, ks);
  return check_launch("mfma_rows_kernel");
}

template <int MATS, typename OutT>
int run_rows(const Shape& s, const tmc_gemv_config& cfg, hipStream_t st) {
  // The LDS reduction holds k_split x MATS x tiles 16x16 fp32 partials.
  TMC_REQUIRE((size_t)cfg.k_split * MATS * cfg.rows_per_wave * 4 * kWave * sizeof(float) <= 65536,
              "GEMV config: MFMA row tiles need k_split * tiles * matrices <= 64 (64 KiB LDS).");
  OutT* y = static_cast<OutT*>(s.y);
  for (int r0 = 0; r0 < s.batch; r0 += 16) {
    const int rows = min(16, s.batch - r0);
    const half_t* xs = s.x + (size_t)r0 * s.k;
    OutT* ys = y + (size_t)r0 * s.n;
    int rc;
    const int ks = cfg.k_split;
    switch (cfg.rows_per_wave * 8 + cfg.unroll) {
    case 9: rc = launch_rows<MATS, 1, 1, OutT>(s, xs, ys, rows, ks, st); break;
    case 10: rc = launch_rows<MATS, 1, 2, OutT>(s, xs, ys, rows, ks, st); break;
    case 12: rc = launch_rows<MATS, 1, 4, OutT>(s, xs, ys, rows, ks, st); break;
    case 17: rc = launch_rows<MATS, 2, 1, OutT>(s, xs, ys, rows, ks, st); break;
    case 18: rc = launch_rows<MATS, 2, 2, OutT>(s, xs, ys, rows, ks, st); break;
    case 20: rc = launch_rows<MATS, 2, 4, OutT>(s, xs, ys, rows, ks, st); break;
    case 33: rc = launch_rows<MATS, 4, 1, OutT>(s, xs, ys, rows, ks, st); break;
    default: rc = launch_rows<MATS, 4, 2, OutT>(s, xs, ys, rows, ks, st); break;
    }
    if (rc) return rc;
  }
  return 0;
}

// Default configuration per shape (the tuner may override it), from graph-
// timed sweeps on MI355X with weights larger than the Infinity Cache: batch 1
// streams rows with the dot algorithm and 4 waves per row (2 rows per wave
// for rows longer than 8K); larger batches use the MFMA row-tile kernel.
// Sweep winners (batch 8 / 16, K 4096 unless noted): N 12288 -> 1|2 tiles,
// unroll 1, 4 waves; N 4096 (K 4096 and K 11008) -> 1 tile, 8 waves; N 32000
// -> 2 tiles, unroll 1, 2 waves; gated N 11008 -> 1 tile, 4 waves, unroll 1
// at batch 8 and 4 at batch 16.
tmc_gemv_config default_config(int batch, int n, int k, int mats) {
  tmc_gemv_config c{};
  (void)k;
  if (batch == 1 && mats == 1 && k > 8192 && k <= 16384) {
    // the down projection (11008 -> 4096 with its residual): the persistent
    // dot, 14.9 us against 15.5 us for the dot at 2 rows per wave
    c.algorithm = 5;
    c.rows_per_wave = 1;
    c.unroll = 1;
    c.k_split = 4;
    return c;
  }
  if (batch == 1) {
    c.algorithm = 1;
    c.rows_per_wave = k > 8192 ? 2 : 1;
    c.unroll = mats == 2 ? 2 : 4;
    c.k_split = 4;
    if (mats == 1 && n <= 4096 && k <= 8192) {
      // 4096 x 4096 (the o projection, C1): 6.6 us against 7.2 us at 1 row
      // per wave and 4 waves per row
      c.rows_per_wave = 2;
      c.k_split = 2;
    }
    return c;
  }
  c.algorithm = 3;
  if (mats == 2) {
    c.rows_per_wave = 1;
    c.unroll = batch > 8 ? 4 : 1;
    c.k_split = 4;
  } else if (n >= 16384) {
    c.rows_per_wave = 2;
    c.unroll = 1;
    c.k_split = 2;
  } else if (n >= 8192) {
    c.rows_per_wave = batch > 8 ? 2 : 1;
    c.unroll = 1;
    c.k_split = 4;
  } else {
    c.rows_per_wave = 1;
    c.unroll = batch > 8 ? 1 : 2;
    c.k_split = 8;
  }
  return c;
}

int validate_config(const tmc_gemv_config& c) {
  if (c.algorithm == 1) {
    TMC_REQUIRE((c.rows_per_wave == 1 || c.rows_per_wave == 2) &&
                    (c.unroll == 2 || c.unroll == 4) &&
                    (c.k_split == 1 || c.k_split == 2 || c.k_split == 4),
                "GEMV config: dot algorithm needs rows_per_wave 1|2, unroll 2|4, k_split 1|2|4.");
  } else if (c.algorithm == 3) {
    TMC_REQUIRE((c.rows_per_wave == 1 || c.rows_per_wave == 2 || c.rows_per_wave == 4) &&
                    c.k_split >= 1 && c.k_split <= 16 &&
                    (c.unroll == 1 || c.unroll == 2 || (c.unroll == 4 && c.rows_per_wave <= 2)),
                "GEMV config: MFMA row tiles need rows_per_wave 1|2|4 tiles, k_split 1..16 "
                "waves and unroll 1|2 (or 4 with at most 2 tiles).");
  } else if (c.algorithm == 4) {
    return 0;
  } else if (c.algorithm == 5) {
    TMC_REQUIRE((c.rows_per_wave == 1 || c.rows_per_wave == 2) && c.k_split == 4,
                "GEMV config: the persistent dot (algorithm 5) needs rows_per_wave 1|2 rows per "
                "block and k_split 4.");
  } else if (c.algorithm == 2) {
    TMC_REQUIRE(c.rows_per_wave >= 1 && c.k_split >= 1 && c.rows_per_wave * c.k_split <= 16 &&
                    (c.unroll == 1 || c.unroll == 2),
                "GEMV config: MFMA needs n_tiles * k_split <= 16 waves and unroll 1|2.");
  } else {
    return fail("GEMV config: algorithm must be 0 (auto), 1 (dot), 2 (MFMA), 3 (MFMA row tiles), "
                "4 (linear baseline) or 5 (persistent dot, batch 1).");
  }
  return 0;
}

int run_linear(int mats, const void* x, const void* w0, const void* w1, void* y, int y_dtype,
               int64_t batch, int64_t k, int64_t n, const tmc_gemv_config* user, void* stream) {
  const char* what = mats == 2 ? "Gated MLP" : "GEMV";
  TMC_REQUIRE(x && w0 && y && (mats == 1 || w1), std::string(what) + ": null device pointer.");
  TMC_REQUIRE(y_dtype == TMC_F16 || y_dtype == TMC_F32,
              std::string(what) + ": output dtype must be fp16 or fp32.");
  TMC_REQUIRE(batch > 0 && k > 0 && n > 0, std::string(what) + ": dimensions must be positive.");
  TMC_REQUIRE(k < (1LL << 31) && n < (1LL << 31) && batch < (1LL << 31),
              std::string(what) + ": dimensions exceed 32-bit indexing.");
  Shape s{static_cast<const half_t*>(x), static_cast<const half_t*>(w0),
          static_cast<const half_t*>(w1), y, y_dtype, (int)batch, (int)n, (int)k};
  const hipStream_t st = as_stream(stream);
  const bool vec = (k % 8) == 0 && aligned16(x) && aligned16(w0) && (mats == 1 || aligned16(w1));
  if (user && user->algorithm == 4) {
    const long items = (long)batch * n;
    TMC_REQUIRE(items < (1LL << 31) * 128LL, std::string(what) + ": too many outputs.");
    const dim3 grid((unsigned)((items + 127) / 128));
    if (mats == 2)
      hipLaunchKernelGGL((gemv_linear_baseline_kernel<2, half_t>), grid, dim3(128), 0, st, s.x,
                         s.w0, s.w1, static_cast<half_t*>(y), s.batch, s.n, s.k);
    else if (y_dtype == TMC_F32)
      hipLaunchKernelGGL((gemv_linear_baseline_kernel<1, float>), grid, dim3(128), 0, st, s.x,
                         s.w0, s.w1, static_cast<float*>(y), s.batch, s.n, s.k);
    else
      hipLaunchKernelGGL((gemv_linear_baseline_kernel<1, half_t>), grid, dim3(128), 0, st, s.x,
                         s.w0, s.w1, static_cast<half_t*>(y), s.batch, s.n, s.k);
    return check_launch("gemv_linear_baseline_kernel");
  }
  if (!vec) {
    const long items = (long)batch * n;
    const dim3 grid((unsigned)((items + 3) / 4));
    if (mats == 2)
      hipLaunchKernelGGL((gemv_generic_kernel<2, half_t>), grid, dim3(256), 0, st, s.x, s.w0, s.w1,
                         static_cast<half_t*>(y), s.batch, s.n, s.k);
    else if (y_dtype == TMC_F32)
      hipLaunchKernelGGL((gemv_generic_kernel<1, float>), grid, dim3(256), 0, st, s.x, s.w0, s.w1,
                         static_cast<float*>(y), s.batch, s.n, s.k);
    else
      hipLaunchKernelGGL((gemv_generic_kernel<1, half_t>), grid, dim3(256), 0, st, s.x, s.w0,
                         s.w1, static_cast<half_t*>(y), s.batch, s.n, s.k);
    return check_launch("gemv_generic_kernel");
  }
  tmc_gemv_config cfg = default_config(s.batch, s.n, s.k, mats);
  if (user && user->algorithm != 0) cfg = *user;
  if (validate_config(cfg)) return 1;
  if (cfg.algorithm == 5) {
    TMC_REQUIRE(s.batch == 1 && s.k <= 16384 &&
                    (uint64_t)(s.n + 1) * (uint64_t)s.k * 2u < (uint64_t)kBufferAbsent,
                std::string(what) + ": the persistent dot (algorithm 5) needs batch 1, K <= 16384 "
                "and weights below 4 GiB.");
    NormArgs na;
    na.x = s.x;
    if (mats == 2) return launch_norm_gemv<2, half_t, kFuseNone>(s, static_cast<half_t*>(y),
                                                                  cfg.rows_per_wave, na, st);
    return y_dtype == TMC_F32
               ? launch_norm_gemv<1, float, kFuseNone>(s, static_cast<float*>(y),
                                                       cfg.rows_per_wave, na, st)
               : launch_norm_gemv<1, half_t, kFuseNone>(s, static_cast<half_t*>(y),
                                                        cfg.rows_per_wave, na, st);
  }
  if (cfg.algorithm == 1) {
    if (mats == 2) return run_dot<2, half_t>(s, cfg, st);
    return y_dtype == TMC_F32 ? run_dot<1, float>(s, cfg, st) : run_dot<1, half_t>(s, cfg, st);
  }
  if (cfg.algorithm == 3) {
    // raw buffers address at most 4 GiB - 16 bytes
    const uint64_t wb = (uint64_t)s.n * s.k * 2, xb = (uint64_t)min(s.batch, 16) * s.k * 2;
    if (wb < kNoData && xb < kNoData) {
      if (mats == 2) return run_rows<2, half_t>(s, cfg, st);
      return y_dtype == TMC_F32 ? run_rows<1, float>(s, cfg, st) : run_rows<1, half_t>(s, cfg, st);
    }
    cfg = tmc_gemv_config{2, 1, 2, 4};
  }
  if (mats == 2) return run_mfma<2, half_t>(s, cfg, st);
  return y_dtype == TMC_F32 ? run_mfma<1, float>(s, cfg, st) : run_mfma<1, half_t>(s, cfg, st);
}

}  // namespace
}  // namespace tmc

using namespace tmc;

extern "C" int tmc_gemv_f16(const void* x, const void* w, void* y, int y_dtype, int64_t batch,
                            int64_t in_features, int64_t out_features, void* stream) {
  return run_linear(1, x, w, nullptr, y, y_dtype, batch, in_features, out_features, nullptr,
                    stream);
}

extern "C" int tmc_gemv_f16_config(const void* x, const void* w, void* y, int y_dtype,
                                   int64_t batch, int64_t in_features, int64_t out_features,
                                   const tmc_gemv_config* config, void* stream) {
  return run_linear(1, x, w, nullptr, y, y_dtype, batch, in_features, out_features, config,
                    stream);
}

extern "C" int tmc_skinny_gemm_f16_mfma(const void* x, const void* w, void* y, int y_dtype,
                                        int64_t batch, int64_t in_features, int64_t out_features,
                                        void* stream) {
  TMC_REQUIRE(batch > 0 && in_features > 0 && out_features > 0,
              "MFMA GEMM: dimensions must be positive.");
  tmc_gemv_config cfg =
      default_config((int)std::max<int64_t>(batch, 2), (int)out_features, (int)in_features, 1);
  TMC_REQUIRE((in_features % 8) == 0 && aligned16(x) && aligned16(w),
              "MFMA GEMM: in_features must be a multiple of 8 and x, W 16-byte aligned.");
  return run_linear(1, x, w, nullptr, y, y_dtype, batch, in_features, out_features, &cfg, stream);
}

extern "C" int tmc_gate_up_silu_f16(const void* x, const void* w_gate, const void* w_up, void* out,
                                    int64_t batch, int64_t hidden, int64_t intermediate,
                                    void* stream) {
  return run_linear(2, x, w_gate, w_up, out, TMC_F16, batch, hidden, intermediate, nullptr,
                    stream);
}

extern "C" int tmc_gate_up_silu_f16_config(const void* x, const void* w_gate, const void* w_up,
                                           void* out, int64_t batch, int64_t hidden,
                                           int64_t intermediate, const tmc_gemv_config* config,
                                           void* stream) {
  return run_linear(2, x, w_gate, w_up, out, TMC_F16, batch, hidden, intermediate, config,
                    stream);
}

namespace {

// Configuration of the norm fusions: the dot algorithm at k split 4 (the
// wave <-> norm group mapping of gemv_norm_kernel), rows_per_wave 1 or 2
// rows per block; the unroll does not apply (a wave holds all its chunks).
// Default: 2 rows per block for one matrix (halves the row and gamma reads
// per weight byte), 1 for the gated pair (its 2 x 2 weight rows would cost
// occupancy).
int norm_config(const tmc_gemv_config* config, const std::string& what, int mats,
                int& rows_per_block) {
  rows_per_block = mats == 2 ? 1 : 2;
  if (!config || config->algorithm == 0) return 0;
  TMC_REQUIRE(config->algorithm == 1 && config->k_split == 4 &&
                  (config->rows_per_wave == 1 || config->rows_per_wave == 2),
              what + ": config must use the dot algorithm (1) with k_split 4 and rows_per_wave "
                     "1|2.");
  rows_per_block = config->rows_per_wave;
  return 0;
}

int fused_entry(int mats, const void* residual, const void* update, const void* gamma,
                const void* w0, const void* w1, void* sum_out, void* y, int y_dtype,
                int64_t batch, int64_t k, int64_t n, float eps, const tmc_gemv_config* config,
                void* stream) {
  const char* what = mats == 2 ? "Fused norm + gated MLP" : "Fused norm + GEMV";
  TMC_REQUIRE(residual && gamma && w0 && y && (mats == 1 || w1) && (!update || sum_out),
              std::string(what) + ": null device pointer.");
  TMC_REQUIRE(y_dtype == TMC_F16 || y_dtype == TMC_F32,
              std::string(what) + ": output dtype must be fp16 or fp32.");
  TMC_REQUIRE(batch == 1, std::string(what) + ": batch must be 1 (larger batches run the "
                                              "norm and the packed GEMM).");
  TMC_REQUIRE(k > 0 && n > 0 && k % 8 == 0 && k <= 8 * kNormMaxChunks && n < (1LL << 31),
              std::string(what) + ": in_features must be a positive multiple of 8 up to 8192.");
  TMC_REQUIRE((n + 1) * k * 2 < (int64_t)kBufferAbsent,
              std::string(what) + ": a weight matrix must stay below 4 GiB.");
  TMC_REQUIRE(aligned16(residual) && aligned16(gamma) && aligned16(w0) &&
                  (mats == 1 || aligned16(w1)) && (!update || (aligned16(update) && aligned16(sum_out))),
              std::string(what) + ": operands must be 16-byte aligned.");
  TMC_REQUIRE(std::isfinite(eps) && eps > 0.0f, std::string(what) + ": epsilon must be positive.");
  int rpb = 2;
  if (norm_config(config, what, mats, rpb)) return 1;
  NormArgs na;
  na.residual = static_cast<const half_t*>(residual);
  na.update = static_cast<const half_t*>(update);
  na.gamma = static_cast<const half_t*>(gamma);
  na.sum_out = static_cast<half_t*>(sum_out);
  na.eps = eps;
  Shape s{nullptr, static_cast<const half_t*>(w0), static_cast<const half_t*>(w1), y, y_dtype,
          1, (int)n, (int)k};
  const hipStream_t st = as_stream(stream);
  if (update) {
    if (mats == 2) return launch_norm_gemv<2, half_t, kFuseAddNorm>(s, static_cast<half_t*>(y), rpb, na, st);
    return y_dtype == TMC_F32
               ? launch_norm_gemv<1, float, kFuseAddNorm>(s, static_cast<float*>(y), rpb, na, st)
               : launch_norm_gemv<1, half_t, kFuseAddNorm>(s, static_cast<half_t*>(y), rpb, na, st);
  }
  if (mats == 2) return launch_norm_gemv<2, half_t, kFuseNorm>(s, static_cast<half_t*>(y), rpb, na, st);
  return y_dtype == TMC_F32
             ? launch_norm_gemv<1, float, kFuseNorm>(s, static_cast<float*>(y), rpb, na, st)
             : launch_norm_gemv<1, half_t, kFuseNorm>(s, static_cast<half_t*>(y), rpb, na, st);
}

}  // namespace

extern "C" int tmc_add_rmsnorm_gemv_f16(const void* residual, const void* update,
                                        const void* gamma, const void* w, void* sum_out, void* y,
                                        int y_dtype, int64_t batch, int64_t in_features,
                                        int64_t out_features, float epsilon,
                                        const tmc_gemv_config* config, void* stream) {
  return fused_entry(1, residual, update, gamma, w, nullptr, sum_out, y, y_dtype, batch,
                     in_features, out_features, epsilon, config, stream);
}

extern "C" int tmc_rmsnorm_lm_head_partial_argmax_f16(const void* residual, const void* gamma,
                                                     const void* w, void* workspace,
                                                     size_t workspace_bytes, int64_t in_features,
                                                     int64_t vocabulary, float epsilon,
                                                     const tmc_gemv_config* config, void* stream) {
  const std::string what = "LM head partial argmax";
  TMC_REQUIRE(residual && gamma && w && workspace, what + ": null device pointer.");
  TMC_REQUIRE(in_features > 0 && vocabulary > 0 && in_features % 8 == 0 &&
                  in_features <= 8 * kNormMaxChunks && vocabulary < (1LL << 28),
              what + ": in_features must be a positive multiple of 8 up to 8192.");
  TMC_REQUIRE((vocabulary + 1) * in_features * 2 < (int64_t)kBufferAbsent,
              what + ": the weight matrix must stay below 4 GiB.");
  TMC_REQUIRE(workspace_bytes >= tmc_lm_head_argmax_workspace_bytes(1, vocabulary),
              what + ": workspace is smaller than tmc_lm_head_argmax_workspace_bytes().");
  TMC_REQUIRE(aligned16(residual) && aligned16(gamma) && aligned16(w) && aligned16(workspace),
              what + ": operands must be 16-byte aligned.");
  TMC_REQUIRE(std::isfinite(epsilon) && epsilon > 0.0f, what + ": epsilon must be positive.");
  int rpb = 2;
  if (norm_config(config, what, 1, rpb)) return 1;
  NormArgs na;
  na.residual = static_cast<const half_t*>(residual);
  na.gamma = static_cast<const half_t*>(gamma);
  na.eps = epsilon;
  Shape s{nullptr, static_cast<const half_t*>(w), nullptr, workspace, TMC_F32, 1, (int)vocabulary,
          (int)in_features};
  float* out = static_cast<float*>(workspace);
  return rpb == 2
             ? launch_norm_gemv_rpw<1, 2, float, kFuseNorm, false, true>(s, out, na, RopeArgs{},
                                                                        as_stream(stream))
             : launch_norm_gemv_rpw<1, 1, float, kFuseNorm, false, true>(s, out, na, RopeArgs{},
                                                                        as_stream(stream));
}

extern "C" int tmc_add_rmsnorm_gate_up_silu_f16(const void* residual, const void* update,
                                                const void* gamma, const void* w_gate,
                                                const void* w_up, void* sum_out, void* out,
                                                int64_t batch, int64_t hidden,
                                                int64_t intermediate, float epsilon,
                                                const tmc_gemv_config* config, void* stream) {
  return fused_entry(2, residual, update, gamma, w_gate, w_up, sum_out, out, TMC_F16, batch,
                     hidden, intermediate, epsilon, config, stream);
}

extern "C" int tmc_gemv_residual_f16(const void* x, const void* w, const void* residual, void* y,
                                     int64_t batch, int64_t in_features, int64_t out_features,
                                     const tmc_gemv_config* config, void* stream) {
  TMC_REQUIRE(x && w && residual && y, "GEMV + residual: null device pointer.");
  TMC_REQUIRE(batch == 1, "GEMV + residual: batch must be 1.");
  TMC_REQUIRE(in_features > 0 && out_features > 0 && in_features % 8 == 0 &&
                  in_features < (1LL << 31) && out_features < (1LL << 31),
              "GEMV + residual: in_features must be a positive multiple of 8.");
  TMC_REQUIRE(aligned16(x) && aligned16(w), "GEMV + residual: x and W must be 16-byte aligned.");
  tmc_gemv_config cfg = default_config(1, (int)out_features, (int)in_features, 1);
  if (config && config->algorithm != 0) cfg = *config;
  TMC_REQUIRE(cfg.algorithm == 1 || cfg.algorithm == 5,
              "GEMV + residual: config must use the dot algorithm (1) or the persistent dot (5).");
  if (validate_config(cfg)) return 1;
  NormArgs na;
  na.residual = static_cast<const half_t*>(residual);
  Shape s{static_cast<const half_t*>(x), static_cast<const half_t*>(w), nullptr, y, TMC_F16, 1,
          (int)out_features, (int)in_features};
  if (cfg.algorithm == 5) {
    TMC_REQUIRE(in_features <= 16384 &&
                    (out_features + 1) * in_features * 2 < (int64_t)kBufferAbsent,
                "GEMV + residual: the persistent dot needs K <= 16384 and W below 4 GiB.");
    na.x = static_cast<const half_t*>(x);
    return launch_norm_gemv<1, half_t, kFuseResidual>(s, static_cast<half_t*>(y),
                                                      cfg.rows_per_wave, na, as_stream(stream));
  }
  return launch_dot_fused<1, half_t, kFuseResidual>(s, static_cast<half_t*>(y), cfg, na,
                                                    as_stream(stream));
}

namespace {

int launch_qkv_rope(const Shape& s, const tmc_gemv_config& c, hipStream_t st, const RopeArgs& ra) {
  half_t* none = nullptr;
  const NormArgs na{};
  switch ((c.unroll == 2 ? 10 : 0) + (c.k_split == 4 ? 2 : c.k_split == 2 ? 1 : 0)) {
  case 0: return launch_dot<1, 1, 2, 4, 1, half_t, kFuseNone, true>(s, s.x, none, st, na, ra);
  case 1: return launch_dot<1, 1, 2, 4, 2, half_t, kFuseNone, true>(s, s.x, none, st, na, ra);
  case 2: return launch_dot<1, 1, 2, 4, 4, half_t, kFuseNone, true>(s, s.x, none, st, na, ra);
  case 10: return launch_dot<1, 1, 2, 2, 1, half_t, kFuseNone, true>(s, s.x, none, st, na, ra);
  case 11: return launch_dot<1, 1, 2, 2, 2, half_t, kFuseNone, true>(s, s.x, none, st, na, ra);
  default: return launch_dot<1, 1, 2, 2, 4, half_t, kFuseNone, true>(s, s.x, none, st, na, ra);
  }
}

// q.k.v projection + RoPE + paged append at batch 1; fuse: kFuseNone (x is
// the projection input), kFuseAddNorm (x = RMSNorm(residual + update)) or
// kFuseNorm (RMSNorm(residual)).
int qkv_rope_entry(int fuse, const void* x, const NormArgs& na, const void* w,
                   const float* cosine, const float* sine, const int32_t* valid_lengths,
                   const int32_t* block_table, const int32_t* active_count, void* q_out,
                   void* key_pool, void* value_pool, int64_t hidden, int64_t q_heads,
                   int64_t kv_heads, int64_t head_dim, int64_t capacity, int64_t page_size,
                   const tmc_gemv_config* config, void* stream) {
  TMC_REQUIRE((fuse != kFuseNone || x) && w && cosine && sine && valid_lengths && block_table &&
                  active_count && q_out && key_pool && value_pool,
              "Fused q.k.v RoPE append: null pointer.");
  TMC_REQUIRE(hidden > 0 && hidden % 8 == 0 &&
                  (fuse != kFuseNone ? hidden <= 8 * kNormMaxChunks : hidden < (1LL << 31)) &&
                  (fuse != kFuseNone || aligned16(x)) && aligned16(w),
              "Fused q.k.v RoPE append: hidden must be a positive multiple of 8 (at most 8192 "
              "with the norm) and x, W 16-byte aligned.");
  TMC_REQUIRE(q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0 && head_dim > 0 &&
                  head_dim % 2 == 0 && capacity > 0 && page_size > 0 &&
                  (q_heads + 2 * kv_heads) * head_dim < (1LL << 31),
              "Fused q.k.v RoPE append: invalid head geometry, capacity or page size.");
  // measured default (C5 q.k.v shape): unroll 4, k split 4 (the norm form:
  // k split 4 always, the unroll does not apply)
  tmc_gemv_config c{1, 2, 4, 4};
  if (config && config->algorithm != 0) c = *config;
  TMC_REQUIRE(fuse == kFuseNone || c.k_split == 4,
              "Fused norm + q.k.v RoPE append: the norm form needs k_split 4.");
  TMC_REQUIRE(fuse == kFuseNone ||
                  ((q_heads + 2 * kv_heads) * head_dim + 1) * hidden * 2 < (int64_t)kBufferAbsent,
              "Fused norm + q.k.v RoPE append: the weight must stay below 4 GiB.");
  TMC_REQUIRE(c.algorithm == 1 && c.rows_per_wave == 2 && (c.unroll == 2 || c.unroll == 4) &&
                  (c.k_split == 1 || c.k_split == 2 || c.k_split == 4),
              "Fused q.k.v RoPE append: the dot algorithm with rows_per_wave 2, unroll 2|4 and "
              "k_split 1|2|4.");
  const int64_t n = (q_heads + 2 * kv_heads) * head_dim;
  Shape s{static_cast<const half_t*>(x), static_cast<const half_t*>(w), nullptr, nullptr, TMC_F16,
          1, (int)n, (int)hidden};
  RopeArgs ra;
  ra.cosine = cosine;
  ra.sine = sine;
  ra.valid_lengths = valid_lengths;
  ra.block_tables = block_table;
  ra.active_count = active_count;
  ra.q_out = static_cast<half_t*>(q_out);
  ra.k_pool = static_cast<half_t*>(key_pool);
  ra.v_pool = static_cast<half_t*>(value_pool);
  ra.q_heads = (int)q_heads;
  ra.kv_heads = (int)kv_heads;
  ra.head_dim = (int)head_dim;
  ra.capacity = (int)capacity;
  ra.page_size = (int)page_size;
  const hipStream_t st = as_stream(stream);
  if (fuse == kFuseAddNorm)
    return launch_norm_gemv_rpw<1, 2, half_t, kFuseAddNorm, true>(s, nullptr, na, ra, st);
  if (fuse == kFuseNorm)
    return launch_norm_gemv_rpw<1, 2, half_t, kFuseNorm, true>(s, nullptr, na, ra, st);
  return launch_qkv_rope(s, c, st, ra);
}

}  // namespace

extern "C" int tmc_qkv_rope_append_f16(const void* x, const void* w, const float* cosine,
                                       const float* sine, const int32_t* valid_lengths,
                                       const int32_t* block_table, const int32_t* active_count,
                                       void* q_out, void* key_pool, void* value_pool,
                                       int64_t hidden, int64_t q_heads, int64_t kv_heads,
                                       int64_t head_dim, int64_t capacity, int64_t page_size,
                                       const tmc_gemv_config* config, void* stream) {
  return qkv_rope_entry(kFuseNone, x, NormArgs{}, w, cosine, sine, valid_lengths, block_table,
                        active_count, q_out, key_pool, value_pool, hidden, q_heads, kv_heads,
                        head_dim, capacity, page_size, config, stream);
}

extern "C" int tmc_add_rmsnorm_qkv_rope_append_f16(
    const void* residual, const void* update, const void* gamma, const void* w, void* sum_out,
    const float* cosine, const float* sine, const int32_t* valid_lengths,
    const int32_t* block_table, const int32_t* active_count, void* q_out, void* key_pool,
    void* value_pool, int64_t hidden, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
    int64_t capacity, int64_t page_size, float epsilon, const tmc_gemv_config* config,
    void* stream) {
  TMC_REQUIRE(residual && gamma && (!update || sum_out),
              "Fused norm + q.k.v RoPE append: null pointer.");
  TMC_REQUIRE(aligned16(residual) && aligned16(gamma) &&
                  (!update || (aligned16(update) && aligned16(sum_out))),
              "Fused norm + q.k.v RoPE append: operands must be 16-byte aligned.");
  TMC_REQUIRE(std::isfinite(epsilon) && epsilon > 0.0f,
              "Fused norm + q.k.v RoPE append: epsilon must be positive.");
  NormArgs na;
  na.residual = static_cast<const half_t*>(residual);
  na.update = static_cast<const half_t*>(update);
  na.gamma = static_cast<const half_t*>(gamma);
  na.sum_out = static_cast<half_t*>(sum_out);
  na.eps = epsilon;
  return qkv_rope_entry(update ? kFuseAddNorm : kFuseNorm, nullptr, na, w, cosine, sine, valid_lengths, block_table,
                        active_count, q_out, key_pool, value_pool, hidden, q_heads, kv_heads,
                        head_dim, capacity, page_size, config, stream);
}

extern "C" int tmc_gemv_default_config(int64_t batch, int64_t in_features, int64_t out_features,
                                       int gated, tmc_gemv_config* out) {
  TMC_REQUIRE(out && batch > 0 && in_features > 0 && out_features > 0,
              "tmc_gemv_default_config: invalid arguments.");
  *out = default_config((int)batch, (int)out_features, (int)in_features, gated ? 2 : 1);
  return 0;
}
