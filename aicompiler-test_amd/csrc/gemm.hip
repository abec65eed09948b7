// Prompt GEMMs for gfx950: y[m, n] = x[m, k] w[n, k]^T with fp16 operands and
// fp32 accumulation, the linear layers of a chunked-prefill stage
// (emitTiledGEMM, DecodeGEMVMetalEmitter.cpp:134-169; prefillChunked,
// DecoderLLMExecutor.cpp:982-1034).
#include "tmc_abi.hpp"
#include "tmc_device.hpp"

#include <algorithm>

namespace tmc {
namespace {

// ------------------------------------------------------------ prompt GEMM
// y[m, n] = x[m, k] w[n, k]^T with fp16 operands and fp32 accumulation on
// v_mfma_f32_16x16x32_f16.  Both operands are k-contiguous rows, which is the
// MFMA operand order: lane (i, g) of a 16 x 32 fragment holds row i, k
// 8g ... 8g + 7, for x (A) and for w (B) alike.
//
// Block: 256 threads = 2 x 2 waves over a 128 x 128 output tile, each wave
// 64 x 64 (4 x 4 MFMA tiles, 64 accumulators per lane).  K advances in stages
// of 64: while the waves multiply the current stage out of LDS, every thread
// holds its share of the next two stages' x and w tiles (16 KiB each) in
// registers, and stores the next one to the other LDS buffer after the
// multiply; one barrier per stage.  An LDS row is the stage's 64 halves of
// one tile row as eight 16-byte chunks, chunk c stored at slot
// c ^ ((row / 2) % 8): the 16 rows an operand read touches, and the 16 lanes
// of a store, then fall on 16 distinct 4-bank groups.  Raw buffer loads read
// zero past m, n or k, so ragged tiles need no branches.
//
// Tiles are dealt XCD by XCD: blocks b, b + 8, b + 16, ... run on one XCD
// and take consecutive tiles, which walk the m tiles of one n tile first, so
// a weight slice is fetched from HBM once into that XCD's L2.
constexpr int kGemmTile = 128;
#ifndef TMC_GEMM_K
#define TMC_GEMM_K 64
#endif
#ifndef TMC_GEMM_WPE
#define TMC_GEMM_WPE 2
#endif
constexpr int kGemmK = TMC_GEMM_K;
constexpr int kGemmRow = kGemmK;  // halves per LDS row (swizzled chunks, no padding)
constexpr int kGemmThreads = 256;

// Split K (SPLIT): block (tile, split s) multiplies k in [s * k_chunk,
// (s + 1) * k_chunk) and writes fp32 partials y[s][m][n]; gemm_reduce_kernel
// adds them in split order.
template <typename OutT, bool SPLIT>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(TMC_GEMM_WPE, TMC_GEMM_WPE))) void gemm_nt_kernel(
    const half_t* __restrict__ x, const half_t* __restrict__ w, OutT* __restrict__ y, int m,
    int n, int k, int m_tiles, int tiles, int k_chunk, unsigned x_bytes, unsigned w_bytes) {
  __shared__ __attribute__((aligned(16))) half_t lds[2][2][kGemmTile * kGemmRow];
  const int per_xcd = (int)(gridDim.x / 8u);
  const int unit = (int)(blockIdx.x % 8u) * per_xcd + (int)(blockIdx.x / 8u);
  const int splits = SPLIT ? (k + k_chunk - 1) / k_chunk : 1;
  if (unit >= tiles * splits) return;
  const int t = unit % tiles;
  const int k_begin = SPLIT ? (unit / tiles) * k_chunk : 0;
  const int k_end = SPLIT ? min(k, k_begin + k_chunk) : k;
  const int m0 = (t % m_tiles) * kGemmTile;
  const int n0 = (t / m_tiles) * kGemmTile;
  const int tid = (int)threadIdx.x;
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  const int i = lane & 15, g = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  const __amdgpu_buffer_rsrc_t rx = buffer_resource(x, x_bytes);
  const __amdgpu_buffer_rsrc_t rw = buffer_resource(w, w_bytes);

  // Stage loads: each thread moves kPasses 16-byte chunks of both tiles.  Two stages are in flight in registers: the
  // loads of stage st + 2 are issued before stage st is multiplied, and
  // stage st + 1 (loaded one multiply earlier) is stored to LDS after it.
  // A row holds kChunks 16-byte chunks; 256 threads move kPass rows per
  // pass and kPasses passes cover the tile's 128 rows.  A 256-byte LDS bank
  // sweep holds kSweepRows rows; chunk c of row r sits at slot
  // c ^ ((r / kSweepRows) % kChunks).
  constexpr int kChunks = kGemmK / 8, kPass = kGemmThreads / kChunks;
  constexpr int kPasses = kGemmTile / kPass, kSweepRows = 256 / (2 * kGemmK);
  const int lr = tid / kChunks, lc = tid % kChunks;
  struct Stage {
    h8 x[kPasses], w[kPasses];
  };
  auto load_stage = [&](Stage& sg, int k0) {
    const int kk = k_begin + k0 + 8 * lc;
    const bool k_ok = kk < k_end;
#pragma unroll
    for (int q = 0; q < kPasses; ++q) {
      const int r = lr + kPass * q;
      const bool xo = k_ok && m0 + r < m, wo = k_ok && n0 + r < n;
      sg.x[q] = buffer_load_h8(rx, xo ? (unsigned)(((size_t)(m0 + r) * k + kk) * 2) : kBufferAbsent);
      sg.w[q] = buffer_load_h8(rw, wo ? (unsigned)(((size_t)(n0 + r) * k + kk) * 2) : kBufferAbsent);
    }
  };
  auto store_stage = [&](const Stage& sg, int buf) {
#pragma unroll
    for (int q = 0; q < kPasses; ++q) {
      const int r = lr + kPass * q;
      const int slot = lc ^ ((r / kSweepRows) % kChunks);
      *reinterpret_cast<h8*>(&lds[buf][0][r * kGemmRow + 8 * slot]) = sg.x[q];
      *reinterpret_cast<h8*>(&lds[buf][1][r * kGemmRow + 8 * slot]) = sg.w[q];
    }
  };

  f4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  auto multiply = [&](int buf) {
    // rows wm*64 + 16a + i (x) and wn*64 + 16b + i (w); chunk 4s + g of a
    // row sits at slot (4s + g) ^ ((i / kSweepRows) % kChunks) (the row bases
    // are multiples of 16)
    const half_t* ax = lds[buf][0] + (wm * 64 + i) * kGemmRow;
    const half_t* bw = lds[buf][1] + (wn * 64 + i) * kGemmRow;
    const int sw = (i / kSweepRows) % kChunks;
#pragma unroll
    for (int s = 0; s < kGemmK / 32; ++s) {
      const int slot = 8 * ((4 * s + g) ^ sw);
      h8 fa[4], fb[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) fa[a] = *reinterpret_cast<const h8*>(ax + a * 16 * kGemmRow + slot);
#pragma unroll
      for (int b = 0; b < 4; ++b) fb[b] = *reinterpret_cast<const h8*>(bw + b * 16 * kGemmRow + slot);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[a], fb[b], acc[a][b], 0, 0, 0);
    }
  };

  const int stages = (k_end - k_begin + kGemmK - 1) / kGemmK;
  Stage even, odd;  // registers of the stages with even / odd index
  load_stage(even, 0);
  load_stage(odd, kGemmK);
  store_stage(even, 0);
  __syncthreads();
  // Stage st sits in LDS buffer st & 1.  At an even st, `odd` holds stage
  // st + 1 and `even` is free for stage st + 2; at an odd st the other way
  // round (the loop is unrolled by two so the registers are named).  Stages
  // past the end load with out-of-range offsets (zeros, no memory traffic)
  // and an odd stage count multiplies one stage of zeros: no step is
  // conditional, since at a branch join the compiler counts outstanding
  // loads conservatively and storing stage st + 1 would wait for the loads
  // of stage st + 2 as well.
  auto step = [&](int st, Stage& free_regs, const Stage& next_regs) {
    load_stage(free_regs, (st + 2) * kGemmK);
    __builtin_amdgcn_sched_barrier(0);  // the loads go out first
    multiply(st & 1);
    store_stage(next_regs, (st + 1) & 1);
    __syncthreads();
  };
  for (int st = 0; st < stages; st += 2) {
    step(st, even, odd);
    step(st + 1, odd, even);
  }

  // acc[a][b][r] = y[m0 + wm*64 + 16a + 4g + r][n0 + wn*64 + 16b + i]
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + wm * 64 + 16 * a + 4 * g + r;
      if (row >= m) continue;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int col = n0 + wn * 64 + 16 * b + i;
        if (col >= n) continue;
        if constexpr (SPLIT)
          reinterpret_cast<float*>(y)[((size_t)(unit / tiles) * m + row) * n + col] = acc[a][b][r];
        else
          y[(size_t)row * n + col] = from_float<OutT>(acc[a][b][r]);
      }
    }
}

// Big tiles for long prompts: 512 threads = 2 x 4 waves over a 256 x 256
// output tile, each wave 128 x 64 (8 x 4 MFMA tiles, 128 fp32 accumulators
// per lane, which the compiler keeps in AGPRs).  Per flop this moves half the
// LDS bytes of the 128 x 128 kernel (each A fragment feeds 4 MFMAs and each
// B fragment 8, and the staged tile feeds 256 outputs per row), and the
// 128 x 128 kernel waits on LDS issue (SQ_WAIT_INST_LDS 17% of wave cycles at
// 35% MFMA busy).  Same stage pipeline, LDS row format and swizzle, tile
// dealing and split-K as gemm_nt_kernel; LDS holds 2 x (256 + 256) rows of
// 64 halves (128 KiB), one block per CU, two waves per SIMD.
#ifndef TMC_GEMM_BIG_K
#define TMC_GEMM_BIG_K 64
#endif
constexpr int kBigTile = 256;
constexpr int kBigK = TMC_GEMM_BIG_K;  // k per stage (32: no spills, but 37% LDS bank conflicts)
constexpr int kBigThreads = 512;

template <typename OutT, bool SPLIT>
__global__ __launch_bounds__(kBigThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_big_kernel(
    const half_t* __restrict__ x, const half_t* __restrict__ w, OutT* __restrict__ y, int m,
    int n, int k, int m_tiles, int tiles, int k_chunk, unsigned x_bytes, unsigned w_bytes) {
  __shared__ __attribute__((aligned(16))) half_t lds[2][2][kBigTile * kBigK];
  const int per_xcd = (int)(gridDim.x / 8u);
  const int unit = (int)(blockIdx.x % 8u) * per_xcd + (int)(blockIdx.x / 8u);
  const int splits = SPLIT ? (k + k_chunk - 1) / k_chunk : 1;
  if (unit >= tiles * splits) return;
  const int t = unit % tiles;
  const int k_begin = SPLIT ? (unit / tiles) * k_chunk : 0;
  const int k_end = SPLIT ? min(k, k_begin + k_chunk) : k;
  const int m0 = (t % m_tiles) * kBigTile;
  const int n0 = (t / m_tiles) * kBigTile;
  const int tid = (int)threadIdx.x;
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  const int i = lane & 15, g = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;  // rows 128 wm.., columns 64 wn..
  const __amdgpu_buffer_rsrc_t rx = buffer_resource(x, x_bytes);
  const __amdgpu_buffer_rsrc_t rw = buffer_resource(w, w_bytes);

  // 512 threads move kPass rows of kChunks chunks per pass
  constexpr int kChunks = kBigK / 8, kPass = kBigThreads / kChunks;
  constexpr int kPasses = kBigTile / kPass, kSweepRows = 256 / (2 * kBigK);
  const int lr = tid / kChunks, lc = tid % kChunks;
  struct Stage {
    h8 x[kPasses], w[kPasses];
  };
  auto load_stage = [&](Stage& sg, int k0) {
    const int kk = k_begin + k0 + 8 * lc;
    const bool k_ok = kk < k_end;
#pragma unroll
    for (int q = 0; q < kPasses; ++q) {
      const int r = lr + kPass * q;
      const bool xo = k_ok && m0 + r < m, wo = k_ok && n0 + r < n;
      sg.x[q] = buffer_load_h8(rx, xo ? (unsigned)(((size_t)(m0 + r) * k + kk) * 2) : kBufferAbsent);
      sg.w[q] = buffer_load_h8(rw, wo ? (unsigned)(((size_t)(n0 + r) * k + kk) * 2) : kBufferAbsent);
    }
  };
  auto store_stage = [&](const Stage& sg, int buf) {
#pragma unroll
    for (int q = 0; q < kPasses; ++q) {
      const int r = lr + kPass * q;
      const int slot = lc ^ ((r / kSweepRows) % kChunks);
      *reinterpret_cast<h8*>(&lds[buf][0][r * kBigK + 8 * slot]) = sg.x[q];
      *reinterpret_cast<h8*>(&lds[buf][1][r * kBigK + 8 * slot]) = sg.w[q];
    }
  };

  f4 acc[8][4];
#pragma unroll
  for (int a = 0; a < 8; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  auto multiply = [&](int buf) {
    const half_t* ax = lds[buf][0] + (wm * 128 + i) * kBigK;
    const half_t* bw = lds[buf][1] + (wn * 64 + i) * kBigK;
    const int sw = (i / kSweepRows) % kChunks;
#pragma unroll
    for (int s = 0; s < kBigK / 32; ++s) {
      const int slot = 8 * ((4 * s + g) ^ sw);
      h8 fa[8], fb[4];
#pragma unroll
      for (int a = 0; a < 8; ++a) fa[a] = *reinterpret_cast<const h8*>(ax + a * 16 * kBigK + slot);
#pragma unroll
      for (int b = 0; b < 4; ++b) fb[b] = *reinterpret_cast<const h8*>(bw + b * 16 * kBigK + slot);
#pragma unroll
      for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[a], fb[b], acc[a][b], 0, 0, 0);
    }
  };

  const int stages = (k_end - k_begin + kBigK - 1) / kBigK;
  Stage even, odd;
  load_stage(even, 0);
  load_stage(odd, kBigK);
  store_stage(even, 0);
  __syncthreads();
  auto step = [&](int st, Stage& free_regs, const Stage& next_regs) {
    load_stage(free_regs, (st + 2) * kBigK);
    __builtin_amdgcn_sched_barrier(0);  // the loads go out first
    multiply(st & 1);
    store_stage(next_regs, (st + 1) & 1);
    __syncthreads();
  };
  for (int st = 0; st < stages; st += 2) {
    step(st, even, odd);
    step(st + 1, odd, even);
  }

  // acc[a][b][r] = y[m0 + wm*128 + 16a + 4g + r][n0 + wn*64 + 16b + i]
#pragma unroll
  for (int a = 0; a < 8; ++a)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + wm * 128 + 16 * a + 4 * g + r;
      if (row >= m) continue;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int col = n0 + wn * 64 + 16 * b + i;
        if (col >= n) continue;
        if constexpr (SPLIT)
          reinterpret_cast<float*>(y)[((size_t)(unit / tiles) * m + row) * n + col] = acc[a][b][r];
        else
          y[(size_t)row * n + col] = from_float<OutT>(acc[a][b][r]);
      }
    }
}

template <typename OutT>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const float* __restrict__ partial,
                                                         OutT* __restrict__ y, size_t count,
                                                         int splits) {
  for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < count; e += (size_t)gridDim.x * 256) {
    float sum = partial[e];
    for (int s = 1; s < splits; ++s) sum += partial[(size_t)s * count + e];
    y[e] = from_float<OutT>(sum);
  }
}

// Splits of K for a launch of `tiles` output tiles: enough (tile, split)
// units for two workgroups per CU on 256 CUs, each split at least 512 deep,
// and the fp32 partials within `workspace_bytes`.  1 = no split.
int gemm_splits(int64_t tiles, int64_t m, int64_t k, int64_t n, size_t workspace_bytes) {
  int splits = 1;
  while (tiles * splits < 512 && k / (2 * splits) >= 512 &&
         (uint64_t)(splits * 2) * m * n * 4 <= workspace_bytes)
    splits *= 2;
  return splits;
}

// Build parameter: the fewest 256 x 256 tiles (after split-K) for which the
// big-tile kernel runs.
#ifndef TMC_GEMM_BIG_MIN_UNITS
#define TMC_GEMM_BIG_MIN_UNITS 192
#endif

template <typename OutT, bool SPLIT>
int launch_big(const half_t* x, const half_t* w, OutT* y, int64_t m, int64_t k, int64_t n,
               int m_tiles, int tiles, int k_chunk, unsigned blocks, uint64_t xb, uint64_t wb,
               hipStream_t stream) {
  hipLaunchKernelGGL((gemm_big_kernel<OutT, SPLIT>), dim3(blocks), dim3(kBigThreads), 0, stream, x,
                     w, y, (int)m, (int)n, (int)k, m_tiles, tiles, k_chunk, (unsigned)xb,
                     (unsigned)wb);
  return check_launch("gemm_big_kernel");
}

// The 256 x 256 kernel when it fills the GPU: one block per CU, so at least
// TMC_GEMM_BIG_MIN_UNITS (tile, split) units, splitting K (at least 512 deep
// per split) while the tiles alone give fewer than 256.  -1: not taken.
int launch_gemm_big(const half_t* x, const half_t* w, void* y, int out_dtype, int64_t m, int64_t k,
                    int64_t n, void* workspace, size_t workspace_bytes, uint64_t xb, uint64_t wb,
                    hipStream_t stream) {
  const int m_tiles = (int)((m + kBigTile - 1) / kBigTile);
  const int64_t tiles = (int64_t)m_tiles * ((n + kBigTile - 1) / kBigTile);
  int splits = 1;
  if (workspace)
    while (tiles * splits < 256 && k / (2 * splits) >= 512 &&
           (uint64_t)(splits * 2) * m * n * 4 <= workspace_bytes)
      splits *= 2;
  if (tiles * splits < TMC_GEMM_BIG_MIN_UNITS || tiles >= (1LL << 26)) return -1;
  const int k_chunk = (int)(((k + splits - 1) / splits + kBigK - 1) / kBigK * kBigK);
  const int units = (int)(tiles * ((k + k_chunk - 1) / k_chunk));
  const unsigned blocks = (unsigned)((units + 7) / 8 * 8);
  if (units > (int)tiles) {
    float* partial = static_cast<float*>(workspace);
    if (launch_big<float, true>(x, w, partial, m, k, n, m_tiles, (int)tiles, k_chunk, blocks, xb,
                                wb, stream))
      return 1;
    const size_t count = (size_t)m * n;
    const unsigned rb = (unsigned)std::min<size_t>((count + 255) / 256, 8192);
    const int used = (int)((k + k_chunk - 1) / k_chunk);
    if (out_dtype == TMC_F32)
      hipLaunchKernelGGL((gemm_reduce_kernel<float>), dim3(rb), dim3(256), 0, stream, partial,
                         static_cast<float*>(y), count, used);
    else
      hipLaunchKernelGGL((gemm_reduce_kernel<half_t>), dim3(rb), dim3(256), 0, stream, partial,
                         static_cast<half_t*>(y), count, used);
    return check_launch("gemm_reduce_kernel");
  }
  if (out_dtype == TMC_F32)
    return launch_big<float, false>(x, w, static_cast<float*>(y), m, k, n, m_tiles, (int)tiles,
                                    (int)k, blocks, xb, wb, stream);
  return launch_big<half_t, false>(x, w, static_cast<half_t*>(y), m, k, n, m_tiles, (int)tiles,
                                   (int)k, blocks, xb, wb, stream);
}

int launch_gemm_nt(const half_t* x, const half_t* w, void* y, int out_dtype, int64_t m, int64_t k,
                   int64_t n, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const uint64_t xb = (uint64_t)m * k * 2, wb = (uint64_t)n * k * 2;
  TMC_REQUIRE(xb < kBufferAbsent && wb < kBufferAbsent,
              "Prompt GEMM: each operand must stay below 4 GiB.");
  TMC_REQUIRE(k % 8 == 0, "Prompt GEMM: k must be a multiple of 8.");
  TMC_REQUIRE(aligned16(x) && aligned16(w), "Prompt GEMM: x and w must be 16-byte aligned.");
  const int big = launch_gemm_big(x, w, y, out_dtype, m, k, n, workspace, workspace_bytes, xb, wb,
                                  stream);
  if (big >= 0) return big;
  const int m_tiles = (int)((m + kGemmTile - 1) / kGemmTile);
  const int64_t tiles = (int64_t)m_tiles * ((n + kGemmTile - 1) / kGemmTile);
  TMC_REQUIRE(tiles < (1LL << 26), "Prompt GEMM: too many tiles.");
  const int splits = workspace ? gemm_splits(tiles, m, k, n, workspace_bytes) : 1;
  // k per split, in whole 64-deep stages
  const int k_chunk = (int)(((k + splits - 1) / splits + kGemmK - 1) / kGemmK * kGemmK);
  const int units = (int)(tiles * ((k + k_chunk - 1) / k_chunk));
  const unsigned blocks = (unsigned)((units + 7) / 8 * 8);
  if (units > (int)tiles) {
    float* partial = static_cast<float*>(workspace);
    hipLaunchKernelGGL((gemm_nt_kernel<float, true>), dim3(blocks), dim3(kGemmThreads), 0, stream,
                       x, w, partial, (int)m, (int)n, (int)k, m_tiles, (int)tiles, k_chunk,
                       (unsigned)xb, (unsigned)wb);
    if (check_launch("gemm_nt_kernel")) return 1;
    const size_t count = (size_t)m * n;
    const unsigned rb = (unsigned)std::min<size_t>((count + 255) / 256, 8192);
    const int used = (int)((k + k_chunk - 1) / k_chunk);
    if (out_dtype == TMC_F32)
      hipLaunchKernelGGL((gemm_reduce_kernel<float>), dim3(rb), dim3(256), 0, stream, partial,
                         static_cast<float*>(y), count, used);
    else
      hipLaunchKernelGGL((gemm_reduce_kernel<half_t>), dim3(rb), dim3(256), 0, stream, partial,
                         static_cast<half_t*>(y), count, used);
    return check_launch("gemm_reduce_kernel");
  }
  if (out_dtype == TMC_F32)
    hipLaunchKernelGGL((gemm_nt_kernel<float, false>), dim3(blocks), dim3(kGemmThreads), 0, stream,
                       x, w, static_cast<float*>(y), (int)m, (int)n, (int)k, m_tiles, (int)tiles,
                       (int)k, (unsigned)xb, (unsigned)wb);
  else
    hipLaunchKernelGGL((gemm_nt_kernel<half_t, false>), dim3(blocks), dim3(kGemmThreads), 0,
                       stream, x, w, static_cast<half_t*>(y), (int)m, (int)n, (int)k, m_tiles,
                       (int)tiles, (int)k, (unsigned)xb, (unsigned)wb);
  return check_launch("gemm_nt_kernel");
}

}  // namespace
}  // namespace tmc

using namespace tmc;

extern "C" int tmc_gemm_mfma_f16(const void* x, const void* weight, void* y, int out_dtype,
                                 int64_t m, int64_t k, int64_t n, void* stream) {
  TMC_REQUIRE(x && weight && y, "Prompt GEMM: null device pointer.");
  TMC_REQUIRE(out_dtype == TMC_F16 || out_dtype == TMC_F32, "Prompt GEMM: output must be f16 or f32.");
  TMC_REQUIRE(m > 0 && k > 0 && n > 0 && m < (1LL << 31) && k < (1LL << 31) && n < (1LL << 31),
              "Prompt GEMM: invalid shape.");
  return launch_gemm_nt(static_cast<const half_t*>(x), static_cast<const half_t*>(weight), y,
                        out_dtype, m, k, n, nullptr, 0, as_stream(stream));
}

extern "C" size_t tmc_gemm_rows_workspace_bytes(void) { return (size_t)32 << 20; }

extern "C" int tmc_gemm_rows_f16(const void* x, const void* weight, void* y, int out_dtype,
                                 int64_t m, int64_t k, int64_t n, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  TMC_REQUIRE(x && weight && y, "Prompt GEMM: null device pointer.");
  TMC_REQUIRE(out_dtype == TMC_F16 || out_dtype == TMC_F32, "Prompt GEMM: output must be f16 or f32.");
  TMC_REQUIRE(m > 0 && k > 0 && n > 0 && m < (1LL << 31) && k < (1LL << 31) && n < (1LL << 31),
              "Prompt GEMM: invalid shape.");
  TMC_REQUIRE(workspace || workspace_bytes == 0, "Prompt GEMM: null workspace with a nonzero size.");
  TMC_REQUIRE(!workspace || aligned16(workspace), "Prompt GEMM: the workspace must be 16-byte aligned.");
  return launch_gemm_nt(static_cast<const half_t*>(x), static_cast<const half_t*>(weight), y,
                        out_dtype, m, k, n, workspace, workspace_bytes, as_stream(stream));
}

